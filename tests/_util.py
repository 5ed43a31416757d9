"""Helpers shared by the GPU parity tests (device buffers with guard bands)."""
import sys

import numpy as np

GUARD = 32            # words of sentinel on each side (dispatch_tests.rs:12)
SENTINEL = 0x7FC12345  # dispatch_tests.rs:13


def say(*a):
    """Name the case before each GPU step, flushed, so a crash still shows it."""
    print(*a, flush=True)
    sys.stdout.flush()


class Guarded:
    """A device output with GUARD sentinel words before and after."""

    def __init__(self, oco, nbytes: int):
        self.oco = oco
        self.nbytes = nbytes
        words = (nbytes + 3) // 4
        self.buf = oco.DeviceBuffer((words + 2 * GUARD) * 4)
        self.buf.fill32(SENTINEL)
        self.words = words

    @property
    def ptr(self):
        return self.buf.ptr + GUARD * 4

    def read(self, dtype):
        raw = self.buf.download(np.uint32)
        assert np.all(raw[:GUARD] == SENTINEL), "write before the output"
        tail = raw[GUARD + self.words:]
        assert np.all(tail == SENTINEL), "write past the output"
        body = raw[GUARD:GUARD + self.words].view(np.uint8)[:self.nbytes]
        return body.view(dtype)


def upload_at_offset(oco, data: np.ndarray, offset: int):
    """Weights at an arbitrary byte offset (GGUF tensors need not be aligned)."""
    data = np.ascontiguousarray(data, np.uint8)
    buf = oco.DeviceBuffer(data.nbytes + offset + 64)
    if offset:
        buf.upload(np.full(offset, 0xA5, np.uint8))
    buf.upload(data, offset)
    return buf, buf.ptr + offset


def rel_l2(a, e):
    a = np.asarray(a, np.float64).ravel()
    e = np.asarray(e, np.float64).ravel()
    d = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (d if d else 1.0))


def same_bits_nan_aware(got: np.ndarray, want: np.ndarray):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"NaN mask differs at {np.nonzero(gn != wn)[0][:8]}"
    a = got[~gn].view(np.uint32)
    b = want[~wn].view(np.uint32)
    bad = np.nonzero(a != b)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:8]}: {got[~gn][bad[:4]]} vs {want[~wn][bad[:4]]}"
