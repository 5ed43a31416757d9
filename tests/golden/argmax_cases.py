"""Known-answer cases of the reference's argmax test, restated as data.

src/weights/dispatch_tests/numerics.rs:14-69
(gpu_argmax_rejects_nonfinite_logits_and_preserves_finite_ordering): bf16 bit
patterns widened exactly to f32 logits, with the expected token index
(0xffffffff for any non-finite logit).
"""
import numpy as np

NONE = 0xFFFFFFFF


def _bf16(x: float) -> int:
    return int(np.float32(x).view(np.uint32) >> 16)


def cases():
    out = []
    for bits in (0x7F80, 0xFF80, 0x7FC1, 0xFFC1, 0x7F81):  # +Inf, -Inf, NaNs at index 2049 of 2051
        a = [_bf16(2.0)] * 2051
        a[2049] = bits
        out.append((a, NONE))
    out += [([0xFF7F], 0), ([0xFF7F, 0x7F7F], 1), ([0x8000, 0, 0x8001], 0), ([0x8001, 0, 1, 2], 3)]
    for tied in ((31, 32), (1023, 1024), (1024, 2048)):
        a = [_bf16(-2.0)] * 2051
        for i in tied:
            a[i] = _bf16(3.0)
        out.append((a, tied[0]))
    return [(np.array(a, np.uint32).astype(np.uint32) << 16, exp) for a, exp in out]


def logits(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint32).view(np.float32)
