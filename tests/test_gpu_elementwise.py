"""GPU parity of the steps either side of the decode matvec.

- argmax_f32 (argmax.metal:1-47): exact index against the oracle and the
  reference's own known answers (numerics.rs:14-69), at lm_head size too.
- norm / add_norm (elementwise.metal:6-58): every bf16 output within one
  bf16 rounding of the fp64 oracle value (two roundings when full_layer is
  off); add_norm's updated residual bit-exact (one rounding of an exact sum).
- matvec_norm: bit-identical to norm followed by matvec on every format,
  fused (streaming formats) or not.
"""
import numpy as np
import pytest

import argmax_cases as A
import oracle as O
from _util import Guarded, say, upload_at_offset

pytestmark = pytest.mark.gpu


def gpu_argmax(oco, x, use_ws=False):
    xb = oco.DeviceBuffer.from_array(np.ascontiguousarray(x, np.float32)) if x.size else None
    out = Guarded(oco, 4)
    if use_ws:
        need = oco.argmax_workspace(x.size)
        ws = oco.DeviceBuffer(max(need, 4))
        oco.argmax(xb, x.size, out.ptr, workspace=ws, workspace_bytes=need)
    else:
        oco.argmax(xb, x.size, out.ptr)
    oco.synchronize()
    return int(out.read(np.uint32)[0])


def test_argmax_reference_cases(lib):
    for bits, want in A.cases():
        say("argmax case", len(bits), want)
        assert gpu_argmax(lib, A.logits(bits)) == want
    assert gpu_argmax(lib, np.zeros(0, np.float32)) == A.NONE


@pytest.mark.parametrize("n", [1, 777, 4096, 151936, 262144])
def test_argmax_random(lib, n):
    rng = np.random.default_rng(n)
    x = rng.normal(size=n).astype(np.float32)
    say("argmax random", n)
    assert gpu_argmax(lib, x) == O.argmax_f32(x) == int(np.argmax(x))
    assert gpu_argmax(lib, x, use_ws=True) == O.argmax_f32(x)
    t = np.round(x).astype(np.float32)  # ties everywhere: lowest index wins
    assert gpu_argmax(lib, t) == O.argmax_f32(t)
    neg = -np.abs(x) - 1
    assert gpu_argmax(lib, neg) == O.argmax_f32(neg)
    for bad in (np.inf, -np.inf, np.nan):
        y = x.copy()
        y[rng.integers(n)] = bad
        assert gpu_argmax(lib, y) == A.NONE


def _rows(seed, rows, n, scale=1.0):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16((rng.normal(size=(rows, n)) * scale).astype(np.float32)).reshape(rows, n)
    w = (1.0 + 0.5 * rng.normal(size=n)).astype(np.float32)
    return x, w


def _within_rounding(got_bits, exact, roundings):
    got = O.bf16_to_f32(got_bits).astype(np.float64).reshape(exact.shape)
    err = np.abs(got - exact)
    assert np.all(err <= roundings * 2.0 ** -8 * np.abs(exact) * 1.01 + 1e-35), f"max rel {np.max(err / (np.abs(exact) + 1e-30)):.3g}"


@pytest.mark.parametrize("n", [64, 2880, 4096, 12288])
@pytest.mark.parametrize("full", [True, False])
def test_norm_against_oracle(lib, n, full):
    rows = 3
    x, w = _rows(n, rows, n, scale=3.0)
    say("norm", n, full)
    y = Guarded(lib, rows * n * 2)
    lib.norm(lib.DeviceBuffer.from_array(x), lib.DeviceBuffer.from_array(w), y.ptr, rows, n, 1e-6, full)
    lib.synchronize()
    got = y.read(np.uint16)
    want, exact = O.norm(x, w, 1e-6, full)
    _within_rounding(got, exact, 1 if full else 3)
    assert np.mean(got == want.ravel()) > 0.99


@pytest.mark.parametrize("full", [True, False])
def test_add_norm_against_oracle(lib, full):
    rows, n = 4, 4096
    x, w = _rows(7, rows, n)
    y, _ = _rows(8, rows, n)
    say("add_norm", full)
    xb = lib.DeviceBuffer.from_array(x)
    out = Guarded(lib, rows * n * 2)
    lib.add_norm(xb, lib.DeviceBuffer.from_array(y), lib.DeviceBuffer.from_array(w), out.ptr, rows, n, 1e-6, full)
    lib.synchronize()
    want_x, want_out, exact = O.add_norm(x, y, w, 1e-6, full)
    assert np.array_equal(xb.download(np.uint16).reshape(rows, n), want_x)
    _within_rounding(out.read(np.uint16), exact, 1 if full else 3)
    # add_norm == add then norm on the device as well
    y2 = Guarded(lib, rows * n * 2)
    lib.norm(xb, lib.DeviceBuffer.from_array(w), y2.ptr, rows, n, 1e-6, full)
    lib.synchronize()
    assert np.array_equal(y2.read(np.uint16), out.read(np.uint16))


FUSED_CASES = [(8, 300, 4096), (12, 257, 4096), (14, 130, 12288), (39, 201, 2880), (12, 64, 2048),
               (2, 70, 512), (1, 33, 512), (3, 45, 1024)]


@pytest.mark.parametrize("fmt,n,k", FUSED_CASES)
def test_matvec_norm_equals_norm_then_matvec(lib, fmt, n, k):
    from oco_amd import synth
    import packers as P
    say("matvec_norm", fmt, n, k)
    if fmt in (8, 12, 14, 39):
        data = synth.weights(fmt, n, k, seed=fmt + n)
    else:  # formats without a synthetic generator: the reference's packers
        data = np.frombuffer(P.dense_weights(fmt, n, k)[0], np.uint8)
    x, w = _rows(k + n, 1, k, scale=2.0)
    bias = np.random.default_rng(n).normal(size=n).astype(np.float32)
    wb, xb, nb = (lib.DeviceBuffer.from_array(a) for a in (data, x, w))
    bb = lib.DeviceBuffer.from_array(bias)
    for full in (True, False):
        for y_dt, has_bias in ((lib.DType.F32, 0), (lib.DType.BF16, 1)):
            p = lib.Matrix(k, n, 1, 0, 1, 1, has_bias)
            normed = lib.DeviceBuffer(k * 2)
            lib.norm(xb, nb, normed, 1, k, 1e-5, full)
            y1 = Guarded(lib, n * (2 if y_dt == lib.DType.BF16 else 4))
            lib.matvec(fmt, wb, normed, y1.ptr, p, lib.DType.BF16, y_dt, bb if has_bias else None)
            y2 = Guarded(lib, n * (2 if y_dt == lib.DType.BF16 else 4))
            lib.matvec_norm(fmt, wb, xb, nb, 1e-5, y2.ptr, p, full, y_dt, bb if has_bias else None)
            lib.synchronize()
            assert np.array_equal(y1.read(np.uint8), y2.read(np.uint8)), (full, y_dt)
    # against the fp64 oracle of norm -> matvec
    normed_ref, _ = O.norm(x, w, 1e-5, True)
    want, _ = O.matvec_f64(fmt, data, normed_ref.reshape(-1), O.Matrix(k, n, 1, 0, 1, 1, 0))
    y3 = Guarded(lib, n * 4)
    lib.matvec_norm(fmt, wb, xb, nb, 1e-5, y3.ptr, lib.Matrix(k, n, 1, 0, 1, 1, 0), True)
    lib.synchronize()
    got = y3.read(np.float32)
    assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want)  # the input itself differs by one bf16 rounding


@pytest.mark.parametrize("plan", [(1, 2, 2), (1, 4, 2), (1, 1, 3)])
def test_matvec_norm_stream_plans(lib, plan):
    """Fused staging under K splits (the LDS area the norm reduction shares),
    forced through the stream-plan knob."""
    with lib.overridden(lib.Knob.STREAM_PLAN, plan):
        _matvec_norm_stream_plan_case(lib)


def _matvec_norm_stream_plan_case(lib):
    from oco_amd import synth
    fmt, n, k = 14, 100, 8192
    data = synth.weights(fmt, n, k, seed=3)
    x, w = _rows(9, 1, k)
    wb, xb, nb = (lib.DeviceBuffer.from_array(a) for a in (data, x, w))
    p = lib.Matrix(k, n, 1, 0, 1, 1, 0)
    normed = lib.DeviceBuffer(k * 2)
    lib.norm(xb, nb, normed, 1, k, 1e-5, True)
    y1, y2 = Guarded(lib, n * 4), Guarded(lib, n * 4)
    lib.matvec(fmt, wb, normed, y1.ptr, p, lib.DType.BF16)
    lib.matvec_norm(fmt, wb, xb, nb, 1e-5, y2.ptr, p, True)
    lib.synchronize()
    assert np.array_equal(y1.read(np.uint32), y2.read(np.uint32))


def test_matvec_norm_routed_rows(lib):
    """Routed rows: each route normalises its own input row (route / routes)."""
    from oco_amd import synth
    E, n, k = 4, 40, 1024
    data = synth.weights(12, E * n, k, seed=5)
    x, w = _rows(11, 2, k)
    ids = np.array([3, 0, 1, 3], np.uint32)
    wb, xb, nb, ib = (lib.DeviceBuffer.from_array(a) for a in (data, x, w, ids))
    p = lib.Matrix(k, n, 4, 0, 2, E, 0)
    normed = lib.DeviceBuffer(2 * k * 2)
    lib.norm(xb, nb, normed, 2, k, 1e-5, False)
    y1, y2 = Guarded(lib, 4 * n * 4), Guarded(lib, 4 * n * 4)
    lib.matvec(12, wb, normed, y1.ptr, p, lib.DType.BF16, lib.DType.F32, None, ib)
    lib.matvec_norm(12, wb, xb, nb, 1e-5, y2.ptr, p, False, lib.DType.F32, None, ib)
    lib.synchronize()
    assert np.array_equal(y1.read(np.uint32), y2.read(np.uint32))


@pytest.mark.parametrize("words", [4, 4096, 2203200, 2203204])
def test_buffer_xor32(lib, words):
    """oco_buffer_xor32 (the read-floor stream) equals numpy's XOR over the
    words, accumulating into the caller's word; partial rounds and tails."""
    rng = np.random.default_rng(words)
    data = rng.integers(0, 2 ** 32, size=words, dtype=np.uint64).astype(np.uint32)
    buf = lib.DeviceBuffer.from_array(data)
    # stale slots hold garbage before the call: every slot is written
    out = lib.DeviceBuffer.from_array(rng.integers(0, 2 ** 32, size=1024, dtype=np.uint64).astype(np.uint32))
    buf.xor32(out)
    lib.synchronize()
    assert np.bitwise_xor.reduce(out.download(np.uint32)) == np.bitwise_xor.reduce(data)


GROUP_CASES = [(12, 2, 300, 4096, 0), (12, 2, 12288, 4096, 0), (12, 3, 257, 2048, 7), (14, 2, 130, 12288, 0),
               (8, 4, 100, 4096, 0), (39, 2, 201, 2880, 3), (2, 2, 70, 512, 0), (13, 2, 96, 1024, 0),
               (1, 2, 33, 512, 0)]


@pytest.mark.parametrize("fmt,count,n,k,offset", GROUP_CASES)
def test_matvec_group_equals_separate_calls(lib, fmt, count, n, k, offset):
    """oco_matvec_group (the up/gate pair in one grid) equals one
    oco_matvec_norm / oco_matvec call per matrix bit for bit: with and
    without the fused norm (both rounding modes), bias, bf16 and f32
    outputs, two input rows, 2-4 matrices, weights 16-byte aligned (the
    direct Q4_K loads) or at a byte offset (the LDS tile), and formats
    without a streaming kernel (one call per matrix)."""
    from oco_amd import synth
    import packers as P
    say("matvec_group", fmt, count, n, k, offset)
    mats = []
    for i in range(count):
        if fmt in (8, 12, 14, 39):
            data = synth.weights(fmt, n, k, seed=fmt + n + 31 * i)
        else:
            data = np.frombuffer(P.dense_weights(fmt, n, k)[0], np.uint8)[::-1].copy() if i else \
                np.frombuffer(P.dense_weights(fmt, n, k)[0], np.uint8)
        mats.append(upload_at_offset(lib, data, offset))
    wptrs = [ptr for _, ptr in mats]
    rows = 2
    x, w = _rows(k + 3 * n, rows, k, scale=2.0)
    xb, nb = lib.DeviceBuffer.from_array(x), lib.DeviceBuffer.from_array(w)
    xf = lib.DeviceBuffer.from_array(O.bf16_to_f32(x).astype(np.float32))
    biases = [lib.DeviceBuffer.from_array(np.random.default_rng(i).normal(size=n).astype(np.float32))
              for i in range(count)]
    for norm, full, y_dt, has_bias, x_dt in [(True, True, lib.DType.F32, 0, lib.DType.BF16),
                                              (True, False, lib.DType.BF16, 1, lib.DType.BF16),
                                              (False, True, lib.DType.F32, 1, lib.DType.F32),
                                              (False, True, lib.DType.BF16, 0, lib.DType.BF16)]:
        p = lib.Matrix(k, n, rows, 0, 1, 1, has_bias)
        esz = 2 if y_dt == lib.DType.BF16 else 4
        xin = xb if x_dt == lib.DType.BF16 else xf
        sep = [Guarded(lib, rows * n * esz) for _ in range(count)]
        grp = [Guarded(lib, rows * n * esz) for _ in range(count)]
        for i in range(count):
            b = biases[i] if has_bias else None
            if norm:
                lib.matvec_norm(fmt, wptrs[i], xb, nb, 1e-5, sep[i].ptr, p, full, y_dt, b)
            else:
                lib.matvec(fmt, wptrs[i], xin, sep[i].ptr, p, x_dt, y_dt, b)
        lib.matvec_group(fmt, wptrs, xin, [g.ptr for g in grp], p, x_dt, y_dt, nb if norm else None, 1e-5, full,
                         biases if has_bias else None)
        lib.synchronize()
        for i in range(count):
            assert np.array_equal(sep[i].read(np.uint8), grp[i].read(np.uint8)), (i, norm, full, y_dt)
