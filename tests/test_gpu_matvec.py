"""GPU parity of dequantization and decode matvec against the C oracle.

Bars (from the task's north star):
- dequantized weights bit-exact with the oracle (NaN positions equal);
- matvec outputs within relative L2 1e-5 of the fp64 oracle, and every
  element within the reference's roundoff bound gamma_{2K+8} sum|w x| plus
  bf16 storage rounding (matrix_precision.rs:136-142) where stored bf16.
"""
import numpy as np
import pytest

import oracle as O
import packers as P
from _util import Guarded, rel_l2, same_bits_nan_aware, say, upload_at_offset

pytestmark = pytest.mark.gpu

ALL_FORMATS = [P.F32, P.F16, P.BF16, P.Q4_0, P.Q4_1, P.Q8_0, P.Q4_K, P.Q5_K, P.Q6_K, O.MXFP4]


def gpu_dequant(oco, fmt, data, count, offset=0):
    buf, ptr = upload_at_offset(oco, data, offset)
    out = Guarded(oco, count * 4)
    oco.dequant(fmt, ptr, count, out.ptr)
    oco.synchronize()
    return out.read(np.float32)


@pytest.mark.parametrize("fmt", ALL_FORMATS)
def test_dequant_random_bytes_bit_exact(lib, fmt):
    """Random bytes reach every code, subnormal/Inf/NaN scale and E8M0 0/255."""
    say("dequant random bytes fmt", fmt)
    e, b = O.block_layout(fmt)
    nblocks = 4096 // max(e, 1) * 8 if e > 1 else 4096
    data = np.random.default_rng(fmt).integers(0, 256, nblocks * b, dtype=np.uint8)
    count = nblocks * e
    for offset in (0, 7):
        got = gpu_dequant(lib, fmt, data, count, offset)
        same_bits_nan_aware(got, O.dequant(fmt, data, count))


@pytest.mark.parametrize("fmt", [P.F32, P.F16, P.BF16, P.Q4_0, P.Q4_1, P.Q8_0, P.Q4_K, P.Q5_K, P.Q6_K])
def test_dequant_reference_packer_golden(lib, fmt):
    import os
    say("dequant golden fmt", fmt)
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", f"dense_{fmt}.npz"))
    got = gpu_dequant(lib, fmt, f["bytes"], f["coefficients"].size)
    np.testing.assert_array_equal(got, f["coefficients"].astype(np.float32))


def test_dequant_mxfp4_reference_packer(lib):
    say("dequant mxfp4 packer")
    k, n = 2880, 5
    data, coeffs = P.mxfp4_decode_weights(k, n)
    w = np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:]
    got = gpu_dequant(lib, O.MXFP4, w, coeffs.size, offset=P.WEIGHT_OFFSET)
    np.testing.assert_array_equal(got.astype(np.float64), coeffs)


def test_dequant_synthetic_baseline_tensors(lib):
    from oco_amd import synth
    for fmt, rows, k in [(8, 64, 4096), (39, 64, 2880), (12, 64, 4096), (14, 64, 12288)]:
        say("dequant synth", fmt, rows, k)
        data = synth.weights(fmt, rows, k, seed=11)
        got = gpu_dequant(lib, fmt, data, rows * k)
        same_bits_nan_aware(got, O.dequant(fmt, data, rows * k))


def run_matvec(oco, fmt, data, x, p, x_bf16=False, y_bf16=False, bias=None, ids=None, offset=0):
    wbuf, wptr = upload_at_offset(oco, data, offset)
    xb = oco.DeviceBuffer.from_array(x)
    routed_f32 = p.experts > 1 and not p.route_major
    out_bf16 = y_bf16 and not routed_f32
    y = Guarded(oco, p.m * p.n * (2 if out_bf16 else 4))
    bb = oco.DeviceBuffer.from_array(np.asarray(bias, np.float32)) if bias is not None else None
    ib = oco.DeviceBuffer.from_array(np.asarray(ids, np.uint32)) if ids is not None else None
    oco.matvec(fmt, wptr, xb, y.ptr, p, oco.DType.BF16 if x_bf16 else oco.DType.F32,
               oco.DType.BF16 if y_bf16 else oco.DType.F32, bb, ib)
    oco.synchronize()
    got = y.read(np.uint16 if out_bf16 else np.float32)
    return O.bf16_to_f32(got) if out_bf16 else got, out_bf16


def check_matvec(oco, fmt, data, x, p, **kw):
    got, stored_bf16 = run_matvec(oco, fmt, data, x, p, **kw)
    want, mag = O.matvec_f64(fmt, np.asarray(data, np.uint8), x, p, bias=kw.get("bias"),
                             ids=kw.get("ids"))
    assert np.all(np.isfinite(got))
    err = rel_l2(got, want)
    tol = 1e-5 if not stored_bf16 else 4e-3
    assert err <= tol, f"relL2 {err:.3e} > {tol}"
    bound = O.roundoff_bound(want, mag, p.k, stored_bf16)
    bad = np.nonzero(np.abs(got - want) > bound)[0]
    assert bad.size == 0, f"{bad.size} outputs beyond the roundoff bound, first {bad[:4]}"
    return err


SHAPES = {  # BASELINE shapes (lm_head is covered by its own row-slice test), and the other streamed formats
    P.Q8_0: (4096, 4096), O.MXFP4: (5760, 2880), P.Q4_K: (12288, 4096), P.Q6_K: (4096, 12288),
    P.Q4_0: (4096, 4096), P.Q4_1: (4096, 4096), P.Q5_K: (12288, 4096),
}


@pytest.mark.parametrize("fmt", [P.Q8_0, O.MXFP4, P.Q4_K, P.Q6_K, P.Q4_0, P.Q4_1, P.Q5_K])
def test_matvec_baseline_shapes_f32(lib, fmt):
    from oco_amd import synth
    n, k = SHAPES[fmt]
    say("matvec baseline", fmt, n, k)
    data = synth.weights(fmt, n, k, seed=1)
    x = synth.activations(2, k)
    err = check_matvec(lib, fmt, data, x, O.Matrix(k, n, 1, 0, 1, 1, 0))
    say(f"  relL2 {err:.2e}")


@pytest.mark.parametrize("fmt", ALL_FORMATS)
@pytest.mark.parametrize("n", [1, 33, 257])
def test_matvec_reference_packer_tails(lib, fmt, n):
    """K=512 with SIMD-tail row counts (matrix_precision.rs:19-107), bf16 inputs."""
    k = 512
    say("matvec packer", fmt, n)
    if fmt == O.MXFP4:
        data, _ = P.mxfp4_expert_weights(k, n, 1, 1)
        data = np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:]
    else:
        data, _ = P.dense_weights(fmt, n, k)
        data = np.frombuffer(data, np.uint8)
    x = P.dense_input(2, k)
    p = O.Matrix(k, n, 2, 0, 1, 1, 0)
    check_matvec(lib, fmt, data, x, p, x_bf16=True)
    check_matvec(lib, fmt, data, x, p, x_bf16=True, y_bf16=True)


@pytest.mark.parametrize("fmt", [O.MXFP4, P.Q8_0, P.Q4_K, P.Q6_K, P.Q4_0, P.Q4_1, P.Q5_K])
def test_matvec_routed_semantics(lib, fmt):
    """experts > 1: rows through ids[route], input route/routes, f32 output,
    has_bias 2 adds bf16(bias + 1) (vector.metal:76-78, 140-146)."""
    from oco_amd import synth
    E, n, k = 6, 45, 512
    data = synth.weights(fmt, E * n, k, seed=3)
    ids = np.array([3, 0, 5, 1, 1, 4, 2, 0], np.uint32)
    rng = np.random.default_rng(5)
    bias = rng.normal(size=E * n).astype(np.float32)
    x = synth.activations(4, 2 * k).reshape(2, k)
    for has_bias in (0, 1, 2):
        say("matvec routed", fmt, has_bias)
        p = O.Matrix(k, n, 8, 0, 4, E, has_bias)
        check_matvec(lib, fmt, data, x, p, bias=bias if has_bias else None, ids=ids, y_bf16=True)
    xr = synth.activations(6, 8 * k).reshape(8, k)
    p = O.Matrix(k, n, 8, 1, 4, E, 1)
    check_matvec(lib, fmt, data, xr, p, bias=bias, ids=ids)


def test_matvec_mxfp4_unaligned_and_nan_header(lib):
    """Weights at byte offset 7; E8M0 255 makes its row NaN (mxfp4.rs:205-233)."""
    from oco_amd import synth
    n, k = 33, 2880
    data = synth.weights(O.MXFP4, n, k, seed=9).copy()
    x = synth.activations(10, k)
    p = O.Matrix(k, n, 1, 0, 1, 1, 0)
    say("matvec mxfp4 offset 7")
    check_matvec(lib, O.MXFP4, data, x, p, offset=7)
    data[0] = 255
    got, _ = run_matvec(lib, O.MXFP4, data, x, p, offset=7)
    assert np.isnan(got[0]) and np.all(np.isfinite(got[1:]))


def test_matvec_lm_head_row_slices(lib):
    """lm_head [151936 x 4096] Q6_K with f32 output: the full matrix on the
    GPU, checked against the oracle on its first and last 1024 rows."""
    from oco_amd import synth
    n, k = 151936, 4096
    say("matvec lm_head")
    data = synth.weights(P.Q6_K, n, k, seed=21)
    x = synth.activations(22, k)
    got, _ = run_matvec(lib, P.Q6_K, data, x, O.Matrix(k, n, 1, 0, 1, 1, 0))
    rb = k // 256 * 210
    for lo in (0, n - 1024):
        sl = data[lo * rb:(lo + 1024) * rb]
        want, mag = O.matvec_f64(P.Q6_K, sl, x, O.Matrix(k, 1024, 1, 0, 1, 1, 0))
        assert rel_l2(got[lo:lo + 1024], want) <= 1e-5
        assert np.all(np.abs(got[lo:lo + 1024] - want) <= O.roundoff_bound(want, mag, k, False))


def test_matvec_exact_integer_answers(lib):
    """All-ones weights, x = 1 and 2 -> K and 2K exactly (compute/tests.rs:40-80)."""
    k, n = 4096, 100
    for fmt, block in [(P.F32, None), (P.Q8_0, None)]:
        if fmt == P.F32:
            data = np.ones(n * k, np.float32).view(np.uint8)
        else:
            blk = np.frombuffer((0x3C00).to_bytes(2, "little") + bytes([1] * 32), np.uint8)
            data = np.tile(blk, n * k // 32)
        for xv in (1.0, 2.0):
            say("matvec exact", fmt, xv)
            got, _ = run_matvec(lib, fmt, data, np.full(k, xv, np.float32), O.Matrix(k, n, 1, 0, 1, 1, 0))
            np.testing.assert_array_equal(got, np.full(n, k * xv, np.float32))


STREAM_PLANS = ["1,1,1", "1,1,2", "1,2,2", "1,2,1", "1,4,1", "1,4,3"]


@pytest.mark.parametrize("plan", STREAM_PLANS)
def test_matvec_stream_plans(lib, plan):
    """Every streaming-kernel geometry (rows per half-wavefront, K split,
    workgroups per CU) on ragged row counts, f32 and
    bf16 activations, routed rows with bias."""
    with lib.overridden(lib.Knob.STREAM_PLAN, [int(v) for v in plan.split(",")]):
        _stream_plan_cases(lib, plan)


@pytest.mark.parametrize("direct,xreg", [(1, 0), (1, 1), (0, 1), (0, 0)])
def test_matvec_stream_x_source(lib, direct, xreg):
    """Activations staged through LDS or read straight into registers, with
    and without per-lane direct weight loads, on every streaming format."""
    with lib.overridden(lib.Knob.STREAM_DIRECT, [direct, xreg]):
        _stream_plan_cases(lib, f"direct {direct} xreg {xreg}")


def test_matvec_plain_kernel(lib):
    """The plain (non-streaming) matvec, which quantized formats take when
    the activations are not vector-aligned, forced on every format with the
    MATVEC_PLAIN knob."""
    with lib.overridden(lib.Knob.MATVEC_PLAIN, [1]):
        _stream_plan_cases(lib, "plain")


def _stream_plan_cases(lib, plan):
    from oco_amd import synth
    for fmt, n, k in [(O.MXFP4, 131, 2880), (P.Q8_0, 77, 4096), (P.Q4_K, 257, 2048), (P.Q6_K, 300, 4096),
                      (P.Q4_0, 90, 4096), (P.Q4_1, 65, 2048), (P.Q5_K, 130, 4096)]:
        say("matvec plan", plan, fmt, n, k)
        data = synth.weights(fmt, n, k, seed=11)
        x = synth.activations(12, k)
        check_matvec(lib, fmt, data, x, O.Matrix(k, n, 1, 0, 1, 1, 0))
        check_matvec(lib, fmt, data, synth.bf16_bits(x), O.Matrix(k, n, 1, 0, 1, 1, 0), x_bf16=True, y_bf16=True)
    E, n, k = 5, 45, 1024
    data = synth.weights(P.Q6_K, E * n, k, seed=13)
    ids = np.array([3, 0, 4, 1], np.uint32)
    bias = np.random.default_rng(14).normal(size=E * n).astype(np.float32)
    x = synth.activations(15, 2 * k).reshape(2, k)
    check_matvec(lib, P.Q6_K, data, x, O.Matrix(k, n, 4, 0, 2, E, 2), bias=bias, ids=ids)


def _relu_sqr_cases(lib, tag):
    from oco_amd import synth
    cases = [(fmt, 129, 1024) for fmt in [P.F32, P.F16, P.BF16]] + \
            [(O.MXFP4, 131, 2880), (P.Q8_0, 77, 4096), (P.Q4_K, 257, 2048), (P.Q6_K, 100, 4096),
             (P.Q4_0, 90, 4096), (P.Q4_1, 65, 2048), (P.Q5_K, 130, 4096)]
    for fmt, n, k in cases:
        say("matvec relu_sqr", tag, fmt, n, k)
        if fmt in (P.F32, P.F16, P.BF16):
            wf = np.random.default_rng(21).normal(0, 0.02, n * k).astype(np.float32)
            data = (wf if fmt == P.F32 else wf.astype(np.float16) if fmt == P.F16 else synth.bf16_bits(wf)).view(np.uint8)
        else:
            data = synth.weights(fmt, n, k, seed=21)
        x = synth.activations(22, k)
        x[::7] = np.nan  # NaN inputs read as 0
        p = O.Matrix(k, n, 1, 0, 1, 1, 0)
        xr = O.relu_sqr_input(x)
        # The transform on load equals the plain matvec of the transformed
        # input, bit for bit (same kernel, same f32 values, same order).
        wbuf, wptr = upload_at_offset(lib, data, 0)
        outs = []
        for xin, rs in ((x, True), (xr, False)):
            xb = lib.DeviceBuffer.from_array(xin)
            y = Guarded(lib, n * 4)
            lib.matvec(fmt, wptr, xb, y.ptr, p, lib.DType.F32, lib.DType.F32, relu_sqr=rs)
            lib.synchronize()
            outs.append(y.read(np.float32))
        np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        want, mag = O.matvec_f64(fmt, np.asarray(data, np.uint8), xr, p)
        assert rel_l2(outs[0], want) <= 1e-5
        assert np.all(np.abs(outs[0] - want) <= O.roundoff_bound(want, mag, k, False))
        # bf16 activations, bf16 output: against the fp64 oracle of the
        # transformed (f32) input.
        xb16 = synth.bf16_bits(synth.activations(23, k))
        xb = lib.DeviceBuffer.from_array(xb16)
        y = Guarded(lib, n * 2)
        lib.matvec(fmt, wptr, xb, y.ptr, p, lib.DType.BF16, lib.DType.BF16, relu_sqr=True)
        lib.synchronize()
        got = O.bf16_to_f32(y.read(np.uint16))
        want, mag = O.matvec_f64(fmt, np.asarray(data, np.uint8), O.relu_sqr_input(xb16), p)
        assert rel_l2(got, want) <= 4e-3
        assert np.all(np.abs(got - want) <= O.roundoff_bound(want, mag, k, True))
    # routed rows (the relu² experts' down projection): route-major Q4_0 bank
    E, n, k = 4, 64, 1024
    data = synth.weights(P.Q4_0, E * n, k, seed=24)
    ids = np.array([2, 0, 3], np.uint32)
    x = synth.activations(25, 3 * k)
    p = O.Matrix(k, n, 3, 1, 1, E, 0)
    got, _ = run_matvec(lib, P.Q4_0, data, O.relu_sqr_input(x), p, ids=ids)
    wbuf, wptr = upload_at_offset(lib, data, 0)
    xb, ib = lib.DeviceBuffer.from_array(x), lib.DeviceBuffer.from_array(ids)
    y = Guarded(lib, 3 * n * 4)
    lib.matvec(P.Q4_0, wptr, xb, y.ptr, p, lib.DType.F32, lib.DType.F32, ids=ib, relu_sqr=True)
    lib.synchronize()
    np.testing.assert_array_equal(y.read(np.float32).view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("path", ["default", "xreg", "plain"])
def test_matvec_relu_sqr(lib, path):
    """oco_matvec_relu_sqr (the input_relu_sqr specialisation): staged,
    register-read and plain-kernel activations, every format, f32 and bf16
    activations, routed rows."""
    if path == "default":
        _relu_sqr_cases(lib, path)
    elif path == "xreg":
        with lib.overridden(lib.Knob.STREAM_DIRECT, [0, 1]):
            _relu_sqr_cases(lib, path)
    else:
        with lib.overridden(lib.Knob.MATVEC_PLAIN, [1]):
            _relu_sqr_cases(lib, path)
