"""GPU parity of the MFMA prefill matmul against the fp64 oracle.

Bars: relative L2 2e-3 of the fp64 product of the exact coefficients, the
bound for MFMA prefill on bf16 activations, for every format.  K-quant and
Q8_0 weights run f16-operand MFMA, each element within the reference's
roundoff bound of the half-operand product (matrix_precision.rs:119-142).
MXFP4 runs the block-scaled FP6 x FP4 MFMA on the weights as stored, with
each activation block split into two E2M3 terms: each element is within the
fp32 roundoff bound plus mx_split_bound, the split's worst case.
"""
import numpy as np
import pytest

import oracle as O
import packers as P
from _util import Guarded, rel_l2, say

pytestmark = pytest.mark.gpu


MX_BAR = 2e-3


def mx_split_bound(x_bits, w, n, k):
    """Worst-case error of the two-term E2M3 split of each 32-block of
    activations, carried through |W|: per value at most 1/225 of its block's
    max |x| (term 1 leaves |r| <= s1/4 < max/15, term 2 rounds r under
    s2 < 2 max|r| / 7.5 to within s2/4), bounded here by 2^-7 of the block
    maximum, plus as much again for the MFMA's in-block fixed-point sum."""
    X = O.bf16_to_f32(x_bits).astype(np.float64)
    W = np.abs(O.dequant(39, w, n * k).astype(np.float64)).reshape(n, k)
    m = X.shape[0]
    amax = np.abs(X).reshape(m, k // 32, 32).max(-1)
    wsum = W.reshape(n, k // 32, 32).sum(-1)
    return 2.0 ** -6 * (amax @ wsum.T)


def vector_rows(fmt, k, n):
    """Builder::dense's vector_rows (pipelines.rs:271-283): oco_matmul runs the
    matvec (exact weights, fp32) up to this many bf16 rows."""
    if fmt in (P.Q4_0, P.Q4_1):
        return 4
    if fmt == P.Q5_K:
        return 4 if (k, n) == (6144, 5120) else 1
    if fmt == P.Q8_0:
        return 128 if (k, n) == (2880, 512) else 4 if (k, n) in ((2880, 4096), (4096, 2880)) else 1
    if fmt == 0:
        return 1 << 30 if n <= 128 else 1
    return 1


def run(oco, fmt, w, x, m, n, k, y_bf16=False, bias=None):
    wb = oco.DeviceBuffer.from_array(w)
    xb = oco.DeviceBuffer.from_array(x)
    y = Guarded(oco, m * n * (2 if y_bf16 else 4))
    bb = oco.DeviceBuffer.from_array(bias) if bias is not None else None
    p = oco.Matrix(k, n, m, 0, 1, 1, 1 if bias is not None else 0)
    oco.matmul(fmt, wb, xb, y.ptr, p, oco.DType.BF16, oco.DType.BF16 if y_bf16 else oco.DType.F32, bb)
    oco.synchronize()
    got = y.read(np.uint16 if y_bf16 else np.float32)
    return (O.bf16_to_f32(got) if y_bf16 else got).reshape(m, n)


@pytest.mark.parametrize("fmt", [P.Q8_0, P.Q4_K, P.Q6_K, P.Q5_K, P.Q4_0, P.Q4_1, 39])
@pytest.mark.parametrize("m", [1, 9, 21, 64, 130])
def test_matmul_reference_packer(lib, fmt, m):
    """K=512, N=33 packer weights (matrix_precision.rs:19-107), bf16 inputs."""
    k, n = 512, 33
    say("matmul packer", fmt, m)
    if fmt == 39:
        data, _ = P.mxfp4_expert_weights(k, n, 2, 1)
        w = np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:]
    else:
        data, _ = P.dense_weights(fmt, n, k)
        w = np.frombuffer(data, np.uint8)
    x = P.dense_input(m, k)
    got = run(lib, fmt, w, x, m, n, k)
    exact, emag = O.matmul_reference(fmt, w, x, n, k, half_operands=False)
    if m <= vector_rows(fmt, k, n):  # the matvec: north_star's fp32 bar
        assert rel_l2(got, exact) <= 1e-5
        assert np.all(np.abs(got - exact) <= O.roundoff_bound(exact, emag, k, False))
        return
    half, mag = O.matmul_reference(fmt, w, x, n, k, half_operands=(fmt != 39))
    assert rel_l2(got, exact) <= (MX_BAR if fmt == 39 else 2e-3)
    extra = mx_split_bound(x, w, n, k) if fmt == 39 else 0.0
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, False) + extra)


@pytest.mark.parametrize("fmt,n,k", [(39, 5760, 2880), (12, 768, 2048), (8, 512, 4096), (14, 1024, 4096)])
def test_matmul_prefill_shapes(lib, fmt, n, k):
    """BASELINE cfg 5a (MXFP4 5760x2880 x 512 bf16 tokens) and K-quant shapes."""
    from oco_amd import synth
    m = 512
    say("matmul prefill", fmt, n, k)
    w = synth.weights(fmt, n, k, seed=3)
    x = synth.bf16_bits(synth.activations(4, m * k)).reshape(m, k)
    got = run(lib, fmt, w, x, m, n, k)
    exact, mag = O.matmul_reference(fmt, w, x, n, k, half_operands=False)
    assert rel_l2(got, exact) <= (MX_BAR if fmt == 39 else 2e-3)
    if fmt == 39:
        say("  relL2", rel_l2(got, exact))
        assert np.all(np.abs(got - exact) <= O.roundoff_bound(exact, mag, k, False) + mx_split_bound(x, w, n, k))


@pytest.mark.parametrize("fmt,n,k", [(12, 12288, 4096), (14, 4096, 12288), (8, 4096, 4096)])
def test_matmul_dense_prefill_bench_shapes(lib, fmt, n, k):
    """The dense prefill bench configurations as the bench runs them (its
    weight and activation seeds, 512 bf16 tokens, bf16 output, the vendor
    path): every 32nd row against the fp64 oracle, within 2e-3 and the
    per-element half-operand bound with the output rounding."""
    from oco_amd import synth
    m = 512
    say("matmul dense prefill bench shape", fmt, n, k)
    w = synth.weights(fmt, n, k, 7)
    x = synth.bf16_bits(synth.activations(8, m * k)).reshape(m, k)
    assert lib.matmul_workspace(fmt, lib.Matrix(k, n, m, 0, 1, 1, 0)) > 0  # the vendor path
    got = _run_dense(lib, fmt, w, x, m, n, k, y_bf16=True)[::32]
    exact, _ = O.matmul_reference(fmt, w, x[::32], n, k, half_operands=False)
    half, mag = O.matmul_reference(fmt, w, x[::32], n, k, half_operands=True)
    assert rel_l2(got, exact) <= 2e-3
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, True))


def test_matmul_bias_and_bf16_output(lib):
    from oco_amd import synth
    m, n, k = 70, 100, 256
    w = synth.weights(12, n, k, seed=8)
    x = synth.bf16_bits(synth.activations(9, m * k)).reshape(m, k)
    bias = np.random.default_rng(1).normal(size=n).astype(np.float32)
    got = run(lib, 12, w, x, m, n, k, y_bf16=True, bias=bias)
    exact, _ = O.matmul_reference(12, w, x, n, k, half_operands=False)
    want = exact + O.bf16_round(bias)
    assert rel_l2(got, want) <= 5e-3


def _mx_case(m, n, k, seed, scale_rows=None):
    from oco_amd import synth
    w = synth.weights(39, n, k, seed=seed)
    x = synth.activations(seed + 1, m * k).reshape(m, k)
    if scale_rows is not None:
        x = x * scale_rows
    return w, synth.bf16_bits(x.astype(np.float32)).reshape(m, k)


@pytest.mark.parametrize("m,n,k", [(45, 70, 160), (2, 33, 32), (33, 65, 96), (130, 200, 2880)])
def test_matmul_mxfp4_workspace_tail(lib, m, n, k):
    """Block-scaled MFMA path through oco_matmul_ws: K steps of 64 with a
    lone last block (k % 64 == 32), row/column tails, bias, bf16 output."""
    say("matmul mxfp4 ws", m, n, k)
    w, x = _mx_case(m, n, k, 21)
    p = lib.Matrix(k, n, m, 0, 1, 1, 1)
    need = lib.matmul_workspace(39, p)
    assert need > 0
    ws = lib.DeviceBuffer(need)
    bias = np.random.default_rng(5).normal(size=n).astype(np.float32)
    y = Guarded(lib, m * n * 2)
    lib.matmul(39, lib.DeviceBuffer.from_array(w), lib.DeviceBuffer.from_array(x), y.ptr, p,
               lib.DType.BF16, lib.DType.BF16, lib.DeviceBuffer.from_array(bias), workspace=ws,
               workspace_bytes=need)
    lib.synchronize()
    got = O.bf16_to_f32(y.read(np.uint16)).reshape(m, n)
    exact, mag = O.matmul_reference(39, w, x, n, k, half_operands=False)
    b = O.bf16_round(bias)
    want = exact + b
    # bf16 output: fp32 roundoff of the sum plus one bf16 rounding
    assert np.all(np.abs(got - want) <= O.roundoff_bound(want, mag + np.abs(b), k, True) + mx_split_bound(x, w, n, k))


def test_matmul_mxfp4_workspace_too_small(lib):
    m, n, k = 40, 32, 64
    w, x = _mx_case(m, n, k, 2)
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    need = lib.matmul_workspace(39, p)
    ws = lib.DeviceBuffer(need)
    with pytest.raises(RuntimeError, match="workspace"):
        lib.matmul(39, lib.DeviceBuffer.from_array(w), lib.DeviceBuffer.from_array(x),
                   lib.DeviceBuffer(m * n * 4), p, workspace=ws, workspace_bytes=need - 1)


def test_matmul_mxfp4_wide_dynamic_range(lib):
    """Activations spanning 2^-30 .. 2^30 inside each 32-block: the small
    values of a block fall below its E2M3 terms' resolution, so each output
    may lose the split bound of every block; the block-scaled MFMA also sums
    one block's products in a fixed-point adder about 13 bits deep
    (measured: 448 + 2^-5 kept, 448 + 0.0293 dropped), up to 32 * 2^-13 of
    every block's largest |x w| per term (2^-7 here)."""
    m, n, k = 64, 96, 1024
    rng = np.random.default_rng(7)
    mag = 2.0 ** rng.integers(-30, 31, size=(m, k))
    w, x = _mx_case(m, n, k, 31, scale_rows=mag)
    got = run(lib, 39, w, x, m, n, k)
    exact, mag_ = O.matmul_reference(39, w, x, n, k, half_operands=False)
    X = O.bf16_to_f32(x).astype(np.float64)
    W = O.dequant(39, w, n * k).astype(np.float64).reshape(n, k)
    block_max = np.abs(X[:, None, :] * W[None, :, :]).reshape(m, n, k // 32, 32).max(-1).sum(-1)
    say("  relL2", rel_l2(got, exact))
    assert rel_l2(got, exact) <= MX_BAR
    assert np.all(np.abs(got - exact) <= O.roundoff_bound(exact, mag_, k, False) + 2.0 ** -7 * block_max
                  + mx_split_bound(x, w, n, k))


def test_matmul_mxfp4_nan_scale_and_nan_activation(lib):
    """E8M0 255 makes its weight row's outputs NaN; a NaN activation makes its
    row NaN; everything else stays finite and exact."""
    m, n, k = 40, 48, 256
    w, x = _mx_case(m, n, k, 41)
    w = w.copy()
    row_bytes = k // 32 * 17
    w[5 * row_bytes + 2 * 17] = 255          # weight row 5, block 2
    x = x.copy()
    x[7, 100] = 0x7FC0                        # activation row 7: NaN
    got = run(lib, 39, w, x, m, n, k)
    assert np.all(np.isnan(got[:, 5])) and np.all(np.isnan(got[7, :]))
    keep_r = np.array([r for r in range(m) if r != 7])
    keep_c = np.array([c for c in range(n) if c != 5])
    w_ok = w.copy()
    w_ok[5 * row_bytes + 2 * 17] = 127
    x_ok = x.copy()
    x_ok[7, 100] = 0
    exact, _ = O.matmul_reference(39, w_ok, x_ok, n, k, half_operands=False)
    sub = got[np.ix_(keep_r, keep_c)]
    assert np.all(np.isfinite(sub)) and rel_l2(sub, exact[np.ix_(keep_r, keep_c)]) <= MX_BAR


@pytest.mark.parametrize("m,n,k", [(45, 70, 160), (130, 200, 2880), (257, 400, 576), (512, 193, 1056),
                                   (64, 96, 1024), (33, 100, 4128)])
def test_matmul_mxfp4_tails(lib, m, n, k):
    """Tails: lone last block (k % 64 == 32), odd and even K-step counts,
    a partial last stage of eight steps and whole stages only, row and
    column tails; reruns are bit-identical."""
    say("matmul mxfp4 tails", m, n, k)
    w, x = _mx_case(m, n, k, 51)
    exact, mag = O.matmul_reference(39, w, x, n, k, half_operands=False)
    first = run(lib, 39, w, x, m, n, k)
    assert rel_l2(first, exact) <= MX_BAR
    assert np.all(np.abs(first - exact) <= O.roundoff_bound(exact, mag, k, False) + mx_split_bound(x, w, n, k))
    for _ in range(2):
        again = run(lib, 39, w, x, m, n, k)
        assert np.array_equal(again.view(np.uint32), first.view(np.uint32))


# Formats with f16 operands: at 64 activation rows and more (n % 4 == 0)
# they take the dequantize pass and the vendor GEMM unless the knob says
# otherwise.  Both paths run the same operand bits, so both meet the
# half-operand roundoff bound per element.
VENDOR_FORMATS = [P.Q8_0, P.Q4_K, P.Q6_K, P.Q5_K, P.Q4_0, P.Q4_1, 1, 0]


def _dense_weights(fmt, n, k, seed):
    if fmt in (0, 1):  # F32 / F16 weights as stored
        v = np.random.default_rng(seed).normal(0, 0.05, n * k)
        return np.frombuffer(v.astype(np.float16 if fmt == 1 else np.float32).tobytes(), np.uint8)
    from oco_amd import synth
    return synth.weights(fmt, n, k, seed=seed)


def _run_dense(oco, fmt, w, x, m, n, k, x_f16=False, y_bf16=False, bias=None):
    wb = oco.DeviceBuffer.from_array(w)
    xb = oco.DeviceBuffer.from_array(x)
    y = Guarded(oco, m * n * (2 if y_bf16 else 4))
    bb = oco.DeviceBuffer.from_array(bias) if bias is not None else None
    p = oco.Matrix(k, n, m, 0, 1, 1, 1 if bias is not None else 0)
    oco.matmul(fmt, wb, xb, y.ptr, p, oco.DType.F16 if x_f16 else oco.DType.BF16,
               oco.DType.BF16 if y_bf16 else oco.DType.F32, bb)
    oco.synchronize()
    got = y.read(np.uint16 if y_bf16 else np.float32)
    return (O.bf16_to_f32(got) if y_bf16 else got).reshape(m, n)


@pytest.mark.parametrize("fmt", VENDOR_FORMATS)
@pytest.mark.parametrize("m,n", [(64, 256), (200, 132)])
@pytest.mark.parametrize("vendor", [0, 1])
def test_matmul_vendor_and_fused(lib, fmt, m, n, vendor):
    """Both f16-operand paths against the fp64 oracle; 32-block formats at
    k = 1184 (a partial last 128-wide step), K-quants at k = 1280."""
    from oco_amd import synth
    k = 1280 if fmt in (P.Q4_K, P.Q6_K, P.Q5_K) else 1184
    say("matmul vendor/fused", fmt, m, n, k, vendor)
    w = _dense_weights(fmt, n, k, 21)
    x = synth.bf16_bits(synth.activations(22, m * k)).reshape(m, k)
    with lib.overridden(lib.Knob.MATMUL_VENDOR, [vendor]):
        got = _run_dense(lib, fmt, w, x, m, n, k)
    exact, _ = O.matmul_reference(fmt, w, x, n, k, half_operands=False)
    half, mag = O.matmul_reference(fmt, w, x, n, k, half_operands=True)
    assert rel_l2(got, exact) <= 2e-3
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, False))


@pytest.mark.parametrize("vendor", [0, 1])
def test_matmul_f16_input_bias_bf16_output(lib, vendor):
    """f16 activations (no conversion pass), bias and bf16 output through
    the epilogue; reruns bit-identical."""
    from oco_amd import synth
    m, n, k = 96, 260, 768
    w = synth.weights(P.Q4_K, n, k, seed=31)
    x = (synth.activations(32, m * k).reshape(m, k)).astype(np.float16)
    bias = np.random.default_rng(33).normal(size=n).astype(np.float32)
    with lib.overridden(lib.Knob.MATMUL_VENDOR, [vendor]):
        got = _run_dense(lib, P.Q4_K, w, x, m, n, k, x_f16=True, y_bf16=True, bias=bias)
        again = _run_dense(lib, P.Q4_K, w, x, m, n, k, x_f16=True, y_bf16=True, bias=bias)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    half, mag = O.matmul_reference(P.Q4_K, w, x, n, k, half_operands=True)
    want = half + O.bf16_round(bias)
    assert np.all(np.abs(got - want) <= O.roundoff_bound(want, mag + np.abs(O.bf16_round(bias)), k, True))


def test_matmul_vendor_workspace(lib):
    """The vendor path's workspace: the f16 weights, the f16 activations and
    the fp32 product; too small a workspace is refused."""
    from oco_amd import synth
    m, n, k = 128, 512, 1024
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    need = lib.matmul_workspace(P.Q4_K, p)
    assert need >= n * k * 2 + m * k * 2 + m * n * 4
    assert lib.matmul_workspace(P.Q4_K, p, lib.DType.F16) == need - m * k * 2
    w = lib.DeviceBuffer.from_array(synth.weights(P.Q4_K, n, k, seed=5))
    x = lib.DeviceBuffer.from_array(synth.bf16_bits(synth.activations(6, m * k)))
    y = lib.DeviceBuffer(m * n * 4)
    ws = lib.DeviceBuffer(need)
    with pytest.raises(RuntimeError):
        lib.matmul(P.Q4_K, w, x, y, p, workspace=ws, workspace_bytes=need - 256)
    lib.matmul(P.Q4_K, w, x, y, p, workspace=ws, workspace_bytes=need)
    lib.synchronize()


def test_matmul_vendor_in_graph(lib):
    """A shape first seen inside stream capture (its GEMM plan is made
    there), replayed three times with eager work between: every replay
    equals the eager result bit for bit."""
    from oco_amd import synth
    m, n, k = 72, 388, 640
    fmt = P.Q8_0
    w = lib.DeviceBuffer.from_array(synth.weights(fmt, n, k, seed=41))
    x = lib.DeviceBuffer.from_array(synth.bf16_bits(synth.activations(42, m * k)))
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    y = lib.DeviceBuffer(m * n * 2)
    s = lib.Stream()
    g = lib.Graph(s, lambda: lib.matmul(fmt, w, x, y, p, y_dtype=lib.DType.BF16, stream=s))
    s.sync()
    eager = lib.DeviceBuffer(m * n * 2)
    lib.matmul(fmt, w, x, eager, p, y_dtype=lib.DType.BF16)
    lib.synchronize()
    want = eager.download(np.uint16, m * n)
    for _ in range(3):
        y.fill32(0)
        lib.synchronize()
        g.launch()
        s.sync()
        assert np.array_equal(y.download(np.uint16, m * n), want)
        lib.matmul(fmt, w, x, eager, p, y_dtype=lib.DType.BF16)  # eager work between replays
        lib.synchronize()


def test_matmul_f16_input_unaligned(lib):
    """f16 activations at a 2-byte offset: the GEMM reads them as given, so
    such a call takes the fused tiles, with the same bar."""
    from oco_amd import synth
    m, n, k = 64, 128, 512
    w = lib.DeviceBuffer.from_array(synth.weights(P.Q8_0, n, k, seed=61))
    x16 = synth.activations(62, m * k).astype(np.float16)
    xb = lib.DeviceBuffer(m * k * 2 + 16)
    xb.upload(x16, 2)
    y = lib.DeviceBuffer(m * n * 4)
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    lib.matmul(P.Q8_0, w, xb.ptr + 2, y, p, x_dtype=lib.DType.F16)
    lib.synchronize()
    got = y.download(np.float32, m * n).reshape(m, n)
    wn = synth.weights(P.Q8_0, n, k, seed=61)
    half, mag = O.matmul_reference(P.Q8_0, wn, x16.reshape(m, k), n, k, half_operands=True)
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, False))


@pytest.mark.parametrize("m,k,full,offset", [(2, 2880, 1, 0), (45, 160, 0, 0), (130, 2880, 1, 2), (512, 2880, 0, 0),
                                             (33, 4128, 1, 0)])
def test_norm_mx_split_equals_norm_then_matmul(lib, m, k, full, offset):
    """The fused norm + split, then the MXFP4 prefill from the split: the
    normalised rows and the product bit-identical to oco_norm then
    oco_matmul (k % 64 == 32 and a partial last stage included; x at a
    2-byte offset once; without the bf16 rows once)."""
    from oco_amd import synth
    n, eps = 200, 1e-5
    say("norm mx split", m, k, full, offset)
    rng = np.random.default_rng(m + k)
    w = lib.DeviceBuffer.from_array(synth.weights(39, n, k, seed=71))
    xs = synth.bf16_bits((synth.activations(72, m * k) * 3.0).astype(np.float32))
    xb = lib.DeviceBuffer(m * k * 2 + 16)
    xb.upload(xs, offset)
    nw = lib.DeviceBuffer.from_array(rng.normal(1.0, 0.2, k).astype(np.float32))
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    xn = lib.DeviceBuffer(m * k * 2)
    y1 = lib.DeviceBuffer(m * n * 2)
    lib.norm(xb.ptr + offset, nw, xn, m, k, eps, bool(full))
    lib.matmul(39, w, xn, y1, p, y_dtype=lib.DType.BF16)
    need = lib.matmul_workspace(39, p)
    split = lib.DeviceBuffer(need)
    split.fill32(0xdeadbeef)  # the fused kernel writes every byte the product reads
    yn = lib.DeviceBuffer(m * k * 2)
    y2 = lib.DeviceBuffer(m * n * 2)
    lib.norm_mx_split(xb.ptr + offset, nw, yn if m != 2 else None, m, k, eps, bool(full), split, need)
    lib.matmul_mx_split(w, split, need, y2, p, y_dtype=lib.DType.BF16)
    lib.synchronize()
    if m != 2:
        assert np.array_equal(yn.download(np.uint16, m * k), xn.download(np.uint16, m * k))
    assert np.array_equal(y2.download(np.uint16, m * n), y1.download(np.uint16, m * n))
    with pytest.raises(RuntimeError):
        lib.norm_mx_split(xb, nw, None, m, k, eps, bool(full), split, need - 1)


@pytest.mark.parametrize("m,k", [(45, 160), (130, 2880)])
def test_add_norm_mx_split_equals_add_norm_then_matmul(lib, m, k):
    """The residual add form: x updated in place, the normalised rows and the
    product bit-identical to oco_add_norm then oco_matmul."""
    from oco_amd import synth
    n, eps = 136, 1e-6
    rng = np.random.default_rng(k)
    w = lib.DeviceBuffer.from_array(synth.weights(39, n, k, seed=81))
    xs = synth.bf16_bits(synth.activations(82, m * k).astype(np.float32))
    ys = synth.bf16_bits((synth.activations(83, m * k) * 0.5).astype(np.float32))
    nw = lib.DeviceBuffer.from_array(rng.normal(1.0, 0.2, k).astype(np.float32))
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    x1, x2 = lib.DeviceBuffer.from_array(xs), lib.DeviceBuffer.from_array(xs)
    yb = lib.DeviceBuffer.from_array(ys)
    o1, o2 = lib.DeviceBuffer(m * k * 2), lib.DeviceBuffer(m * k * 2)
    p1, p2 = lib.DeviceBuffer(m * n * 4), lib.DeviceBuffer(m * n * 4)
    lib.add_norm(x1, yb, nw, o1, m, k, eps, False)
    lib.matmul(39, w, o1, p1, p)
    need = lib.matmul_workspace(39, p)
    split = lib.DeviceBuffer(need)
    lib.add_norm_mx_split(x2, yb, nw, o2, m, k, eps, False, split, need)
    lib.matmul_mx_split(w, split, need, p2, p)
    lib.synchronize()
    assert np.array_equal(x2.download(np.uint16, m * k), x1.download(np.uint16, m * k))
    assert np.array_equal(o2.download(np.uint16, m * k), o1.download(np.uint16, m * k))
    assert np.array_equal(p2.download(np.uint32, m * n), p1.download(np.uint32, m * n))


@pytest.mark.parametrize("fmt,m,n,k", [(P.Q4_0, 3, 64, 256), (P.Q4_1, 4, 96, 512), (39, 1, 70, 2880),
                                       (P.Q8_0, 100, 512, 2880), (0, 200, 64, 96), (P.Q4_K, 1, 256, 512)])
def test_matmul_vector_rows_take_the_matvec(lib, fmt, m, n, k):
    """Up to the reference's vector_rows, oco_matmul is oco_matvec on each
    row, bit for bit, with no workspace."""
    from oco_amd import synth
    say("matmul vector rows", fmt, m, n, k)
    assert m <= vector_rows(fmt, k, n)
    if fmt == 0:
        w = np.frombuffer(np.random.default_rng(3).normal(0, 0.1, n * k).astype(np.float32).tobytes(), np.uint8)
    else:
        w = synth.weights(fmt, n, k, seed=91)
    x = synth.bf16_bits(synth.activations(92, m * k))
    p = lib.Matrix(k, n, m, 0, 1, 1, 0)
    assert lib.matmul_workspace(fmt, p) == 0
    wb, xb = lib.DeviceBuffer.from_array(w), lib.DeviceBuffer.from_array(x)
    y1, y2 = lib.DeviceBuffer(m * n * 2), lib.DeviceBuffer(m * n * 2)
    lib.matmul(fmt, wb, xb, y1, p, y_dtype=lib.DType.BF16)
    lib.matvec(fmt, wb, xb, y2, p, x_dtype=lib.DType.BF16, y_dtype=lib.DType.BF16)
    lib.synchronize()
    assert np.array_equal(y1.download(np.uint16, m * n), y2.download(np.uint16, m * n))


def test_matmul_f32_small_n_past_the_matvec_row_limit(lib):
    """F32 matrices of at most 128 outputs take the matvec at every m up to
    its 65,535-row grid limit (no workspace); past it they take the
    f16-operand product, which meets the half-operand bound."""
    from oco_amd import synth
    n, k = 64, 256
    w = _dense_weights(0, n, k, 41)
    assert lib.matmul_workspace(0, lib.Matrix(k, n, 65535, 0, 1, 1, 0)) == 0
    m = 65600
    say("matmul f32 past the matvec row limit", m, n, k)
    assert lib.matmul_workspace(0, lib.Matrix(k, n, m, 0, 1, 1, 0)) > 0
    x = synth.bf16_bits(synth.activations(42, m * k)).reshape(m, k)
    got = _run_dense(lib, 0, w, x, m, n, k)
    half, mag = O.matmul_reference(0, w, x, n, k, half_operands=True)
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, False))


def test_matmul_q4_row_gain(lib):
    """Q4_0 with more than 1024 outputs: each activation row is scaled by the
    reference's power-of-two gain before the f16 rounding, so rows far
    outside f16 range (2^20 and 2^-30 times N(0,1)) stay finite and within
    the half-operand bound of the gained operands."""
    from oco_amd import synth
    m, n, k = 40, 1100, 256
    w = synth.weights(P.Q4_0, n, k, seed=95)
    xf = synth.activations(96, m * k).reshape(m, k).astype(np.float64)
    xf[::3] *= 2.0 ** 20
    xf[1::3] *= 2.0 ** -30
    xf[5] = 0.0  # a zero row: gain 1
    x = synth.bf16_bits(xf.astype(np.float32)).reshape(m, k)
    got = run(lib, P.Q4_0, w, x, m, n, k)
    assert np.all(np.isfinite(got))
    half, mag = O.matmul_reference(P.Q4_0, w, x, n, k, half_operands=True, row_gain=True)
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, False))
    exact, _ = O.matmul_reference(P.Q4_0, w, x, n, k, half_operands=False)
    for r in range(m):  # each row within the bar of its own scale
        if r == 5:
            assert np.all(got[r] == 0.0)
            continue
        assert rel_l2(got[r], exact[r]) <= 2e-3


@pytest.mark.parametrize("m", [31, 32, 33])
@pytest.mark.parametrize("fmt", [P.Q4_K, P.Q8_0])
def test_matmul_around_the_vendor_threshold(lib, fmt, m):
    """Either side of the 32-row switch between the fused tiles and the
    vendor GEMM: both within the half-operand bound, bias and bf16 output."""
    from oco_amd import synth
    n, k = 260, 512
    w = synth.weights(fmt, n, k, seed=101)
    x = synth.bf16_bits(synth.activations(102, m * k)).reshape(m, k)
    bias = np.random.default_rng(103).normal(size=n).astype(np.float32)
    got = run(lib, fmt, w, x, m, n, k, y_bf16=True, bias=bias)
    half, mag = O.matmul_reference(fmt, w, x, n, k, half_operands=True)
    b = O.bf16_round(bias)
    want = half + b
    assert np.all(np.abs(got - want) <= O.roundoff_bound(want, mag + np.abs(b), k, True))
