"""GPU parity of the MFMA prefill matmul against the fp64 oracle.

Bars: relative L2 2e-3 of the fp64 product of the exact coefficients for
f16-operand MFMA (the task's bf16/f16-activation bound), 1e-5 for MXFP4 on
bf16 MFMA (exact operands); every element within the reference's roundoff
bound of the half-operand product (matrix_precision.rs:119-142).
"""
import numpy as np
import pytest

import oracle as O
import packers as P
from _util import Guarded, rel_l2, say

pytestmark = pytest.mark.gpu


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
    exact, _ = O.matmul_reference(fmt, w, x, n, k, half_operands=False)
    half, mag = O.matmul_reference(fmt, w, x, n, k, half_operands=(fmt != 39))
    assert rel_l2(got, exact) <= (1e-5 if fmt == 39 else 2e-3)
    assert np.all(np.abs(got - half) <= O.roundoff_bound(half, mag, k, False))


@pytest.mark.parametrize("fmt,n,k", [(39, 5760, 2880), (12, 768, 2048), (8, 512, 4096), (14, 1024, 4096)])
def test_matmul_prefill_shapes(lib, fmt, n, k):
    """BASELINE cfg 5a (MXFP4 5760x2880 x 512 bf16 tokens) and K-quant shapes."""
    from oco_amd import synth
    m = 512
    say("matmul prefill", fmt, n, k)
    w = synth.weights(fmt, n, k, seed=3)
    x = synth.bf16_bits(synth.activations(4, m * k)).reshape(m, k)
    got = run(lib, fmt, w, x, m, n, k)
    exact, _ = O.matmul_reference(fmt, w, x, n, k, half_operands=False)
    assert rel_l2(got, exact) <= (1e-5 if fmt == 39 else 2e-3)


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
