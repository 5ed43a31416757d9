"""oco_experts_forward_static (no allocation, static scratch) against
oco_experts_forward with a caller workspace: the same kernels on the same
inputs, so routes, selections and the combined output agree bit for bit, on
two calls in a row (the second smaller, over the first call's leftovers)."""
import ctypes

import numpy as np
import pytest

import oracle as O
from _util import say

pytestmark = pytest.mark.gpu


def _dev(lib, a):
    return lib.DeviceBuffer.from_array(np.ascontiguousarray(a))


def _layer(lib, E, hidden, ffn, k, seed):
    from oco_amd import synth
    rng = np.random.default_rng(seed)
    g, u, d = (synth.weights(39, E * ffn, hidden, seed), synth.weights(39, E * ffn, hidden, seed + 1),
               synth.weights(39, E * hidden, ffn, seed + 2))
    biases = [(rng.normal(size=E * n) * 0.1).astype(np.float32) for n in (ffn, ffn, hidden)]
    bank = lib.ExpertBank(39, hidden, ffn, E, k, *[_dev(lib, a) for a in (g, u, d)],
                          *[_dev(lib, b) for b in biases])
    rw = _dev(lib, (rng.normal(size=(E, hidden)) / np.sqrt(hidden)).astype(np.float32))
    rb = _dev(lib, (rng.normal(size=E) * 0.1).astype(np.float32))
    return bank, rw, rb


def _run(lib, bank, rw, rb, x, resid, tokens, k, static):
    hidden = x.shape[1]
    out = _dev(lib, resid)
    ids, probs = lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    routed = lib.DeviceBuffer(tokens * k * hidden * 4)
    xb = _dev(lib, x)
    if static:
        rc = lib.load_library().oco_experts_forward_static(ctypes.byref(bank.desc), rw.ptr, rb.ptr, xb.ptr,
                                                          int(lib.DType.F32), tokens, out.ptr, ids.ptr, probs.ptr,
                                                          routed.ptr, None)
        assert rc == 0, lib.load_library().oco_last_error()
    else:
        bank.forward(rw, rb, xb, lib.DType.F32, tokens, out, ids, probs, routed=routed)
    lib.synchronize()
    return [b.download(np.uint8) for b in (out, ids, probs, routed)]


def test_static_forward_matches_workspace_forward(lib):
    E, hidden, ffn, k = 32, 2880, 2880, 4
    bank, rw, rb = _layer(lib, E, hidden, ffn, k, seed=500)
    rng = np.random.default_rng(501)
    for tokens in (16, 4, 1):  # each call smaller than the one before
        say("forward_static", tokens)
        x = rng.normal(size=(tokens, hidden)).astype(np.float32)
        resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
        want = _run(lib, bank, rw, rb, x, resid, tokens, k, static=False)
        got = _run(lib, bank, rw, rb, x, resid, tokens, k, static=True)
        for g_, w_ in zip(got, want):
            np.testing.assert_array_equal(g_, w_)


def test_static_forward_rejects_oversize(lib):
    E, hidden, ffn, k = 32, 2880, 2880, 4
    bank, rw, rb = _layer(lib, E, hidden, ffn, k, seed=510)
    L = lib.load_library()
    tokens = 64
    assert bank.workspace_bytes(tokens) > 8 << 20
    rc = L.oco_experts_forward_static(ctypes.byref(bank.desc), rw.ptr, rb.ptr, rw.ptr, int(lib.DType.F32), tokens,
                                      rw.ptr, rw.ptr, rw.ptr, None, None)
    assert rc == 1 and b"scratch" in L.oco_last_error()
