"""GPU parity of the routing and routed-expert path against the oracle.

Known answers and fixtures from the reference's own tests
(src/weights/dispatch_tests/mxfp4.rs): logits_selecting([3,0,2,1]), the
MXFP4 decode packer at K=2880/N=33 with the unaligned byte offset, the
E8M0=255 NaN rule, and the batch-17/257 id pattern with overfull experts.
"""
import numpy as np
import pytest

import oracle as O
import packers as P
from _util import Guarded, rel_l2, say, upload_at_offset

pytestmark = pytest.mark.gpu

# Bar of the MXFP4 expert tiles (from 4 tokens on): north_star's 1e-5 for
# f32 activations with fp32 accumulation.  The block-scaled MFMA takes the
# input rows and the f32 gate/up activations as four E2M3 terms each (at
# most 1/50625 of the block maximum per value); measured ~1.1e-6 on N(0,1)
# rows and the heavy-tailed SwiGLU activations of the down pass, at
# hidden = ffn = 512 and at gpt-oss shape.
MX_TILE_BAR = 1e-5


def dev(oco, a):
    return oco.DeviceBuffer.from_array(np.ascontiguousarray(a))


def out_bound(want, routes, k):
    """Per-element bound on the bf16 layer output: the output's own rounding,
    the bf16 roundings of the k routes and of their weighted sum on both
    sides (a route error can flip any of them), and the route error carried
    into the sum; `routes` is the oracle's [tokens * k, hidden]."""
    mag = np.abs(routes).reshape(-1, k, routes.shape[-1]).sum(axis=1)
    return 2 ** -6 * np.abs(want) + (2 * k * 2 ** -9 + 1e-4) * mag + 2e-2


# ---- routing ------------------------------------------------------------------

@pytest.mark.parametrize("tokens,experts,k", [(1, 32, 4), (16, 32, 4), (257, 32, 4), (512, 128, 8),
                                              (3, 5, 5), (7, 256, 8)])
def test_route_select_matches_oracle(lib, tokens, experts, k):
    say("route_select", tokens, experts, k)
    rng = np.random.default_rng(tokens * 1000 + experts)
    logits = rng.normal(size=(tokens, experts)).astype(np.float32)
    logits[0, :4] = 0.5  # a tie at the top: lowest index wins
    ids_b, probs_b = lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    lib.route_select(dev(lib, logits), tokens, experts, k, ids_b, probs_b)
    lib.synchronize()
    ids, probs = ids_b.download(np.uint32).reshape(tokens, k), probs_b.download(np.float32).reshape(tokens, k)
    want_ids, want_probs = O.select_experts(logits, k)
    np.testing.assert_array_equal(ids, want_ids)
    # probabilities are bf16: equal up to one bf16 step (exp is not bit-pinned)
    np.testing.assert_allclose(probs, want_probs, rtol=2 ** -7, atol=0)


def test_route_select_known_answer_and_nan(lib):
    logits = np.stack([P.logits_selecting([3, 0, 2, 1]), np.zeros(32, np.float32),
                       np.where(np.arange(32) == 5, np.nan, 0.0).astype(np.float32)])
    ids_b, probs_b = lib.DeviceBuffer(3 * 16), lib.DeviceBuffer(3 * 16)
    lib.route_select(dev(lib, logits), 3, 32, 4, ids_b, probs_b)
    lib.synchronize()
    ids, probs = ids_b.download(np.uint32).reshape(3, 4), probs_b.download(np.float32).reshape(3, 4)
    assert list(ids[0]) == [3, 0, 2, 1]
    assert list(ids[1]) == [0, 1, 2, 3] and np.all(probs[1] == 0.25)
    assert np.all(ids[2] < 32) and np.all(np.isnan(probs[2]))


@pytest.mark.parametrize("tokens,hidden,experts,dtype,offset", [
    (5, 2880, 32, "f32", 0), (16, 2880, 32, "bf16", 0), (1, 2048, 128, "bf16", 0),
    (7, 2882, 32, "f32", 0),   # hidden % 4 != 0: the one-wavefront kernel
    (3, 2880, 32, "f32", 4)])  # rows not 16-byte aligned: the one-wavefront kernel
def test_router_logits(lib, tokens, hidden, experts, dtype, offset):
    k = 4
    say("router", tokens, hidden, experts, dtype, offset)
    rng = np.random.default_rng(11)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    w = (rng.normal(size=(experts, hidden)) * 0.02).astype(np.float32)
    b = rng.normal(size=experts).astype(np.float32)
    xin, dt = (x, lib.DType.F32) if dtype == "f32" else (O.f32_to_bf16(x), lib.DType.BF16)
    if dtype == "bf16":
        x = O.bf16_to_f32(xin)
    xbuf = lib.DeviceBuffer(xin.nbytes + offset)
    xbuf.upload(xin, offset)
    lb, ib, pb = lib.DeviceBuffer(tokens * experts * 4), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    lib.router(xbuf.ptr + offset, dt, dev(lib, w), dev(lib, b), tokens, hidden, experts, k, lb, ib, pb)
    lib.synchronize()
    got = lb.download(np.float32).reshape(tokens, experts)
    want = O.bf16_round(x) @ O.bf16_round(w).T + O.bf16_round(b)
    assert rel_l2(got, want) < 1e-5
    want_ids, _ = O.select_experts(got, k)
    np.testing.assert_array_equal(ib.download(np.uint32).reshape(tokens, k), want_ids)


@pytest.mark.parametrize("batch,experts,tile,invalid", [(1, 32, 16, 0), (17, 32, 64, 0), (257, 32, 64, 0),
                                                        (512, 128, 16, 0), (600, 128, 32, 0), (2048, 128, 64, 0),
                                                        (300, 256, 16, 0), (700, 64, 16, 1), (3000, 64, 32, 1)])
def test_route_plan_bit_exact(lib, batch, experts, tile, invalid):
    """The one-pass plan (up to 8 chunks of 1024 routes) and the chunked one
    (3000 x 8 routes); `invalid`: about 5% of the ids are >= experts, which
    the plan leaves out (routing.metal:4-39 skips them too)."""
    say("route_plan", batch, experts, tile, invalid)
    if experts == 32 and batch > 1:
        ids = P.expert_ids(batch)
    elif batch == 1:
        ids = np.array([3, 0, 2, 1], np.uint32)
    else:
        rng = np.random.default_rng(3)
        ids = rng.integers(0, experts, batch * 8).astype(np.uint32)
        if invalid:
            bad = rng.random(ids.size) < 0.05
            ids[bad] = experts + rng.integers(0, 1000, int(bad.sum())).astype(np.uint32)
    routes = ids.size
    words = lib.route_plan_words(routes, experts)
    assert words == O.route_plan_words(routes, experts)
    out = Guarded(lib, words * 4)
    lib.route_plan(dev(lib, ids), routes, experts, tile, 9, 5, out.ptr)
    lib.synchronize()
    want, tiles = O.route_plan(ids, experts, tile, 9, 5)
    got = out.read(np.uint32)
    # Defined words: grids, used tile pairs, each list's count and entries,
    # sorted offsets and route rows (unused slots are unspecified).
    defined = np.zeros(words, bool)
    defined[:6 + 2 * tiles] = True
    grouped = 6 + 2 * ((routes + 15) // 16 + experts)
    for e in range(experts):
        base = grouped + e * (routes + 1)
        defined[base:base + 1 + want[base]] = True
    defined[grouped + experts * (routes + 1):] = True
    # a left-out route has no row (the reference never writes it)
    defined[grouped + experts * (routes + 1) + experts + np.nonzero(ids >= experts)[0]] = False
    np.testing.assert_array_equal(got[defined], want[defined])


@pytest.mark.parametrize("hidden,k", [(2880, 4), (2884, 4), (2880, 8), (2884, 1), (2880, 3)])
def test_moe_sum(lib, hidden, k):
    """hidden % 8 == 0 takes the eight-wide kernel, else the scalar one; k
    from 1 to the limit of 8."""
    tokens = 16
    rng = np.random.default_rng(5)
    routes = O.f32_to_bf16(rng.normal(size=(tokens * k, hidden)).astype(np.float32))
    probs = O.bf16_round(rng.dirichlet(np.ones(k), size=tokens)).astype(np.float32)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    outb = dev(lib, resid)
    lib.moe_sum(dev(lib, routes), lib.DType.BF16, dev(lib, probs), outb, hidden, tokens, k)
    lib.synchronize()
    got = outb.download(np.uint16).reshape(tokens, hidden)
    want = O.moe_sum(routes, probs, resid, k)
    # fp32 sums may differ by fused rounding: at most one bf16 step apart
    diff = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert diff.max() <= 1 and (diff > 0).mean() < 0.01
    # the eight-wide and scalar kernels agree bit for bit (an output 2 bytes
    # past a 16-byte boundary takes the scalar kernel)
    buf = lib.DeviceBuffer(resid.nbytes + 16)
    buf.upload(resid, 2)
    lib.moe_sum(dev(lib, routes), lib.DType.BF16, dev(lib, probs), buf.ptr + 2, hidden, tokens, k)
    lib.synchronize()
    assert np.array_equal(buf.download(np.uint16, tokens * hidden, 2).reshape(tokens, hidden), got)


# ---- expert projections -------------------------------------------------------

def bank(oco, fmt, experts, hidden, ffn, seed):
    from oco_amd import synth
    g = synth.weights(fmt, experts * ffn, hidden, seed)
    u = synth.weights(fmt, experts * ffn, hidden, seed + 1)
    d = synth.weights(fmt, experts * hidden, ffn, seed + 2)
    rng = np.random.default_rng(seed)
    gb = (rng.normal(size=experts * ffn) * 0.1).astype(np.float32)
    ub = (rng.normal(size=experts * ffn) * 0.1).astype(np.float32)
    db = (rng.normal(size=experts * hidden) * 0.1).astype(np.float32)
    return (g, u, d, gb, ub, db), [dev(oco, a) for a in (g, u, d, gb, ub, db)]


def test_expert_expand_reference_fixture(lib):
    """expert_expand at K=2880, N=33 on the reference's MXFP4 packer, weights at
    byte offset 7, ids [3,0,2,1] chosen from logits (mxfp4.rs:46-179)."""
    k, n = 2880, 33
    data, coeffs = P.mxfp4_decode_weights(k, n)
    body = np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:]
    wbuf, wptr = upload_at_offset(lib, body, P.WEIGHT_OFFSET)
    x = P.mxfp4_decode_input(k)[:k]
    xb = O.f32_to_bf16(x)
    bias = np.array([((P.noise(i + 151) % 997) - 498) / 509.0 for i in range(4 * n)], np.float32)
    bias32 = np.zeros(32 * n, np.float32)
    bias32[:4 * n] = bias
    ids = [3, 0, 2, 1]
    bk = lib.ExpertBank(39, k, n, 32, 4, wptr, wptr, wptr, dev(lib, bias32), dev(lib, bias32), None)
    up, act = Guarded(lib, 4 * n * 4), Guarded(lib, 4 * n * 4)
    ib, pb = lib.DeviceBuffer(16), lib.DeviceBuffer(16)
    bk.expand(dev(lib, xb), lib.DType.BF16, dev(lib, P.logits_selecting(ids)), ib, pb, up.ptr, act.ptr)
    lib.synchronize()
    assert list(ib.download(np.uint32)) == ids
    W = coeffs.reshape(4, n, k)
    xf = O.bf16_to_f32(xb).astype(np.float64)
    got_up, got_act = up.read(np.float32).reshape(4, n), act.read(np.float32).reshape(4, n)
    for r, e in enumerate(ids):
        ub = O.bf16_round(bias[e * n:(e + 1) * n] + 1.0)
        gb = O.bf16_round(bias[e * n:(e + 1) * n])
        want_up = W[e] @ xf + ub
        mag = np.abs(W[e]) @ np.abs(xf) + np.abs(ub)
        assert np.all(np.abs(got_up[r] - want_up) <= O.roundoff_bound(want_up, mag, k, False))
        want_act = O.swiglu_clipped_f64(W[e] @ xf + gb, want_up)
        assert np.all(np.abs(got_act[r] - want_act) <= 1e-3 * np.maximum(np.abs(want_act), 1.0))
    # E8M0 255 in the first selected expert's first block propagates NaN (mxfp4.rs:205-233)
    bad = body.copy()
    bad[ids[0] * n * (k // 32) * 17] = 255
    wbuf.upload(bad, P.WEIGHT_OFFSET)
    bk.expand(dev(lib, xb), lib.DType.BF16, dev(lib, P.logits_selecting(ids)), ib, pb, up.ptr, act.ptr)
    lib.synchronize()
    assert np.isnan(up.read(np.float32)[0])


@pytest.mark.parametrize("fmt", [39, 12])
@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_experts_apply_matches_oracle(lib, fmt, tokens):
    """Full routed layer after the router: gate/up + clipped SwiGLU + down +
    weighted combine with residual, batches 1/4/16 (BASELINE cfg 4 shapes
    scaled down to hidden = ffn = 512)."""
    E, hidden, ffn, k = 32, 512, 512, 4
    say("experts_apply", fmt, tokens)
    host, devs = bank(lib, fmt, E, hidden, ffn, seed=40 + tokens)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(tokens)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    act = 0 if fmt == 39 else 1
    bk = lib.ExpertBank(fmt, hidden, ffn, E, k, *devs, activation=act, up_bias_one=(fmt == 39))
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, x), lib.DType.F32, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    got_out = outb.download(np.uint16).reshape(tokens, hidden)
    got_routed = routed.read(np.float32).reshape(tokens * k, hidden)
    ref = O.experts_reference(fmt, hidden, ffn, g, u, d, x, ids, probs, resid, gb, ub, db,
                              activation=act, up_one=(fmt == 39))
    err = rel_l2(got_routed, ref["down"])
    say("relL2", err)
    # MXFP4 banks from 4 tokens on run the E2M3-split MFMA tiles; the rest
    # the routed fp32 kernel
    assert err < (MX_TILE_BAR if fmt == 39 and tokens >= 4 else 1e-5)
    want = O.bf16_to_f32(ref["out"])
    diff = np.abs(O.bf16_to_f32(got_out).astype(np.float64) - want)
    assert np.all(diff <= out_bound(want, ref["down"], k))


@pytest.mark.parametrize("tokens", [6, 20])
def test_experts_apply_mx_tiles_bf16_lone_blocks(lib, tokens):
    """MXFP4 banks on the block-scaled MFMA tiles at decode batch sizes (16-
    and 32-row plan tiles) with bf16 inputs (split beside the router or the
    route plan) and block counts that leave a lone last block in both projections
    (hidden = 96, ffn = 160: the gate/up tiles zero the activations' partner
    block)."""
    E, hidden, ffn, k = 16, 96, 160, 4
    say("experts_apply mx tiles bf16", tokens)
    host, devs = bank(lib, 39, E, hidden, ffn, seed=90 + tokens)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(100 + tokens)
    xb = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(39, hidden, ffn, E, k, *devs, activation=0, up_bias_one=True)
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, xb), lib.DType.BF16, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    ref = O.experts_reference(39, hidden, ffn, g, u, d, O.bf16_to_f32(xb), ids, probs, resid, gb, ub, db,
                              activation=0, up_one=True)
    assert rel_l2(routed.read(np.float32).reshape(tokens * k, hidden), ref["down"]) < MX_TILE_BAR
    got = O.bf16_to_f32(outb.download(np.uint16).reshape(tokens, hidden)).astype(np.float64)
    want = O.bf16_to_f32(ref["out"])
    assert np.all(np.abs(got - want) <= out_bound(want, ref["down"], k))


def test_experts_overfull_tiles(lib):
    """Batch 257 with ids [31, t%15, 15+t%8, 30]: experts 30/31 own 257 routes each,
    spanning many tiles (mxfp4.rs:309-482).  An MXFP4 bank at 257 tokens runs
    on the block-scaled MFMA tiles of 32 rows (f32 inputs and activations in
    four E2M3 terms): bar MX_TILE_BAR."""
    E, hidden, ffn, k, tokens = 32, 96, 96, 4, 257
    say("experts overfull")
    host, devs = bank(lib, 39, E, hidden, ffn, seed=77)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(7)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids = P.expert_ids(tokens).reshape(tokens, k)
    probs = np.full((tokens, k), 0.25, np.float32)
    resid = np.zeros((tokens, hidden), np.uint16)
    bk = lib.ExpertBank(39, hidden, ffn, E, k, *devs)
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, x), lib.DType.F32, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    ref = O.experts_reference(39, hidden, ffn, g, u, d, x, ids, probs, resid, gb, ub, db)
    err = rel_l2(routed.read(np.float32).reshape(-1, hidden), ref["down"])
    say("overfull relL2", err)
    assert err < MX_TILE_BAR


@pytest.mark.parametrize("tokens", [1, 4, 16])
def test_experts_full_shape(lib, tokens):
    """gpt-oss-20b shape: 32 experts, hidden = ffn = 2880, MXFP4, top-4, at the
    decode batches of the benchmark.  Batch 1 runs the routed fp32 kernel
    (bar 1e-5); batch 4 the MXFP4 tiles with the K-split down pass and
    batch 16 the unsplit down pass (2 x 1656 workgroups exceed three rounds
    of 256 CUs), both on four-term E2M3 activations (bar MX_TILE_BAR)."""
    E, hidden, ffn, k = 32, 2880, 2880, 4
    say("experts full shape", tokens)
    host, devs = bank(lib, 39, E, hidden, ffn, seed=5)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(9)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(39, hidden, ffn, E, k, *devs)
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, x), lib.DType.F32, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    ref = O.experts_reference(39, hidden, ffn, g, u, d, x, ids, probs, resid, gb, ub, db)
    err = rel_l2(routed.read(np.float32).reshape(-1, hidden), ref["down"])
    say("full shape relL2", tokens, err)
    assert err < (1e-5 if tokens == 1 else MX_TILE_BAR)
    want = O.bf16_to_f32(ref["out"])
    diff = np.abs(O.bf16_to_f32(outb.download(np.uint16).reshape(tokens, hidden)).astype(np.float64) - want)
    assert np.all(diff <= out_bound(want, ref["down"], k))

    # The timed path: oco_experts_forward from the router weights (at 4 and 16
    # tokens the selection and route plan run inside every gate/up
    # workgroup; at one token inside the routed kernel) equals oco_router
    # followed by oco_experts_apply bit for bit at this shape.
    rw = (rng.normal(size=(E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    rb = (rng.normal(size=E) * 0.1).astype(np.float32)
    xb, rwb, rbb = dev(lib, x), dev(lib, rw), dev(lib, rb)
    out1, ids1, probs1 = dev(lib, resid), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    routed1 = Guarded(lib, tokens * k * hidden * 4)
    bk.forward(rwb, rbb, xb, lib.DType.F32, tokens, out1, ids1, probs1, routed=routed1.ptr)
    logits = lib.DeviceBuffer(tokens * E * 4)
    out2, ids2, probs2 = dev(lib, resid), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    routed2 = Guarded(lib, tokens * k * hidden * 4)
    lib.router(xb, lib.DType.F32, rwb, rbb, tokens, hidden, E, k, logits, ids2, probs2)
    bk.apply(xb, lib.DType.F32, ids2, probs2, tokens, out2, routed=routed2.ptr)
    lib.synchronize()
    np.testing.assert_array_equal(ids1.download(np.uint32), ids2.download(np.uint32))
    np.testing.assert_array_equal(probs1.download(np.uint32), probs2.download(np.uint32))
    np.testing.assert_array_equal(routed1.read(np.uint32), routed2.read(np.uint32))
    np.testing.assert_array_equal(out1.download(np.uint16), out2.download(np.uint16))
    want_ids, _ = O.select_experts(logits.download(np.float32).reshape(tokens, E), k)
    np.testing.assert_array_equal(ids1.download(np.uint32).reshape(tokens, k), want_ids)


@pytest.mark.parametrize("tokens", [1, 4, 40])
def test_experts_nonfinite_gate_and_up(lib, tokens):
    """One gate row and one up row of expert 0 carry a block whose E8M0
    scale is 2^127 with a code of 6 (6 * 2^127 overflows f32): those gate and
    up values are non-finite, the activation rule turns them into NaN
    (projections.metal:5-8), and every route through expert 0 comes out NaN
    in every column, as in the oracle; routes through other experts stay
    finite and within their bar.  Batch 1 runs the routed kernel, 4 the
    block-scaled MFMA tiles, 40 the prefill tiles."""
    E, hidden, ffn, k = 8, 256, 128, 2
    say("experts nonfinite gate/up", tokens)
    host, _ = bank(lib, 39, E, hidden, ffn, seed=210 + tokens)
    g, u, d, gb, ub, db = [a.copy() for a in host]
    rb = hidden // 32 * 17
    for arr, row in ((g, 5), (u, 77)):  # expert 0: gate row 5, up row 77, second block
        blk = row * rb + 17
        arr[blk] = 254
        arr[blk + 1:blk + 17] = 0
        arr[blk + 1] = 0x7  # code 7 = 6.0 in column 0 of the block
    rng = np.random.default_rng(211)
    x = np.abs(rng.normal(size=(tokens, hidden))).astype(np.float32) + 0.5
    logits = rng.normal(size=(tokens, E)).astype(np.float32)
    logits[:, 0] += 10.0  # every token routes through expert 0 ...
    logits[0, 0] -= 20.0  # ... except token 0
    ids, probs = O.select_experts(logits, k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(39, hidden, ffn, E, k, *[dev(lib, a) for a in (g, u, d, gb, ub, db)])
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, x), lib.DType.F32, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    ref = O.experts_reference(39, hidden, ffn, g, u, d, x, ids, probs, resid, gb, ub, db)
    assert np.isnan(ref["act"][ids.reshape(-1) == 0][:, [5, 77]]).all()
    got = routed.read(np.float32).reshape(-1, hidden)
    bad = np.isnan(ref["down"]).any(axis=1)
    assert bad.sum() == tokens - 1 and not bad[:k].any()
    np.testing.assert_array_equal(bad, ids.reshape(-1) == 0)
    assert np.isnan(got[bad]).all()
    assert np.isfinite(got[~bad]).all()
    bar = 1e-5 if tokens == 1 else MX_TILE_BAR if tokens < 32 else 2e-3
    assert rel_l2(got[~bad], ref["down"][~bad]) < bar
    out = O.bf16_to_f32(outb.download(np.uint16).reshape(tokens, hidden))
    np.testing.assert_array_equal(np.isnan(out), np.isnan(O.bf16_to_f32(ref["out"])))


@pytest.mark.parametrize("ks", [1, 2])
@pytest.mark.parametrize("ffn", [512, 640])
def test_experts_mx_down_k_split(lib, ks, ffn):
    """The MXFP4 down tiles of 16 rows with and without the split of K over
    two halves of the workgroup, forced either way: ffn 640 gives 3 quads of
    K steps, so the two parts hold unequal real work (2 and 1 quads)."""
    E, hidden, k, tokens = 16, 256, 4, 6
    say("experts mx down ks", ks, ffn)
    host, devs = bank(lib, 39, E, hidden, ffn, seed=120 + ffn)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(121)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(39, hidden, ffn, E, k, *devs)
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    with lib.overridden(lib.Knob.MX_EXPERTS_KS, [ks]):
        bk.apply(dev(lib, x), lib.DType.F32, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
        lib.synchronize()
    ref = O.experts_reference(39, hidden, ffn, g, u, d, x, ids, probs, resid, gb, ub, db)
    err = rel_l2(routed.read(np.float32).reshape(-1, hidden), ref["down"])
    say("relL2", err)
    assert err < MX_TILE_BAR


# ---- prefill: grouped MFMA tiles -----------------------------------------------

def _prefill_case(lib, fmt, E, hidden, ffn, k, tokens, x_dtype, seed, clipped):
    host, devs = bank(lib, fmt, E, hidden, ffn, seed=seed)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    act = 0 if clipped else 1
    if clipped:
        bk = lib.ExpertBank(fmt, hidden, ffn, E, k, *devs, activation=act, up_bias_one=True)
    else:  # Qwen3 MoE: no biases, plain SwiGLU
        bk = lib.ExpertBank(fmt, hidden, ffn, E, k, devs[0], devs[1], devs[2], activation=act, up_bias_one=False)
        gb = ub = db = None
    if x_dtype == "bf16":
        xin, xdt = O.f32_to_bf16(x), lib.DType.BF16
        x = O.bf16_to_f32(xin)
    else:
        xin, xdt = x, lib.DType.F32
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, xin), xdt, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    ref = O.experts_reference(fmt, hidden, ffn, g, u, d, x, ids, probs, resid, gb, ub, db,
                              activation=act, up_one=clipped)
    return routed.read(np.float32).reshape(tokens * k, hidden), outb.download(np.uint16).reshape(tokens, hidden), ref


@pytest.mark.parametrize("fmt,clipped", [(12, False), (12, True), (14, False), (8, False), (39, True)])
@pytest.mark.parametrize("tokens,x_dtype", [(32, "f32"), (130, "bf16")])
def test_experts_prefill_matches_oracle(lib, fmt, clipped, tokens, x_dtype):
    """Grouped MFMA prefill (expert_up_tensor / moe_activate / expert_down_tensor,
    projections.metal:192-376): f16 operands and f16 activations as in the
    reference's tiles; bar relL2 2e-3 on the route outputs, the combine within
    bf16 roundings of the reference's."""
    E, hidden, ffn, k = 16, 512, 256, 4
    say("experts prefill", fmt, tokens, x_dtype)
    got, out, ref = _prefill_case(lib, fmt, E, hidden, ffn, k, tokens, x_dtype, 60 + fmt + tokens, clipped)
    assert rel_l2(got, ref["down"]) < 2e-3
    want = O.bf16_to_f32(ref["out"])
    diff = np.abs(O.bf16_to_f32(out).astype(np.float64) - want)
    # bf16 roundings of the output plus those of the k partial sums (each up
    # to 2^-9 of sum |y_r| p_r, on both sides: 2 k 2^-9 = 1.6e-2 at k = 4),
    # plus the route error carried by that sum
    mag = np.abs(ref["down"]).reshape(tokens, k, hidden).sum(axis=1)
    assert np.all(diff <= 2 ** -6 * np.abs(want) + (2 * k * 2 ** -9 + 2e-3) * mag + 2e-2)


def test_experts_prefill_qwen3_shape(lib):
    """Qwen3-30B-A3B layer geometry (hidden 2048, ffn 768, Q4_K, top-8, SwiGLU)
    at 512 tokens over 8 experts: ~512 routes per expert, many 64-row tiles."""
    E, hidden, ffn, k, tokens = 8, 2048, 768, 8, 512
    say("experts prefill qwen3 shape")
    got, _, ref = _prefill_case(lib, 12, E, hidden, ffn, k, tokens, "bf16", 91, False)
    assert rel_l2(got, ref["down"]) < 2e-3


def test_experts_prefill_qwen3_30b_a3b_geometry(lib):
    """BASELINE cfg 5b at its own geometry: 128 experts of hidden 2048 / ffn
    768, Q4_K, SwiGLU without biases, top-8 of N(0,1) logits over 512 tokens
    (4,096 routes, 32 per expert on average).  The plan then takes 48-row
    tiles over all 128 experts; experts past 48 routes spill into overflow
    tiles (more than 128 tiles in all), which hand some persistent
    workgroups an extra unit.  This is the layer the bench times."""
    E, hidden, ffn, k, tokens = 128, 2048, 768, 8, 512
    say("experts prefill qwen3-30b-a3b geometry")
    host, devs = bank(lib, 12, E, hidden, ffn, seed=95)
    g, u, d = host[:3]
    rng = np.random.default_rng(95)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    tiles = int(np.sum((counts + 47) // 48))
    say("routes per expert", counts.min(), counts.max(), "tiles of 48:", tiles)
    assert (counts > 0).all() and counts.max() > 48 and tiles > E
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(12, hidden, ffn, E, k, devs[0], devs[1], devs[2], activation=1, up_bias_one=False)
    xin = O.f32_to_bf16(x)
    outb = dev(lib, resid)
    routed = Guarded(lib, tokens * k * hidden * 4)
    bk.apply(dev(lib, xin), lib.DType.BF16, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed.ptr)
    lib.synchronize()
    ref = O.experts_reference(12, hidden, ffn, g, u, d, O.bf16_to_f32(xin), ids, probs, resid,
                              activation=1, up_one=False)
    got = routed.read(np.float32).reshape(tokens * k, hidden)
    err = rel_l2(got, ref["down"])
    say("relL2", err)
    assert err < 2e-3
    want = O.bf16_to_f32(ref["out"])
    diff = np.abs(O.bf16_to_f32(outb.download(np.uint16).reshape(tokens, hidden)).astype(np.float64) - want)
    mag = np.abs(ref["down"]).reshape(tokens, k, hidden).sum(axis=1)
    assert np.all(diff <= 2 ** -6 * np.abs(want) + (2 * k * 2 ** -9 + 2e-3) * mag + 2e-2)
    # forced 64-row tiles (every expert in one tile) give the same routes
    # within the bar: the tile choice only regroups rows
    with lib.overridden(lib.Knob.MOE_Q4_ROWS, [64]):
        routed64 = Guarded(lib, tokens * k * hidden * 4)
        bk.apply(dev(lib, xin), lib.DType.BF16, dev(lib, ids), dev(lib, probs), tokens, dev(lib, resid),
                 routed=routed64.ptr)
        lib.synchronize()
    assert rel_l2(routed64.read(np.float32).reshape(tokens * k, hidden), ref["down"]) < 2e-3


def test_experts_prefill_q4k_ranges_over_tiles(lib):
    """Q4_K prefill where each persistent workgroup runs several units over
    more than one tile (hidden 256: two column chunks per down tile; 1024
    tokens: more units than workgroups), with biases and the clipped
    activation."""
    E, hidden, ffn, k, tokens = 32, 256, 256, 8, 1024
    say("experts prefill q4k ranges")
    got, _, ref = _prefill_case(lib, 12, E, hidden, ffn, k, tokens, "bf16", 93, True)
    assert rel_l2(got, ref["down"]) < 2e-3


@pytest.mark.parametrize("fmt", [12, 39])
def test_experts_prefill_bf16_routes_bit_identical(lib, fmt):
    """Without `routed` the down tiles store bf16 routes (as the reference
    does); moe_sum rounds f32 routes to bf16 first, so both runs agree bit
    for bit."""
    E, hidden, ffn, k, tokens = 16, 512, 256, 4, 64
    host, devs = bank(lib, fmt, E, hidden, ffn, seed=17)
    rng = np.random.default_rng(17)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    ids, probs = O.select_experts(rng.normal(size=(tokens, E)).astype(np.float32), k)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(fmt, hidden, ffn, E, k, *devs, activation=0 if fmt == 39 else 1, up_bias_one=fmt == 39)
    outs = []
    for with_routed in (True, False):
        outb = dev(lib, resid)
        routed = lib.DeviceBuffer(tokens * k * hidden * 4) if with_routed else None
        bk.apply(dev(lib, x), lib.DType.F32, dev(lib, ids), dev(lib, probs), tokens, outb, routed=routed)
        lib.synchronize()
        outs.append(outb.download(np.uint16))
    np.testing.assert_array_equal(outs[0], outs[1])


# ---- the layer from the router on ---------------------------------------------

@pytest.mark.parametrize("fmt,tokens", [(39, 1), (39, 4), (39, 16), (12, 2), (12, 40)])
def test_experts_forward_from_router(lib, fmt, tokens):
    """oco_experts_forward (router logits -> selection -> experts -> combine,
    feed_forward.rs:107-275) equals oco_router followed by oco_experts_apply
    bit for bit (one token: the selection runs inside the gate/up kernel, as
    expert_expand does), its ids are the oracle's top-k of the GPU logits,
    and its routes match the fp64 oracle."""
    E, hidden, ffn, k = 32, 512, 256, 4
    say("experts forward", fmt, tokens)
    host, devs = bank(lib, fmt, E, hidden, ffn, seed=130 + tokens)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(131 + tokens)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    rw = (rng.normal(size=(E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    rb = (rng.normal(size=E) * 0.1).astype(np.float32)
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    act = 0 if fmt == 39 else 1
    bk = lib.ExpertBank(fmt, hidden, ffn, E, k, *devs, activation=act, up_bias_one=(fmt == 39))
    xb, rwb, rbb = dev(lib, x), dev(lib, rw), dev(lib, rb)

    out1, ids1, probs1 = dev(lib, resid), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    routed1 = Guarded(lib, tokens * k * hidden * 4)
    bk.forward(rwb, rbb, xb, lib.DType.F32, tokens, out1, ids1, probs1, routed=routed1.ptr)
    lib.synchronize()

    logits = lib.DeviceBuffer(tokens * E * 4)
    out2, ids2, probs2 = dev(lib, resid), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
    routed2 = Guarded(lib, tokens * k * hidden * 4)
    lib.router(xb, lib.DType.F32, rwb, rbb, tokens, hidden, E, k, logits, ids2, probs2)
    bk.apply(xb, lib.DType.F32, ids2, probs2, tokens, out2, routed=routed2.ptr)
    lib.synchronize()

    ids = ids1.download(np.uint32).reshape(tokens, k)
    np.testing.assert_array_equal(ids, ids2.download(np.uint32).reshape(tokens, k))
    np.testing.assert_array_equal(probs1.download(np.uint32), probs2.download(np.uint32))
    np.testing.assert_array_equal(routed1.read(np.uint32), routed2.read(np.uint32))
    np.testing.assert_array_equal(out1.download(np.uint16), out2.download(np.uint16))
    want_ids, want_probs = O.select_experts(logits.download(np.float32).reshape(tokens, E), k)
    np.testing.assert_array_equal(ids, want_ids)
    np.testing.assert_allclose(probs1.download(np.float32).reshape(tokens, k), want_probs, rtol=2 ** -7, atol=0)
    ref = O.experts_reference(fmt, hidden, ffn, g, u, d, x, ids, probs1.download(np.float32).reshape(tokens, k),
                              resid, gb, ub, db, activation=act, up_one=(fmt == 39))
    err = rel_l2(routed1.read(np.float32).reshape(-1, hidden), ref["down"])
    say("relL2", err)
    bar = MX_TILE_BAR if fmt == 39 and tokens >= 4 else 2e-3 if tokens >= 32 else 1e-5
    assert err < bar


@pytest.mark.parametrize("tokens,case,E", [(4, "ties", 32), (16, "ties", 32), (16, "nonfinite", 32), (1, "plain", 32),
                                          (9, "plain", 32), (8, "plain", 64), (5, "ties", 48), (8, "nonfinite", 64)])
def test_experts_forward_in_tile_plan(lib, tokens, case, E):
    """MXFP4 decode batches (routes <= 64, experts <= 64): every gate/up
    workgroup selects and plans by itself and the input split rides in the
    router's launch.  Selection by rank must equal the repeated maximum of
    oco_route_select bit for bit, ties to the lowest expert included (all
    router weights zero, biases with repeated values) and non-finite logits
    (a NaN input row: that token's probabilities are NaN); batch 1 is forced
    onto the tiles through the MOE_MX_TOKENS knob.  32 experts take the
    32-wide rank rows, 48 and 64 the 64-wide ones (at most 8 tokens)."""
    hidden, ffn, k = 256, 128, 4
    say("experts forward in-tile plan", tokens, case, E)
    host, devs = bank(lib, 39, E, hidden, ffn, seed=150 + tokens)
    g, u, d, gb, ub, db = host
    rng = np.random.default_rng(151 + tokens)
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    rw = (rng.normal(size=(E, hidden)) / np.sqrt(hidden)).astype(np.float32)
    rb = (rng.normal(size=E) * 0.1).astype(np.float32)
    if case == "ties":
        rw[:] = 0
        rb = np.array([0.5, 0.25, 0.5, 0.25] * (E // 4), np.float32)
    if case == "nonfinite":
        x[3, 7] = np.nan  # token 3: every logit NaN
    resid = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    bk = lib.ExpertBank(39, hidden, ffn, E, k, *devs, activation=0, up_bias_one=True)
    xb, rwb, rbb = dev(lib, x), dev(lib, rw), dev(lib, rb)
    with lib.overridden(lib.Knob.MOE_MX_TOKENS, [1]):
        out1, ids1, probs1 = dev(lib, resid), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
        routed1 = Guarded(lib, tokens * k * hidden * 4)
        bk.forward(rwb, rbb, xb, lib.DType.F32, tokens, out1, ids1, probs1, routed=routed1.ptr)
        logits = lib.DeviceBuffer(tokens * E * 4)
        out2, ids2, probs2 = dev(lib, resid), lib.DeviceBuffer(tokens * k * 4), lib.DeviceBuffer(tokens * k * 4)
        routed2 = Guarded(lib, tokens * k * hidden * 4)
        lib.router(xb, lib.DType.F32, rwb, rbb, tokens, hidden, E, k, logits, ids2, probs2)
        bk.apply(xb, lib.DType.F32, ids2, probs2, tokens, out2, routed=routed2.ptr)
        lib.synchronize()
    ids = ids1.download(np.uint32).reshape(tokens, k)
    np.testing.assert_array_equal(ids, ids2.download(np.uint32).reshape(tokens, k))
    np.testing.assert_array_equal(probs1.download(np.uint32), probs2.download(np.uint32))
    np.testing.assert_array_equal(out1.download(np.uint16), out2.download(np.uint16))
    p = probs1.download(np.float32).reshape(tokens, k)
    if case == "ties":  # experts 0, 2, 4, 6 (bias 0.5, lowest indices first)
        np.testing.assert_array_equal(ids, np.tile(np.array([0, 2, 4, 6], np.uint32), (tokens, 1)))
        np.testing.assert_array_equal(p, np.full((tokens, k), 0.25, np.float32))
    if case == "nonfinite":
        assert np.isnan(p[3]).all() and not np.isnan(np.delete(p, 3, axis=0)).any()
        return
    np.testing.assert_array_equal(routed1.read(np.uint32), routed2.read(np.uint32))
    want_ids, want_probs = O.select_experts(logits.download(np.float32).reshape(tokens, E), k)
    np.testing.assert_array_equal(ids, want_ids)
    ref = O.experts_reference(39, hidden, ffn, g, u, d, x, ids, p, resid, gb, ub, db, activation=0, up_one=True)
    assert rel_l2(routed1.read(np.float32).reshape(-1, hidden), ref["down"]) < MX_TILE_BAR
