"""CPU tests that pin the C oracle (oracle/oco_oracle.c) before it is trusted.

Each check is chosen so a plausible mistake (dropped term, wrong shift or
index, transposed operand) fails: the reference's own packers as known
answers, closed forms, invariants and brute force on tiny inputs.
"""
import itertools
import math
import os
import subprocess

import numpy as np
import pytest

import oracle as O
import packers as P

FORMATS = [P.F32, P.F16, P.BF16, P.Q4_0, P.Q4_1, P.Q8_0, P.Q4_K, P.Q5_K, P.Q6_K]


@pytest.fixture(scope="module", autouse=True)
def built():
    O.build()


@pytest.mark.parametrize("fmt", FORMATS)
def test_dequant_reproduces_reference_packer(fmt):
    """decode(pack(codes)) == recorded coefficients (matrix_precision.rs:145-287)."""
    k, n = 512, 33
    data, coeffs = P.dense_weights(fmt, n, k)
    elems, nbytes = O.block_layout(fmt)
    assert len(data) == n * k // elems * nbytes
    got = O.dequant(fmt, np.frombuffer(data, np.uint8), n * k)
    want = np.array([c for c, _ in coeffs], np.float64)
    # Coefficients are exact in f64; decode rounds at most once, to nearest.
    np.testing.assert_array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("fmt", FORMATS + [O.MXFP4])
def test_embed_rows_from_reference_packer(fmt):
    """embed (weights.metal:90-109): row ids[r] of the packed tensor equals
    the packer's recorded coefficients rounded to bf16 (numpy rounding of the
    exact values), ids >= vocabulary splice the feature rows, and ids past
    them give NaN rows; native BF16 rows keep their stored bits, so a NaN
    payload that a float round trip would quieten (0x7f81 -> 0x7fc1)
    survives."""
    k, n = 512, 33
    if fmt == O.MXFP4:
        data, values = P.mxfp4_expert_weights(k, n, salt=3, experts=1)
        w = np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:]
        coeffs = np.asarray(values, np.float64).reshape(n, k)
    else:
        data, cs = P.dense_weights(fmt, n, k)
        w = np.frombuffer(data, np.uint8).copy()
        coeffs = np.array([c for c, _ in cs], np.float64).reshape(n, k)
        if fmt == P.BF16:
            w.view(np.uint16)[3 * k + 5] = 0x7f81
            coeffs[3, 5] = np.nan
    feats = O.f32_to_bf16(np.random.default_rng(1).normal(size=(2, k)).astype(np.float32))
    ids = np.array([0, 3, n - 1, n, n + 1, n + 2, 7, 3], np.uint32)
    got = O.embed(fmt, w, k, n, ids, feats)
    for r, i in enumerate(ids):
        if i < n:
            want = coeffs[i].astype(np.float32)
            rounded = ((want.view(np.uint32).astype(np.uint64) + 0x7FFF + ((want.view(np.uint32) >> 16) & 1)) >> 16)
            finite = np.isfinite(want)
            # as values: the MXFP4 packer records code 8 (-0) as +0
            np.testing.assert_array_equal(O.bf16_to_f32(got[r])[finite],
                                          O.bf16_to_f32(rounded.astype(np.uint16))[finite])
        elif i - n < 2:
            np.testing.assert_array_equal(got[r], feats[i - n])
        else:
            assert (got[r] == 0x7fc0).all()
    if fmt == P.BF16:
        assert got[1][5] == 0x7f81
    assert (O.embed(fmt, w, k, n, ids[:3]) == got[:3]).all()


def test_mxfp4_decode_reproduces_reference_packer():
    """mxfp4.rs:46-81 at the reference's K=2880, with the unaligned start."""
    k, n = 2880, 5
    data, coeffs = P.mxfp4_decode_weights(k, n)
    w = np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:]
    got = O.dequant(O.MXFP4, w, 4 * n * k)
    np.testing.assert_array_equal(got.astype(np.float64), coeffs)


def test_mxfp4_expert_packer():
    data, values = P.mxfp4_expert_weights(96, 3, salt=5, experts=2)
    got = O.dequant(O.MXFP4, np.frombuffer(data, np.uint8)[P.WEIGHT_OFFSET:], values.size)
    np.testing.assert_array_equal(got, values)


def test_committed_golden_fixtures_match_generators():
    here = os.path.join(os.path.dirname(__file__), "golden")
    for fmt in FORMATS:
        f = np.load(os.path.join(here, f"dense_{fmt}.npz"))
        data, coeffs = P.dense_weights(fmt, int(f["n"]), int(f["k"]))
        np.testing.assert_array_equal(np.frombuffer(data, np.uint8), f["bytes"])
        np.testing.assert_array_equal(np.array([c for c, _ in coeffs]), f["coefficients"])
        np.testing.assert_array_equal(O.dequant(fmt, f["bytes"], f["coefficients"].size),
                                      f["coefficients"].astype(np.float32))


def test_fp16_conversions_special_cases():
    L = O.lib()
    assert L.oo_fp16(0x0001) == 2.0 ** -24            # smallest subnormal
    assert L.oo_fp16(0x03FF) == 1023 * 2.0 ** -24     # largest subnormal
    assert L.oo_fp16(0x0400) == 2.0 ** -14
    assert L.oo_fp16(0x3C00) == 1.0
    assert L.oo_fp16(0xC000) == -2.0
    assert L.oo_fp16(0x7BFF) == 65504.0
    assert math.isinf(L.oo_fp16(0x7C00)) and L.oo_fp16(0xFC00) < 0
    assert math.isnan(L.oo_fp16(0x7E00))
    # every half converts like numpy's IEEE half
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([L.oo_fp16(int(b)) for b in bits[::97]], np.float32)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref[::97]))
    ok = ~np.isnan(ref[::97])
    np.testing.assert_array_equal(got[ok], ref[::97][ok])
    # f32 -> f16 round to nearest even agrees with numpy over random values and ties
    xs = np.concatenate([np.random.default_rng(1).normal(0, 3, 2000).astype(np.float32),
                         np.array([2.0 ** -25, 3 * 2.0 ** -25, 65519.0, 65520.0, 1 + 2.0 ** -11],
                                  np.float32)])
    for x in xs:
        assert L.oo_f32_to_f16(float(x)) == int(np.float16(x).view(np.uint16)), x


def test_bf16_rounding_ties_to_even():
    L = O.lib()
    assert L.oo_f32_to_bf16(1.0) == 0x3F80
    assert L.oo_f32_to_bf16(float(np.uint32(0x3F808000).view(np.float32))) == 0x3F80  # tie -> even
    assert L.oo_f32_to_bf16(float(np.uint32(0x3F818000).view(np.float32))) == 0x3F82  # tie -> even
    assert L.oo_f32_to_bf16(float(np.uint32(0x3F808001).view(np.float32))) == 0x3F81
    x = np.random.default_rng(2).normal(0, 1, 1000).astype(np.float32)
    np.testing.assert_array_equal(O.f32_to_bf16(x), [L.oo_f32_to_bf16(float(v)) for v in x])


def _q8_block(d_bits: int, codes) -> bytes:
    return int(d_bits).to_bytes(2, "little") + bytes(np.array(codes, np.int8).view(np.uint8))


def test_special_scales():
    # Q8_0 with subnormal, inf and nan scales
    for d_bits, d in [(0x0001, 2.0 ** -24), (0x0200, 512 * 2.0 ** -24), (0x3C00, 1.0)]:
        codes = np.arange(-16, 16)
        got = O.dequant(O.Q8_0, np.frombuffer(_q8_block(d_bits, codes), np.uint8), 32)
        np.testing.assert_array_equal(got, (codes * d).astype(np.float32))
    got = O.dequant(O.Q8_0, np.frombuffer(_q8_block(0x7C00, [1] * 32), np.uint8), 32)
    assert np.all(np.isinf(got))
    got = O.dequant(O.Q8_0, np.frombuffer(_q8_block(0x7C00, [0] * 32), np.uint8), 32)
    assert np.all(np.isnan(got))  # 0 * inf
    # MXFP4: E8M0 0 -> 2^-127, 255 -> NaN, 127 -> 1
    for e, scale in [(127, 1.0), (0, 2.0 ** -127), (118, 2.0 ** -9), (254, 2.0 ** 127)]:
        codes = np.arange(16, dtype=np.uint8)
        blk = bytes([e]) + bytes(codes | (codes[::-1] << 4))
        got = O.dequant(O.MXFP4, np.frombuffer(blk, np.uint8), 32).astype(np.float64)
        e2m1 = np.array(P.HALVES, np.float64) * 0.5
        want = np.concatenate([e2m1[codes], e2m1[codes[::-1]]]) * scale
        with np.errstate(over="ignore"):
            np.testing.assert_array_equal(got, want.astype(np.float32))
    blk = bytes([255]) + bytes(16)
    assert np.all(np.isnan(O.dequant(O.MXFP4, np.frombuffer(blk, np.uint8), 32)))
    # Q6_K: code 0 -> -32 * sc * d; scale -128
    blk = bytearray(210)
    blk[192:208] = bytes([0x80] * 16)  # int8 -128
    blk[208:210] = (0x3C00).to_bytes(2, "little")
    got = O.dequant(O.Q6_K, np.frombuffer(bytes(blk), np.uint8), 256)
    np.testing.assert_array_equal(got, np.full(256, 4096.0, np.float32))


def test_q4k_min_and_scale_unpacking_against_brute_force():
    """Every (sub-block, scale, min) pattern of the 12-byte 6-bit table."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        packed = [0] * 12
        for i in range(8):  # the packing the reference's encoder uses
            if i < 4:
                packed[i] = int(sc[i]); packed[i + 4] = int(mn[i])
            else:
                packed[i + 4] = (int(sc[i]) & 15) | ((int(mn[i]) & 15) << 4)
                packed[i - 4] |= (int(sc[i]) >> 4) << 6
                packed[i] |= (int(mn[i]) >> 4) << 6
        q = rng.integers(0, 16, 256)
        qs = bytearray(128)
        for j in range(256):
            qs[j // 64 * 32 + j % 32] |= int(q[j]) << (j % 64 // 32 * 4)
        blk = (0x3C00).to_bytes(2, "little") + (0x3800).to_bytes(2, "little") + bytes(packed) + qs
        got = O.dequant(O.Q4_K, np.frombuffer(blk, np.uint8), 256)
        want = np.array([sc[j // 32] * q[j] - 0.5 * mn[j // 32] for j in range(256)], np.float32)
        np.testing.assert_array_equal(got, want)


def _matrix(k, n, m=1, route_major=0, routes=1, experts=1, has_bias=0):
    return O.Matrix(k, n, m, route_major, routes, experts, has_bias)


def test_matvec_exact_integer_answers():
    """All-ones weights with x=1 and x=2 give K and 2K (compute/tests.rs:40-80)."""
    k, n = 512, 7
    w = np.ones(n * k, np.float32).view(np.uint8)
    for xv in (1.0, 2.0):
        x = np.full(k, xv, np.float32)
        y = O.matvec_f32(O.F32, w, x, _matrix(k, n))
        np.testing.assert_array_equal(y, np.full(n, k * xv, np.float32))
        y64, mag = O.matvec_f64(O.F32, w, x, _matrix(k, n))
        np.testing.assert_array_equal(y64, np.full(n, k * xv))
        np.testing.assert_array_equal(mag, np.full(n, k * xv))


@pytest.mark.parametrize("fmt", [P.Q8_0, P.Q4_K, P.Q6_K, P.Q5_K, P.Q4_0, P.Q4_1, P.BF16])
def test_matvec_oracle_against_numpy_fp64(fmt):
    """Dense packer weights times bf16 inputs: fp64 oracle == numpy fp64 of the
    recorded coefficients; fp32 oracle within the reference's roundoff bound."""
    k, n = 512, 33
    data, coeffs = P.dense_weights(fmt, n, k)
    W = np.array([c for c, _ in coeffs]).reshape(n, k)
    A = np.array([a for _, a in coeffs]).reshape(n, k)
    xb = P.dense_input(2, k)
    w = np.frombuffer(data, np.uint8)
    for t in range(2):
        x = xb[t]
        xf = O.bf16_to_f32(x).astype(np.float64)
        y64, mag = O.matvec_f64(fmt, w, x, _matrix(k, n))
        assert np.all(np.abs(y64 - W @ xf) <= 1e-12 * (np.abs(W) @ np.abs(xf)))
        y32 = O.matvec_f32(fmt, w, x, _matrix(k, n))
        bound = O.roundoff_bound(y64, A @ np.abs(xf), k, False)
        assert np.all(np.abs(y32 - y64) <= bound)


def test_relu_sqr_input_closed_form():
    """max(x, 0)^2 in f32; NaN reads as 0 and -0 as 0; squares overflow to
    Inf as f32 products do; bf16 bits are widened first."""
    x = np.array([-2.0, -0.0, 0.0, 1.5, 3.0, np.nan, np.inf, -np.inf, 1e20, 2.0 ** -80], np.float32)
    want = np.array([0, 0, 0, 2.25, 9, 0, np.inf, 0, np.inf, 0], np.float32)
    got = O.relu_sqr_input(x)
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, want)
    assert not np.any(np.signbit(got))
    bits = np.array([0xBF80, 0x4000, 0x7FC0, 0x3F81], np.uint16)  # -1, 2, NaN, 1.0078125
    np.testing.assert_array_equal(O.relu_sqr_input(bits), np.float32([0, 4, 0, np.float32(1.0078125) ** 2]))


def test_matvec_linearity_and_bias_rules():
    k, n = 256, 5
    data, _ = P.dense_weights(P.Q4_K, n, k)
    w = np.frombuffer(data, np.uint8)
    rng = np.random.default_rng(4)
    x1 = rng.normal(size=k).astype(np.float32)
    x2 = rng.normal(size=k).astype(np.float32)
    y1, _ = O.matvec_f64(O.Q4_K, w, x1, _matrix(k, n))
    y2, _ = O.matvec_f64(O.Q4_K, w, x2, _matrix(k, n))
    y12, _ = O.matvec_f64(O.Q4_K, w, (x1 + 2 * x2).astype(np.float32), _matrix(k, n))
    np.testing.assert_allclose(y12, y1 + 2 * y2, rtol=1e-6, atol=1e-9)
    bias = rng.normal(size=n).astype(np.float32)
    yb, _ = O.matvec_f64(O.Q4_K, w, x1, _matrix(k, n, has_bias=1), bias=bias)
    np.testing.assert_array_equal(yb - y1, O.bf16_to_f32(O.f32_to_bf16(bias)))
    yb2, _ = O.matvec_f64(O.Q4_K, w, x1, _matrix(k, n, has_bias=2), bias=bias)
    np.testing.assert_array_equal(yb2 - y1, O.bf16_to_f32(O.f32_to_bf16(bias + 1)))


def test_routed_indexing():
    """expert = ids[route]; input = route/routes unless route_major (vector.metal:76-78)."""
    k, n, E = 64, 3, 4
    w = np.random.default_rng(5).normal(size=E * n * k).astype(np.float32)
    x = np.random.default_rng(6).normal(size=(2, k)).astype(np.float32)
    ids = np.array([3, 0, 2, 1], np.uint32)
    y, _ = O.matvec_f64(O.F32, w.view(np.uint8), x, _matrix(k, n, m=4, routes=2, experts=E), ids=ids)
    W = w.reshape(E, n, k).astype(np.float64)
    for r in range(4):
        np.testing.assert_allclose(y[r * n:(r + 1) * n], W[ids[r]] @ x[r // 2], rtol=1e-12)
    xr = np.random.default_rng(7).normal(size=(4, k)).astype(np.float32)
    y, _ = O.matvec_f64(O.F32, w.view(np.uint8), xr, _matrix(k, n, m=4, route_major=1, routes=2,
                                                              experts=E), ids=ids)
    for r in range(4):
        np.testing.assert_allclose(y[r * n:(r + 1) * n], W[ids[r]] @ xr[r], rtol=1e-12)


def test_select_experts_known_answer_and_brute_force():
    ids, probs = O.select_experts(P.logits_selecting([3, 0, 2, 1])[None], 4)
    assert list(ids[0]) == [3, 0, 2, 1]
    e = np.exp(np.array([0.0, -1.0, -2.0, -3.0], np.float32))
    want = O.bf16_to_f32(O.f32_to_bf16((e / e.sum()).astype(np.float32)))
    np.testing.assert_allclose(probs[0], want, rtol=0, atol=2 ** -8)
    rng = np.random.default_rng(8)
    for experts, k in [(32, 4), (128, 8), (5, 5)]:
        logits = rng.normal(size=(20, experts)).astype(np.float32)
        ids, probs = O.select_experts(logits, k)
        for t in range(20):
            best = max(itertools.combinations(range(experts), k) if experts <= 8 else [None],
                       key=lambda c: -1 if c is None else sum(logits[t][list(c)]))
            order = np.argsort(-logits[t], kind="stable")[:k]
            assert list(ids[t]) == list(order)
            if best is not None:
                assert set(best) == set(order)
            c = O.bf16_to_f32(O.f32_to_bf16(logits[t][order]))
            ex = np.exp(c.astype(np.float64) - c[0])
            np.testing.assert_allclose(probs[t], ex / ex.sum(), rtol=2 ** -7)
            assert abs(probs[t].sum() - 1) < 0.02


def test_select_experts_ties_and_non_finite():
    logits = np.zeros((1, 32), np.float32)
    ids, probs = O.select_experts(logits, 4)
    assert list(ids[0]) == [0, 1, 2, 3]
    np.testing.assert_array_equal(probs[0], np.full(4, 0.25, np.float32))
    logits[0, 7] = np.nan
    ids, probs = O.select_experts(logits, 4)
    assert list(ids[0]) == [0, 1, 2, 3] and np.all(np.isnan(probs))
    logits[0, 7] = np.inf
    ids, probs = O.select_experts(logits, 4)
    assert np.all(ids[0] < 32) and np.all(np.isnan(probs))


def test_swiglu_clipped_closed_form():
    for g, u in [(0.5, 1.0), (-3.0, 2.0), (9.0, 10.0), (7.0, -7.0), (-30.0, 1.0), (0.0, 5.0)]:
        gc, uc = min(g, 7.0), min(max(u, -6.0), 8.0)
        want = gc / (1 + math.exp(-1.702 * gc)) * uc
        assert abs(O.swiglu_clipped(g, u) - want) <= 1e-6 * max(1.0, abs(want))
    assert math.isnan(O.swiglu_clipped(float("inf"), 1.0))
    assert math.isnan(O.swiglu_clipped(1.0, float("nan")))


def test_layer_activations_follow_the_nonfinite_rule():
    """The fp64 layer activations agree with the C oracle's f32 clipped
    SwiGLU on finite inputs (including ones far past the clipping points and
    where exp overflows), and give NaN for every non-finite gate or up, as
    projections.metal:5-8 and elementwise.metal:76-80 do -- without numpy
    overflow warnings."""
    import warnings
    rng = np.random.default_rng(4)
    g = np.concatenate([rng.normal(0, 3, 200), [1e30, -1e30, 500.0, -500.0, 7.0, -6.0, 0.0]])
    u = np.concatenate([rng.normal(0, 5, 200), [1.0, 2.0, -1e30, 1e30, 8.5, -6.5, 3.0]])
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        got = O.swiglu_clipped_f64(g, u)
        silu = O.swiglu_f64(g, u)
    want = np.array([O.swiglu_clipped(float(a), float(b)) for a, b in zip(g, u)], np.float64)
    assert np.all(np.abs(got - want) <= 1e-6 * np.maximum(1.0, np.abs(want)))
    # silu(g) u: closed form where exp does not overflow, 0 * u and g * u at the tails
    mid = np.abs(g) < 50
    gm, um = g[mid], u[mid]
    np.testing.assert_allclose(silu[mid], gm / (1 + np.exp(-gm)) * um, rtol=1e-12, atol=1e-300)
    assert silu[-6] == 0.0 * u[-6] and silu[-7] == g[-7] * u[-7]
    inf, nan = np.inf, np.nan
    gs = np.array([inf, -inf, nan, 1.0, 1.0, 1.0, inf])
    us = np.array([1.0, 1.0, 1.0, inf, -inf, nan, inf])
    for fn in (O.swiglu_clipped_f64, O.swiglu_f64):
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            assert np.all(np.isnan(fn(gs, us)))
    assert all(math.isnan(O.swiglu_clipped(float(a), float(b))) for a, b in zip(gs, us))


@pytest.mark.parametrize("batch,experts,tile", [(17, 32, 64), (257, 32, 64), (512, 128, 16), (1, 32, 64)])
def test_route_plan_brute_force(batch, experts, tile):
    if experts == 32:
        ids = P.expert_ids(batch) if batch > 1 else np.array([3, 0, 2, 1], np.uint32)
    else:
        ids = np.random.default_rng(9).integers(0, experts, batch * 8).astype(np.uint32)
    routes = ids.size
    plan, tiles = O.route_plan(ids, experts, tile, 11, 7)
    assert plan.size == O.route_plan_words(routes, experts)
    assert list(plan[:6]) == [11, tiles, 1, 7, tiles, 1]
    grouped = 6 + 2 * ((routes + 15) // 16 + experts)
    sorted_ = grouped + experts * (routes + 1)
    seen = np.zeros(routes, bool)
    offset = 0
    expect_tiles = []
    for e in range(experts):
        base = grouped + e * (routes + 1)
        count = plan[base]
        lst = plan[base + 1:base + 1 + count]
        assert list(lst) == list(np.nonzero(ids == e)[0])  # route order preserved
        assert plan[sorted_ + e] == offset
        for i, r in enumerate(lst):
            assert plan[sorted_ + experts + r] == offset + i
            seen[r] = True
        expect_tiles += [(e, b) for b in range(0, count, tile)]
        offset += count
    assert seen.all()
    assert [(plan[6 + 2 * t], plan[7 + 2 * t]) for t in range(tiles)] == expect_tiles
    assert tiles <= (routes + 15) // 16 + experts


def test_moe_sum_rounding_points():
    hidden, batch, k = 3, 2, 4
    routes = O.f32_to_bf16(np.arange(batch * k * hidden, dtype=np.float32).reshape(-1, hidden) / 7)
    probs = np.array([[0.5, 0.25, 0.125, 0.125], [1, 0, 0, 0]], np.float32)
    out = O.f32_to_bf16(np.full((batch, hidden), 100.0, np.float32))
    got = O.moe_sum(routes, probs, out, k)
    r = O.bf16_to_f32(routes).reshape(batch, k, hidden)
    for t in range(batch):
        s = np.float32(0)
        for j in range(k):
            s = np.float32(s + r[t, j] * probs[t, j])
        want = O.f32_to_bf16(np.float32(100.0) + O.bf16_to_f32(O.f32_to_bf16(s)))
        np.testing.assert_array_equal(got[t], want)


def test_oracle_under_sanitizers():
    """The oracle's C runs clean under ASan/UBSan on a self-test driver."""
    here = os.path.dirname(O.__file__)
    r = subprocess.run(["make", "-s", "-B", "-C", here, "oracle_asan"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([os.path.join(here, "oracle_asan")], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr


def test_argmax_reference_known_answers():
    """The reference's own cases (numerics.rs:14-69)."""
    import argmax_cases as A
    for bits, want in A.cases():
        assert O.argmax_f32(A.logits(bits)) == want
    assert O.argmax_f32(np.zeros(0, np.float32)) == A.NONE


def test_argmax_brute_force_finite():
    rng = np.random.default_rng(3)
    for n in (1, 5, 1000, 151936):
        x = rng.normal(size=n).astype(np.float32)
        assert O.argmax_f32(x) == int(np.argmax(x))
        x = np.round(x * 2).astype(np.float32)  # many ties: numpy also keeps the first
        assert O.argmax_f32(x) == int(np.argmax(x))


def test_norm_closed_forms():
    n = 256
    # a constant row c normalises to c / sqrt(c^2 + eps) = 1 (eps -> 0)
    x = O.f32_to_bf16(np.full((1, n), 3.0, np.float32)).reshape(1, n)
    y, exact = O.norm(x, np.ones(n, np.float32), 0.0, True)
    assert np.allclose(exact, 1.0, rtol=0, atol=1e-12) and np.all(O.bf16_to_f32(y) == 1.0)
    # numpy fp64 restatement of the same formula on random rows, both rounding modes
    rng = np.random.default_rng(4)
    xr = O.f32_to_bf16(rng.normal(size=(3, n)).astype(np.float32)).reshape(3, n)
    w = rng.normal(size=n).astype(np.float32)
    X = O.bf16_to_f32(xr).astype(np.float64).reshape(3, n)
    inv = 1.0 / np.sqrt((X * X).mean(axis=1, keepdims=True) + 1e-5)
    y1, e1 = O.norm(xr, w, 1e-5, True)
    assert np.allclose(e1, X * inv * w.astype(np.float64), rtol=1e-6, atol=0)
    y0, e0 = O.norm(xr, w, 1e-5, False)
    want0 = O.bf16_round((X * inv).astype(np.float32)).astype(np.float64) * O.bf16_round(w).astype(np.float64)
    assert np.allclose(e0, want0, rtol=1e-6, atol=0)
    # scale invariance: 4x the row gives the same normalised row (powers of two are exact in bf16)
    y4, _ = O.norm(O.f32_to_bf16(X.astype(np.float32) * 4).reshape(3, n), w, 0.0, True)
    yz, _ = O.norm(xr, w, 0.0, True)
    assert np.array_equal(y4, yz)


def test_add_norm_is_add_then_norm():
    rng = np.random.default_rng(5)
    n = 96
    x = O.f32_to_bf16(rng.normal(size=(2, n)).astype(np.float32)).reshape(2, n)
    y = O.f32_to_bf16(rng.normal(size=(2, n)).astype(np.float32)).reshape(2, n)
    w = rng.normal(size=n).astype(np.float32)
    xs, out, _ = O.add_norm(x, y, w, 1e-6, True)
    want_x = O.f32_to_bf16((O.bf16_to_f32(x) + O.bf16_to_f32(y)).astype(np.float32)).reshape(2, n)
    assert np.array_equal(xs, want_x)
    assert np.array_equal(out, O.norm(want_x, w, 1e-6, True)[0])


def test_q4_row_gain_closed_form():
    """The scaled Q4 tiles' gain (q4_tile.metal:44-49): 2^(141 - e) for the
    peak's f32 exponent e, clamped to 2^+-120, 1 for a zero row; x * gain
    then has its peak in [2^14, 2^15)."""
    assert O.q4_row_gain(0.0) == 1.0
    assert O.q4_row_gain(1.0) == 2.0 ** 14
    assert O.q4_row_gain(1.5) == 2.0 ** 14
    assert O.q4_row_gain(2.0 ** 14) == 1.0
    assert O.q4_row_gain(32767.0) == 1.0
    assert O.q4_row_gain(2.0 ** 15) == 0.5
    assert O.q4_row_gain(1e30) == 2.0 ** (141 - (127 + 99))
    assert O.q4_row_gain(1e-38) == 2.0 ** 120  # exponent 0..: clamped
    for peak in [3e-5, 0.7, 123.0, 6e4, 2.5e9]:
        assert 2.0 ** 14 <= peak * O.q4_row_gain(peak) < 2.0 ** 15
