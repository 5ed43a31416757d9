"""ctypes view of the C oracle (oracle/oco_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
as the checker, and by bench.py's ``cpu_baseline`` leg.  The product library
(``oco_amd``) never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboco_oracle.so")

F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16, MXFP4 = 0, 1, 2, 3, 8, 12, 13, 14, 30, 39
DT_F32, DT_BF16, DT_F16 = 0, 1, 2
FORMATS = {"f32": F32, "f16": F16, "q4_0": Q4_0, "q4_1": Q4_1, "q8_0": Q8_0, "q4_k": Q4_K,
           "q5_k": Q5_K, "q6_k": Q6_K, "bf16": BF16, "mxfp4": MXFP4}


class Matrix(ctypes.Structure):
    """shaders/matrix/weights.metal:87-89"""
    _fields_ = [(name, ctypes.c_uint32) for name in
                ("k", "n", "m", "route_major", "routes", "experts", "has_bias")]


def build() -> None:
    subprocess.run(["make", "-s", "-B", "-C", HERE, "liboco_oracle.so"], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        vp, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
        L.oo_block_layout.argtypes = [u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]
        L.oo_fp16.argtypes = [ctypes.c_uint16]
        L.oo_fp16.restype = ctypes.c_float
        L.oo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oo_f32_to_bf16.restype = ctypes.c_uint16
        L.oo_f32_to_f16.argtypes = [ctypes.c_float]
        L.oo_f32_to_f16.restype = ctypes.c_uint16
        L.oo_dequant.argtypes = [u32, vp, u64, vp]
        L.oo_embed.argtypes = [u32, vp, u32, u32, vp, u32, vp, u32, vp]
        L.oo_matvec_f64.argtypes = [u32, vp, vp, i32, vp, vp, ctypes.POINTER(Matrix), vp, vp]
        L.oo_matvec_f32.argtypes = [u32, vp, vp, i32, vp, vp, ctypes.POINTER(Matrix), vp, i32, i32]
        L.oo_select_experts.argtypes = [vp, u32, u32, vp, vp]
        L.oo_swiglu_clipped.argtypes = [ctypes.c_float, ctypes.c_float]
        L.oo_swiglu_clipped.restype = ctypes.c_float
        L.oo_route_plan_words.argtypes = [u32, u32]
        L.oo_route_plan_words.restype = u64
        L.oo_route_plan.argtypes = [vp, u32, u32, u32, u32, u32, vp]
        L.oo_route_plan.restype = u64
        L.oo_moe_sum.argtypes = [vp, vp, vp, u32, u32, u32]
        L.oo_argmax_f32.argtypes = [vp, u32]
        L.oo_argmax_f32.restype = u32
        L.oo_norm.argtypes = [vp, vp, vp, vp, u32, u32, ctypes.c_float, i32]
        L.oo_add_norm.argtypes = [vp, vp, vp, vp, vp, u32, u32, ctypes.c_float, i32]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def block_layout(fmt: int) -> tuple[int, int]:
    e, b = ctypes.c_uint32(), ctypes.c_uint32()
    if lib().oo_block_layout(fmt, ctypes.byref(e), ctypes.byref(b)):
        raise ValueError(f"unknown format {fmt}")
    return e.value, b.value


def dequant(fmt: int, w: np.ndarray, count: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(count, np.float32)
    rc = lib().oo_dequant(fmt, _p(w), count, _p(out))
    if rc:
        raise ValueError(f"oo_dequant failed: {rc}")
    return out


def embed(fmt: int, w: np.ndarray, k: int, vocab: int, ids, features=None) -> np.ndarray:
    """bf16 token rows (weights.metal:90-109) of a [vocab][k] GGUF tensor."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty((ids.size, k), np.uint16)
    feats = None if features is None else np.ascontiguousarray(features, np.uint16)
    nf = 0 if feats is None else feats.size // k
    rc = lib().oo_embed(fmt, _p(w), k, vocab, _p(ids), ids.size, _p(feats) if feats is not None else None, nf,
                        _p(out))
    if rc:
        raise ValueError(f"oo_embed failed: {rc}")
    return out


def _x_dtype(x: np.ndarray) -> int:
    if x.dtype == np.float32:
        return DT_F32
    if x.dtype == np.uint16:  # bf16 bits
        return DT_BF16
    raise TypeError(x.dtype)


def relu_sqr_input(x: np.ndarray) -> np.ndarray:
    """The relu² input transform of the vector kernels, as f32: max(v, 0)
    squared in f32 (weights.metal:22-24, vector.metal:120-123,
    q8-dot.metal:12-15); x is f32 or bf16 bits.  A NaN element becomes 0
    (fmax keeps the non-NaN operand)."""
    v = bf16_to_f32(x) if x.dtype == np.uint16 else np.asarray(x, np.float32)
    r = np.fmax(v, np.float32(0))
    with np.errstate(over="ignore"):
        return (r * r).astype(np.float32)


def matvec_f64(fmt, w, x, p: Matrix, bias=None, ids=None, xdt=None):
    """fp64 y (routes*n) and magnitude sum|w x| + |b| per output."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x)
    y = np.empty(p.m * p.n, np.float64)
    mag = np.empty(p.m * p.n, np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    i = None if ids is None else np.ascontiguousarray(ids, np.uint32)
    rc = lib().oo_matvec_f64(fmt, _p(w), _p(x), _x_dtype(x) if xdt is None else xdt, _p(b), _p(i),
                             ctypes.byref(p), _p(y), _p(mag))
    if rc:
        raise ValueError(rc)
    return y, mag


def matvec_f32(fmt, w, x, p: Matrix, bias=None, ids=None, y_bf16=False, threads=1):
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x)
    f32_out = (not y_bf16) or (p.experts > 1 and not p.route_major)
    y = np.empty(p.m * p.n, np.float32 if f32_out else np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    i = None if ids is None else np.ascontiguousarray(ids, np.uint32)
    rc = lib().oo_matvec_f32(fmt, _p(w), _p(x), _x_dtype(x), _p(b), _p(i), ctypes.byref(p), _p(y),
                             DT_F32 if not y_bf16 else DT_BF16, threads)
    if rc:
        raise ValueError(rc)
    return y


def select_experts(logits: np.ndarray, k: int):
    """Per-token top-k with softmax over the selected (routing.metal:71-94)."""
    logits = np.ascontiguousarray(logits, np.float32)
    tokens, experts = logits.shape
    ids = np.empty((tokens, k), np.uint32)
    probs = np.empty((tokens, k), np.float32)
    for t in range(tokens):
        row = np.ascontiguousarray(logits[t])
        rc = lib().oo_select_experts(_p(row), experts, k, _p(ids[t]), _p(probs[t]))
        if rc:
            raise ValueError(rc)
    return ids, probs


def swiglu_clipped(g: float, u: float) -> float:
    return lib().oo_swiglu_clipped(g, u)


def route_plan(ids: np.ndarray, experts: int, tile_rows: int, up_tiles: int, down_tiles: int):
    ids = np.ascontiguousarray(ids, np.uint32).ravel()
    words = lib().oo_route_plan_words(ids.size, experts)
    plan = np.zeros(words, np.uint32)
    tiles = lib().oo_route_plan(_p(ids), ids.size, experts, tile_rows, up_tiles, down_tiles, _p(plan))
    if tiles == 2 ** 64 - 1:
        raise ValueError("tile_rows must be >= 16")
    return plan, int(tiles)


def route_plan_words(routes: int, experts: int) -> int:
    return int(lib().oo_route_plan_words(routes, experts))


def moe_sum(routes_bf16: np.ndarray, probs: np.ndarray, out_bf16: np.ndarray, k: int) -> np.ndarray:
    out = np.array(out_bf16, np.uint16, copy=True)
    batch, hidden = out.shape
    r = np.ascontiguousarray(routes_bf16, np.uint16)
    p = np.ascontiguousarray(probs, np.float32)
    lib().oo_moe_sum(_p(r), _p(p), _p(out), hidden, batch, k)
    return out


# --- scalar conversions (vectorised in numpy, exactly as the C helpers) ------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round to nearest even; NaN stays quiet NaN."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def relative_l2(actual: np.ndarray, expected: np.ndarray) -> float:
    a = np.asarray(actual, np.float64).ravel()
    e = np.asarray(expected, np.float64).ravel()
    den = np.linalg.norm(e)
    return float(np.linalg.norm(a - e) / (den if den > 0 else 1.0))


def roundoff_bound(expected, magnitude, k: int, stored_bf16: bool):
    """gamma_{2k+8} * sum|w x| plus bf16 storage (matrix_precision.rs:136-142)."""
    unit = 2.0 ** -24
    ops = 2 * k + 8
    gamma = ops * unit / (1 - ops * unit)
    storage = 2.0 ** -8 if stored_bf16 else 0.0
    return (1 + storage) * gamma * np.asarray(magnitude) + storage * np.abs(np.asarray(expected))


# --- composed references for the expert path and prefill ----------------------

def expert_rows(fmt: int, w: np.ndarray, expert: int, n: int, k: int) -> np.ndarray:
    """Rows of one expert of a bank [experts][n][k rows of GGUF blocks], fp64."""
    rb = k // block_layout(fmt)[0] * block_layout(fmt)[1]
    sl = np.ascontiguousarray(np.asarray(w, np.uint8)[expert * n * rb:(expert + 1) * n * rb])
    return dequant(fmt, sl, n * k).astype(np.float64).reshape(n, k)


def bf16_round(x) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(np.asarray(x, np.float32))).astype(np.float64)


def _nonfinite_to_nan(g, u, act):
    """The activations' rule for invalid operands: any non-finite gate or up
    value gives NaN (projections.metal:5-8, routing.metal:53-58,
    elementwise.metal:76-80), checked before any clipping."""
    bad = ~(np.isfinite(g) & np.isfinite(u))
    return np.where(bad, np.nan, act)


def swiglu_clipped_f64(g, u):
    """projections.metal:4-13 in fp64: sigmoid(1.702 g') g' u', g' = min(g, 7),
    u' = clamp(u, -6, 8); NaN for a non-finite g or u."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        gc = np.minimum(np.where(np.isfinite(g), g, 0.0), 7.0)
        uc = np.clip(np.where(np.isfinite(u), u, 0.0), -6.0, 8.0)
        act = gc / (1.0 + np.exp(-1.702 * gc)) * uc
    return _nonfinite_to_nan(g, u, act)


def swiglu_f64(g, u):
    """silu(g) * u (elementwise.metal:70-88 without its bf16 storage); NaN
    for a non-finite g or u."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        gf = np.where(np.isfinite(g), g, 0.0)
        # sigmoid from exp(-|g|), as the kernels take it, so large |g| does not overflow
        e = np.exp(-np.abs(gf))
        sig = np.where(gf < 0, e, 1.0) / (1.0 + e)
        act = sig * gf * np.where(np.isfinite(u), u, 0.0)
    return _nonfinite_to_nan(g, u, act)


def experts_reference(fmt, hidden, ffn, gate, up, down, x, ids, probs, residual_bf16,
                      gate_bias=None, up_bias=None, down_bias=None, activation=0, up_one=True,
                      act_override=None):
    """Bindings::experts (feed_forward.rs:107-275) in fp64 after routing:
    per route r of token t = r / k with expert e = ids[r]:
      g = gate_e . x_t + bf16(gate_bias), u = up_e . x_t + bf16(up_bias + 1)
      a = act(g, u); y_r = down_e . a + bf16(down_bias)
    out[t] = bf16(residual + bf16(sum_r bf16(y_r) p_r))   (routing.metal:157-168).
    `act_override` (routes x ffn) feeds the down projection with given values
    (the GPU's own f32 activations), as the reference's test does (mxfp4.rs:458-470)."""
    x = np.asarray(x)
    xf = bf16_to_f32(x).astype(np.float64) if x.dtype == np.uint16 else x.astype(np.float64)
    tokens = xf.shape[0]
    ids = np.asarray(ids, np.uint32).reshape(-1)
    k = ids.size // tokens
    routes = ids.size
    act = np.zeros((routes, ffn))
    upv = np.zeros((routes, ffn))
    gat = np.zeros((routes, ffn))
    mag_up = np.zeros((routes, ffn))
    y = np.zeros((routes, hidden))
    mag_y = np.zeros((routes, hidden))
    for e in np.unique(ids):  # the routes of one expert as matrix products
        e = int(e)
        rs = np.nonzero(ids == e)[0]
        G, U, D = (expert_rows(fmt, gate, e, ffn, hidden), expert_rows(fmt, up, e, ffn, hidden),
                   expert_rows(fmt, down, e, hidden, ffn))
        X = xf[rs // k]
        gb = bf16_round(gate_bias[e * ffn:(e + 1) * ffn]) if gate_bias is not None else 0.0
        ub = (bf16_round(up_bias[e * ffn:(e + 1) * ffn] + (1.0 if up_one else 0.0)) if up_bias is not None
              else (1.0 if up_one else 0.0))
        gat[rs] = X @ G.T + gb
        upv[rs] = X @ U.T + ub
        mag_up[rs] = np.abs(X) @ np.abs(U).T + np.abs(ub)
        act[rs] = (swiglu_clipped_f64 if activation == 0 else swiglu_f64)(gat[rs], upv[rs])
        a_in = act[rs] if act_override is None else np.asarray(act_override, np.float64)[rs]
        db = bf16_round(down_bias[e * hidden:(e + 1) * hidden]) if down_bias is not None else 0.0
        y[rs] = a_in @ D.T + db
        mag_y[rs] = np.abs(a_in) @ np.abs(D).T + np.abs(db)
    p = np.asarray(probs, np.float64).reshape(tokens, k)
    yb = bf16_round(y).reshape(tokens, k, hidden)
    s = np.einsum("tkh,tk->th", yb, p)
    res = bf16_to_f32(np.asarray(residual_bf16, np.uint16)).astype(np.float64)
    out = f32_to_bf16((res + bf16_round(s)).astype(np.float32))
    return {"gate": gat, "up": upv, "up_mag": mag_up, "act": act, "down": y, "down_mag": mag_y, "out": out}


def q4_row_gain(peak: float) -> float:
    """Power-of-two row gain of the scaled Q4 tiles (q4_tile.metal:44-49):
    the f32 exponent e of the row's max |x| gives 2^clamp(141 - e, -120, 120),
    1 for a zero row; x * gain is then rounded to half, and the product
    multiplied by 1 / gain (batch.metal:44-68, 90-98)."""
    bits = int(np.float32(peak).view(np.uint32))
    e = (bits >> 23) & 255
    shift = 0 if peak == 0.0 else min(max(141 - e, -120), 120)
    return float(2.0 ** shift)


def matmul_reference(fmt, w, x, n, k, half_operands: bool, row_gain: bool = False):
    """Y = X W^T in fp64 (matrix_precision.rs:119-142): optionally with both
    operands rounded to f16 first (the reference's tiled kernels' half(w),
    half(x)), and sum |w x| for the roundoff bound.  row_gain: each row
    rounded as half(x * gain) / gain with q4_row_gain of its peak, as the
    scaled Q4_0/Q4_1 tiles do."""
    W = dequant(fmt, w, n * k).astype(np.float64).reshape(n, k)
    x = np.asarray(x)
    X = bf16_to_f32(x).astype(np.float64) if x.dtype == np.uint16 else x.astype(np.float64)
    if half_operands:
        W = W.astype(np.float16).astype(np.float64)
        if row_gain:
            g = np.array([q4_row_gain(float(np.abs(r).max())) for r in X])[:, None]
            X = (X * g).astype(np.float16).astype(np.float64) / g
        else:
            X = X.astype(np.float16).astype(np.float64)
    return X @ W.T, np.abs(X) @ np.abs(W).T


def argmax_f32(logits: np.ndarray) -> int:
    """Greedy selection (argmax.metal:1-47); 0xffffffff for any non-finite logit."""
    x = np.ascontiguousarray(logits, np.float32)
    return int(lib().oo_argmax_f32(_p(x), x.size))


def norm(x_bf16: np.ndarray, w: np.ndarray, epsilon: float, full_layer: bool):
    """RMS norm of bf16 rows (elementwise.metal:6-28): (bf16 bits, f64 values before rounding)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    rows, n = x.shape
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    exact = np.empty(x.shape, np.float64)
    lib().oo_norm(_p(x), _p(w), _p(y), _p(exact), rows, n, epsilon, 1 if full_layer else 0)
    return y, exact


def add_norm(x_bf16: np.ndarray, y_bf16: np.ndarray, w: np.ndarray, epsilon: float, full_layer: bool):
    """Residual add then norm (elementwise.metal:32-58): (new residual, normed, f64 values)."""
    x = np.ascontiguousarray(x_bf16, np.uint16).copy()
    y = np.ascontiguousarray(y_bf16, np.uint16)
    rows, n = x.shape
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    exact = np.empty(x.shape, np.float64)
    lib().oo_add_norm(_p(x), _p(y), _p(w), _p(out), _p(exact), rows, n, epsilon, 1 if full_layer else 0)
    return x, out, exact
