"""oco_amd: MI355X (gfx950) quantized-weight matrix path of oco.

The product is the native library ``liboco_hip.so`` (HIP kernels behind the C
ABI in ``include/oco_hip.h``).  This package loads it with ctypes and mirrors
the reference's operator seam so callers and tests read like oco's own:

- ``WeightFormat`` / ``block_layout``   -> src/tensor.rs:9-38
- ``DeviceBuffer``                      -> src/gpu/buffer.rs (ReadOnly / BufferView)
- ``DenseMatrix`` (apply_row / apply)   -> src/weights/operands.rs:4-9, compute/matrix.rs:63,130
- ``Output``                            -> compute/matrix.rs:519-548 (f32 logits)
- ``ExpertBank`` / ``Router``           -> operands.rs ExpertWeight/Router, feed_forward.rs:107

There is no CPU fallback: every compute call goes through the HIP library,
and loading fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes
import enum
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboco_hip.so")


class WeightFormat(enum.IntEnum):
    """GGUF format codes (src/tensor.rs:9-20)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q8_0 = 8
    Q4K = 12
    Q5K = 13
    Q6K = 14
    Bf16 = 30
    Mxfp4 = 39


class Knob(enum.IntEnum):
    """oco_knob: kernel-choice overrides (tests and tuning runs)."""
    STREAM_PLAN = 0
    MATVEC_PLAN = 1
    MATVEC_PLAIN = 2
    MX_TILE = 3
    MX_PREFILL_OFF = 4
    MATMUL_TILE = 5
    MOE_MX_TOKENS = 6
    MOE_MFMA_TOKENS = 7
    MOE_Q4_ROWS = 8
    MOE_WG = 9
    MX_EXPERTS_KS = 10
    STREAM_DIRECT = 11
    MATMUL_VENDOR = 12


class DType(enum.IntEnum):
    F32 = 0
    BF16 = 1
    F16 = 2


class Activation(enum.IntEnum):
    SWIGLU_CLIPPED = 0
    SWIGLU = 1


_BLOCKS = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34),
           12: (256, 144), 13: (256, 176), 14: (256, 210), 39: (32, 17)}


def block_layout(fmt: int) -> tuple[int, int]:
    """(elements, bytes) per block (src/tensor.rs:24-38)."""
    return _BLOCKS[int(fmt)]


def row_bytes(fmt: int, k: int) -> int:
    e, b = block_layout(fmt)
    if k % e:
        raise ValueError(f"k={k} is not a multiple of the {WeightFormat(fmt).name} block ({e})")
    return k // e * b


class OcoError(RuntimeError):
    """Raised for a non-zero status from the C ABI (src/error.rs:9-27)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class Matrix(ctypes.Structure):
    """oco_matrix / Matrix (weights.metal:87-89)."""
    _fields_ = [(n, ctypes.c_uint32) for n in
                ("k", "n", "m", "route_major", "routes", "experts", "has_bias")]


def as_matrix(p) -> Matrix:
    """Accept any object with the Matrix fields (e.g. a struct from another module)."""
    if isinstance(p, Matrix):
        return p
    return Matrix(*[int(getattr(p, f)) for f, _ in Matrix._fields_])


class ExpertsDesc(ctypes.Structure):
    """oco_experts."""
    _fields_ = [("format", ctypes.c_uint32), ("hidden", ctypes.c_uint32), ("ffn", ctypes.c_uint32),
                ("experts", ctypes.c_uint32), ("k", ctypes.c_uint32),
                ("activation", ctypes.c_uint32), ("up_bias_one", ctypes.c_uint32),
                ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("gate_bias", ctypes.c_void_p), ("up_bias", ctypes.c_void_p),
                ("down_bias", ctypes.c_void_p)]


class GgufEntry(ctypes.Structure):
    """oco_gguf_entry (Entry, gguf.rs:24-33)."""
    _fields_ = [("shape", ctypes.c_uint64 * 4), ("rank", ctypes.c_uint32), ("code", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("extent", ctypes.c_uint64)]


class GgufTensor(ctypes.Structure):
    """oco_gguf_tensor (Tensor, gguf.rs:17-22)."""
    _fields_ = [("format", ctypes.c_uint32), ("rank", ctypes.c_uint32), ("shape", ctypes.c_uint64 * 4),
                ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


# Every symbol include/oco_hip.h declares, with its ctypes signature.
_vp, _u32, _u64, _i32, _sz = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_size_t
_MP = ctypes.POINTER(Matrix)
_EP = ctypes.POINTER(ExpertsDesc)
SIGNATURES = {
    "oco_last_error": (ctypes.c_char_p, []),
    "oco_plan_override": (_i32, [_u32, ctypes.POINTER(ctypes.c_int32), _u32]),
    "oco_block_layout": (_i32, [_u32, ctypes.POINTER(_u32), ctypes.POINTER(_u32)]),
    "oco_row_bytes": (_u64, [_u32, _u32]),
    "oco_device_open": (_i32, [_i32, ctypes.POINTER(_i32)]),
    "oco_buffer_alloc": (_i32, [_sz, ctypes.POINTER(_vp)]),
    "oco_buffer_free": (_i32, [_vp]),
    "oco_buffer_upload": (_i32, [_vp, _vp, _sz]),
    "oco_buffer_download": (_i32, [_vp, _vp, _sz]),
    "oco_buffer_copy": (_i32, [_vp, _vp, _sz, _vp]),
    "oco_buffer_fill32": (_i32, [_vp, _u32, _sz, _vp]),
    "oco_buffer_xor32": (_i32, [_vp, _sz, _vp, _vp]),
    "oco_buffer_xor32_geometry": (_i32, [_u64, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "oco_stream_create": (_i32, [ctypes.POINTER(_vp)]),
    "oco_stream_sync": (_i32, [_vp]),
    "oco_stream_destroy": (_i32, [_vp]),
    "oco_event_create": (_i32, [ctypes.POINTER(_vp)]),
    "oco_event_record": (_i32, [_vp, _vp]),
    "oco_event_elapsed_ms": (_i32, [_vp, _vp, ctypes.POINTER(ctypes.c_float)]),
    "oco_event_destroy": (_i32, [_vp]),
    "oco_graph_begin": (_i32, [_vp]),
    "oco_graph_end": (_i32, [_vp, ctypes.POINTER(_vp)]),
    "oco_graph_launch": (_i32, [_vp, _vp]),
    "oco_graph_destroy": (_i32, [_vp]),
    "oco_dequant": (_i32, [_u32, _vp, _u64, _vp, _vp]),
    "oco_embed": (_i32, [_u32, _vp, _u32, _u32, _vp, _u32, _vp, _u32, _vp, _vp]),
    "oco_matvec": (_i32, [_u32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _MP, _vp]),
    "oco_matvec_relu_sqr": (_i32, [_u32, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _MP, _vp]),
    "oco_matmul": (_i32, [_u32, _vp, _vp, _i32, _vp, _i32, _vp, _MP, _vp]),
    "oco_matmul_workspace": (_u64, [_u32, _i32, _MP]),
    "oco_matmul_ws": (_i32, [_u32, _vp, _vp, _i32, _vp, _i32, _vp, _MP, _vp, _u64, _vp]),
    "oco_norm_mx_split": (_i32, [_vp, _vp, _vp, _u32, _u32, ctypes.c_float, _i32, _vp, _u64, _vp]),
    "oco_add_norm_mx_split": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float, _i32, _vp, _u64, _vp]),
    "oco_matmul_mx_split": (_i32, [_vp, _vp, _u64, _vp, _i32, _vp, _MP, _vp]),
    "oco_route_select": (_i32, [_vp, _u32, _u32, _u32, _vp, _vp, _vp]),
    "oco_router": (_i32, [_vp, _i32, _vp, _vp, _u32, _u32, _u32, _u32, _vp, _vp, _vp, _vp]),
    "oco_route_plan_words": (_u64, [_u32, _u32]),
    "oco_route_plan": (_i32, [_vp, _u32, _u32, _u32, _u32, _u32, _vp, _vp]),
    "oco_experts_workspace": (_u64, [_EP, _u32]),
    "oco_experts_apply": (_i32, [_EP, _vp, _i32, _vp, _vp, _u32, _vp, _vp, _vp, _u64, _vp]),
    "oco_experts_forward": (_i32, [_EP, _vp, _vp, _vp, _i32, _u32, _vp, _vp, _vp, _vp, _vp, _u64, _vp]),
    "oco_experts_forward_static": (_i32, [_EP, _vp, _vp, _vp, _i32, _u32, _vp, _vp, _vp, _vp, _vp]),
    "oco_expert_expand": (_i32, [_EP, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "oco_moe_sum": (_i32, [_vp, _i32, _vp, _vp, _u32, _u32, _u32, _vp]),
    "oco_norm": (_i32, [_vp, _vp, _vp, _u32, _u32, ctypes.c_float, _i32, _vp]),
    "oco_add_norm": (_i32, [_vp, _vp, _vp, _vp, _u32, _u32, ctypes.c_float, _i32, _vp]),
    "oco_matvec_norm": (_i32, [_u32, _vp, _vp, _vp, ctypes.c_float, _i32, _vp, _i32, _vp, _vp, _MP, _vp]),
    "oco_matvec_group": (_i32, [_u32, _u32, _vp, _vp, _i32, _vp, ctypes.c_float, _i32, _vp, _i32, _vp, _MP, _vp]),
    "oco_argmax_f32": (_i32, [_vp, _u32, _vp, _vp]),
    "oco_argmax_workspace": (_u64, [_u32]),
    "oco_argmax_f32_ws": (_i32, [_vp, _u32, _vp, _vp, _u64, _vp]),
    "oco_gguf_open": (_i32, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), _u32, ctypes.POINTER(_vp)]),
    "oco_gguf_close": (_i32, [_vp]),
    "oco_gguf_has": (_i32, [_vp, ctypes.c_char_p]),
    "oco_gguf_text": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp), ctypes.POINTER(_sz)]),
    "oco_gguf_number": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "oco_gguf_boolean": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_i32)]),
    "oco_gguf_unsigned": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
    "oco_gguf_array": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_u32), ctypes.POINTER(_u64)]),
    "oco_gguf_array_string": (_i32, [_vp, ctypes.c_char_p, _u64, ctypes.POINTER(_vp), ctypes.POINTER(_sz)]),
    "oco_gguf_array_unsigned": (_i32, [_vp, ctypes.c_char_p, _vp, _u64]),
    "oco_gguf_directory": (_i32, [_vp, ctypes.POINTER(_u64)]),
    "oco_gguf_entry_at": (_i32, [_vp, _u64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(GgufEntry)]),
    "oco_gguf_find": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(GgufEntry)]),
    "oco_gguf_select": (_i32, [ctypes.POINTER(GgufEntry), ctypes.POINTER(GgufTensor)]),
    "oco_gguf_data": (_vp, [_vp, ctypes.POINTER(GgufTensor)]),
    "oco_gguf_upload": (_i32, [_vp, ctypes.POINTER(GgufTensor), _vp, _vp]),
}

_lib = None


def load_library(path: str = LIB_PATH):
    """Load liboco_hip.so and bind every declared symbol (fails loudly if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise OSError(f"{path} is missing: run __graft_entry__.build() (hipcc for gfx950) first")
    L = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name, None)
        if fn is None:  # tests/test_abi.py asserts every declared symbol is exported
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise OcoError(rc, load_library().oco_last_error().decode())


_device_open = False


def open_device(ordinal: int = 0) -> int:
    """Gpu::new (src/gpu.rs:41-50): select the device, return its CU count."""
    global _device_open
    cu = ctypes.c_int()
    _check(load_library().oco_device_open(ordinal, ctypes.byref(cu)))
    _device_open = True
    return cu.value


def _ensure_device():
    if not _device_open:
        open_device(0)


def plan_override(knob: int, values=()):
    """Override one kernel-choice table entry (empty `values` clears it)."""
    vals = (ctypes.c_int32 * max(len(values), 1))(*[int(v) for v in values])
    _check(load_library().oco_plan_override(int(knob), vals, len(values)))


class overridden:
    """Context manager: `with overridden(Knob.X, (a, b)):` ... then cleared."""

    def __init__(self, knob: int, values):
        self.knob, self.values = knob, tuple(values)

    def __enter__(self):
        plan_override(self.knob, self.values)
        return self

    def __exit__(self, *a):
        plan_override(self.knob, ())


class Stream:
    """One HIP stream (the reference's per-session queue, compute.rs:36-55)."""

    def __init__(self):
        _ensure_device()
        h = ctypes.c_void_p()
        _check(load_library().oco_stream_create(ctypes.byref(h)))
        self.handle = h

    def sync(self):
        _check(load_library().oco_stream_sync(self.handle))

    def close(self):
        if self.handle:
            _check(load_library().oco_stream_destroy(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        h = ctypes.c_void_p()
        _check(load_library().oco_event_create(ctypes.byref(h)))
        self.handle = h

    def record(self, stream=None):
        _check(load_library().oco_event_record(self.handle, _stream(stream)))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(load_library().oco_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.oco_event_destroy(self.handle)
        except Exception:
            pass


class Graph:
    """Captured launches replayed natively (stream capture into a HIP graph)."""

    def __init__(self, stream: "Stream", record):
        _check(load_library().oco_graph_begin(stream.handle))
        try:
            record()
        finally:
            h = ctypes.c_void_p()
            rc = load_library().oco_graph_end(stream.handle, ctypes.byref(h))
        _check(rc)
        self.handle = h
        self.stream = stream

    def launch(self):
        _check(load_library().oco_graph_launch(self.handle, self.stream.handle))

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.oco_graph_destroy(self.handle)
        except Exception:
            pass


def _stream(s):
    if s is None:
        return None
    return s.handle if isinstance(s, Stream) else s


class DeviceBuffer:
    """Device allocation (src/gpu/buffer.rs BufferView / ReadOnly)."""

    def __init__(self, nbytes: int):
        _ensure_device()
        p = ctypes.c_void_p()
        _check(load_library().oco_buffer_alloc(max(int(nbytes), 1), ctypes.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        _check(load_library().oco_buffer_upload(self.ptr + offset, a.ctypes.data, a.nbytes))

    def download(self, dtype, count=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        _check(load_library().oco_buffer_download(out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def fill32(self, pattern: int, stream=None):
        _check(load_library().oco_buffer_fill32(self.ptr, pattern & 0xFFFFFFFF, self.nbytes // 4,
                                                _stream(stream)))

    def xor32(self, out, stream=None, offset: int = 0, nbytes=None):
        """out[0..1023] (device) XOR to the XOR of the buffer's 32-bit words (oco_buffer_xor32)."""
        n = (self.nbytes - offset) if nbytes is None else nbytes
        _check(load_library().oco_buffer_xor32(self.ptr + offset, n // 4, _addr(out), _stream(stream)))

    def at(self, offset: int) -> int:
        return self.ptr + offset

    def free(self):
        if self.ptr:
            _check(load_library().oco_buffer_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.oco_buffer_free(self.ptr)
        except Exception:
            pass


def _addr(b) -> int | None:
    if b is None:
        return None
    if isinstance(b, DeviceBuffer):
        return b.ptr
    return int(b)


def synchronize(stream=None):
    if stream is None:
        _check(load_library().oco_stream_sync(None))
    else:
        _check(load_library().oco_stream_sync(_stream(stream)))


# ---- operations (thin wrappers over the C ABI) -------------------------------

def dequant(fmt: int, w, count: int, out, stream=None):
    _check(load_library().oco_dequant(int(fmt), _addr(w), count, _addr(out), _stream(stream)))


def embed(fmt: int, w, k: int, vocabulary: int, ids, rows: int, out, features=None, feature_rows: int = 0,
          stream=None):
    """Token rows to bf16 (embed, weights.metal:90-109): ids >= vocabulary take feature rows."""
    _check(load_library().oco_embed(int(fmt), _addr(w), k, vocabulary, _addr(ids), rows, _addr(features),
                                    feature_rows, _addr(out), _stream(stream)))


class Embedding:
    """Embedding operand (src/weights/operands.rs Embedding; Builder::embedding,
    pipelines.rs:180-193): a GGUF tensor [width, vocabulary] and its lookup."""

    def __init__(self, fmt: int, values, width: int, vocabulary: int):
        self.format, self.values, self.width, self.vocabulary = int(fmt), values, width, vocabulary

    def embed(self, ids, rows: int, out, features=None, feature_rows: int = 0, stream=None):
        """Compute::embed (compute/matrix.rs:487-516)."""
        embed(self.format, self.values, self.width, self.vocabulary, ids, rows, out, features, feature_rows, stream)


def matvec(fmt: int, w, x, y, p: Matrix, x_dtype=DType.F32, y_dtype=DType.F32, bias=None,
           ids=None, stream=None, relu_sqr: bool = False):
    """oco_matvec, or oco_matvec_relu_sqr (x -> max(x, 0)^2 on load) when relu_sqr."""
    lib = load_library()
    fn = lib.oco_matvec_relu_sqr if relu_sqr else lib.oco_matvec
    _check(fn(int(fmt), _addr(w), _addr(x), int(x_dtype), _addr(y), int(y_dtype), _addr(bias), _addr(ids),
              ctypes.byref(as_matrix(p)), _stream(stream)))


def matmul(fmt: int, w, x, y, p: Matrix, x_dtype=DType.BF16, y_dtype=DType.F32, bias=None,
           stream=None, workspace=None, workspace_bytes: int = 0):
    """oco_matmul, or oco_matmul_ws when a workspace is given."""
    lib = load_library()
    if workspace is None:
        _check(lib.oco_matmul(int(fmt), _addr(w), _addr(x), int(x_dtype), _addr(y), int(y_dtype),
                              _addr(bias), ctypes.byref(as_matrix(p)), _stream(stream)))
    else:
        _check(lib.oco_matmul_ws(int(fmt), _addr(w), _addr(x), int(x_dtype), _addr(y), int(y_dtype),
                                 _addr(bias), ctypes.byref(as_matrix(p)), _addr(workspace),
                                 int(workspace_bytes), _stream(stream)))


def matmul_workspace(fmt: int, p: Matrix, x_dtype=DType.BF16) -> int:
    return int(load_library().oco_matmul_workspace(int(fmt), int(x_dtype), ctypes.byref(as_matrix(p))))


def norm_mx_split(x, w, y, rows: int, n: int, epsilon: float, full_layer: bool, split, split_bytes: int,
                  stream=None):
    """oco_norm_mx_split: RMS norm rows (y optional) and their MXFP4-prefill split records."""
    _check(load_library().oco_norm_mx_split(_addr(x), _addr(w), _addr(y), rows, n, float(epsilon),
                                            1 if full_layer else 0, _addr(split), int(split_bytes),
                                            _stream(stream)))


def add_norm_mx_split(x, y, w, out, rows: int, n: int, epsilon: float, full_layer: bool, split, split_bytes: int,
                      stream=None):
    """oco_add_norm_mx_split: x = bf16(x + y), then norm_mx_split of x (out optional)."""
    _check(load_library().oco_add_norm_mx_split(_addr(x), _addr(y), _addr(w), _addr(out), rows, n, float(epsilon),
                                                1 if full_layer else 0, _addr(split), int(split_bytes),
                                                _stream(stream)))


def matmul_mx_split(w, split, split_bytes: int, y, p: Matrix, y_dtype=DType.F32, bias=None, stream=None):
    """oco_matmul_mx_split: the MXFP4 prefill from rows split by norm_mx_split."""
    _check(load_library().oco_matmul_mx_split(_addr(w), _addr(split), int(split_bytes), _addr(y), int(y_dtype),
                                              _addr(bias), ctypes.byref(as_matrix(p)), _stream(stream)))


def route_select(logits, tokens: int, experts: int, k: int, ids, probs, stream=None):
    _check(load_library().oco_route_select(_addr(logits), tokens, experts, k, _addr(ids),
                                           _addr(probs), _stream(stream)))


def router(x, x_dtype, w, bias, tokens, hidden, experts, k, logits, ids, probs, stream=None):
    _check(load_library().oco_router(_addr(x), int(x_dtype), _addr(w), _addr(bias), tokens, hidden,
                                     experts, k, _addr(logits), _addr(ids), _addr(probs),
                                     _stream(stream)))


def route_plan_words(routes: int, experts: int) -> int:
    return int(load_library().oco_route_plan_words(routes, experts))


def route_plan(ids, routes, experts, tile_rows, up_tiles, down_tiles, plan, stream=None):
    _check(load_library().oco_route_plan(_addr(ids), routes, experts, tile_rows, up_tiles,
                                         down_tiles, _addr(plan), _stream(stream)))


def moe_sum(routes, routes_dtype, probs, out, hidden, tokens, k, stream=None):
    _check(load_library().oco_moe_sum(_addr(routes), int(routes_dtype), _addr(probs), _addr(out),
                                      hidden, tokens, k, _stream(stream)))


def norm(x, w, y, rows: int, n: int, epsilon: float, full_layer: bool = True, stream=None):
    """Compute::norm (elementwise.metal:6-28) over bf16 rows."""
    _check(load_library().oco_norm(_addr(x), _addr(w), _addr(y), rows, n, epsilon, int(full_layer),
                                   _stream(stream)))


def add_norm(x, y, w, out, rows: int, n: int, epsilon: float, full_layer: bool = True, stream=None):
    """add_norm (elementwise.metal:32-58): x = bf16(x + y) in place, out = norm(x)."""
    _check(load_library().oco_add_norm(_addr(x), _addr(y), _addr(w), _addr(out), rows, n, epsilon,
                                       int(full_layer), _stream(stream)))


def matvec_norm(fmt: int, w, x, norm_w, epsilon: float, y, p: Matrix, full_layer: bool = True,
                y_dtype=DType.F32, bias=None, ids=None, stream=None):
    """norm -> matvec with the norm fused into the matvec's activation staging."""
    _check(load_library().oco_matvec_norm(int(fmt), _addr(w), _addr(x), _addr(norm_w), epsilon,
                                          int(full_layer), _addr(y), int(y_dtype), _addr(bias), _addr(ids),
                                          ctypes.byref(as_matrix(p)), _stream(stream)))


def matvec_group(fmt: int, ws, x, ys, p: Matrix, x_dtype=DType.BF16, y_dtype=DType.F32, norm_w=None,
                 epsilon: float = 1e-6, full_layer: bool = True, biases=None, stream=None):
    """Several matrices over the same input rows in one grid (the concurrent
    up/gate pair of feed_forward.rs:97-104); norm_w: fused RMS norm of bf16 x."""
    n = len(ws)
    wa = (ctypes.c_void_p * n)(*[_addr(w) for w in ws])
    ya = (ctypes.c_void_p * n)(*[_addr(y) for y in ys])
    ba = (ctypes.c_void_p * n)(*[_addr(b) for b in biases]) if biases is not None else None
    _check(load_library().oco_matvec_group(int(fmt), n, wa, _addr(x), int(x_dtype), _addr(norm_w), epsilon,
                                           int(full_layer), ya, int(y_dtype), ba, ctypes.byref(as_matrix(p)),
                                           _stream(stream)))


def argmax_workspace(n: int) -> int:
    return int(load_library().oco_argmax_workspace(n))


def argmax(logits, n: int, out, stream=None, workspace=None, workspace_bytes: int = 0):
    """Compute::argmax (compute.rs:132-140): greedy token over f32 logits."""
    lib = load_library()
    if workspace is None:
        _check(lib.oco_argmax_f32(_addr(logits), n, _addr(out), _stream(stream)))
    else:
        _check(lib.oco_argmax_f32_ws(_addr(logits), n, _addr(out), _addr(workspace), int(workspace_bytes),
                                     _stream(stream)))


# ---- GGUF checkpoints (src/gguf.rs) ---------------------------------------------

class Gguf:
    """Gguf (gguf.rs:98-348): an open, structurally validated GGUF v3 file."""

    def __init__(self, path: str, keep=()):
        lib = load_library()
        keys = [k.encode() for k in keep]
        arr = (ctypes.c_char_p * max(len(keys), 1))(*keys)
        h = ctypes.c_void_p()
        _check(lib.oco_gguf_open(os.fsencode(path), arr, len(keys), ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            load_library().oco_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _bytes(self, fn, key, *extra):
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        _check(fn(self.handle, key.encode(), *extra, ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""

    def has(self, key: str) -> bool:
        return bool(load_library().oco_gguf_has(self.handle, key.encode()))

    def text(self, key: str) -> str:
        return self._bytes(load_library().oco_gguf_text, key)

    def number(self, key: str) -> float:
        v = ctypes.c_double()
        _check(load_library().oco_gguf_number(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def boolean(self, key: str) -> bool:
        v = ctypes.c_int()
        _check(load_library().oco_gguf_boolean(self.handle, key.encode(), ctypes.byref(v)))
        return bool(v.value)

    def optional_unsigned(self, key: str):
        if not self.has(key):
            return None
        v = ctypes.c_uint64()
        _check(load_library().oco_gguf_unsigned(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def strings(self, key: str) -> list:
        kind, count = ctypes.c_uint32(), ctypes.c_uint64()
        _check(load_library().oco_gguf_array(self.handle, key.encode(), ctypes.byref(kind), ctypes.byref(count)))
        return [self._bytes(load_library().oco_gguf_array_string, key, ctypes.c_uint64(i)) for i in range(count.value)]

    def unsigned_integers(self, key: str) -> list:
        kind, count = ctypes.c_uint32(), ctypes.c_uint64()
        _check(load_library().oco_gguf_array(self.handle, key.encode(), ctypes.byref(kind), ctypes.byref(count)))
        out = np.zeros(max(count.value, 1), np.uint64)
        _check(load_library().oco_gguf_array_unsigned(self.handle, key.encode(), out.ctypes.data, count.value))
        return [int(v) for v in out[:count.value]]

    def directory(self) -> dict:
        lib = load_library()
        n = ctypes.c_uint64()
        _check(lib.oco_gguf_directory(self.handle, ctypes.byref(n)))
        out = {}
        for i in range(n.value):
            name, e = ctypes.c_char_p(), GgufEntry()
            _check(lib.oco_gguf_entry_at(self.handle, i, ctypes.byref(name), ctypes.byref(e)))
            out[name.value.decode()] = e
        return out

    @staticmethod
    def select(entry: GgufEntry) -> GgufTensor:
        t = GgufTensor()
        _check(load_library().oco_gguf_select(ctypes.byref(entry), ctypes.byref(t)))
        return t

    def data(self, t: GgufTensor) -> np.ndarray:
        p = load_library().oco_gguf_data(self.handle, ctypes.byref(t))
        if not p:
            raise OcoError(5, "tensor outside the mapping")
        return np.ctypeslib.as_array((ctypes.c_uint8 * t.bytes).from_address(p)).copy()

    def upload(self, t: GgufTensor, dst=None, stream=None) -> "DeviceBuffer":
        buf = dst if dst is not None else DeviceBuffer(t.bytes)
        _check(load_library().oco_gguf_upload(self.handle, ctypes.byref(t), _addr(buf), _stream(stream)))
        return buf


# ---- operator mirror -----------------------------------------------------------

class DenseMatrix:
    """A learned linear map with its GGUF storage (operands.rs:4-9).

    ``input``/``output`` follow oco's [input, output] GGUF shape convention
    (load.rs:175-186); ``values`` is the device buffer of GGUF rows.
    """

    def __init__(self, values: DeviceBuffer, fmt: int, input: int, output: int, offset: int = 0):
        self.values, self.format, self.input, self.output = values, int(fmt), input, output
        self.offset = offset
        row_bytes(fmt, input)

    def _w(self):
        return self.values.ptr + self.offset

    def apply_row(self, x, y, x_dtype=DType.F32, y_dtype=DType.F32, bias=None, rows: int = 1,
                  stream=None):
        """Decode path (compute/matrix.rs:63): y[r] = W x[r] for `rows` rows."""
        p = Matrix(self.input, self.output, rows, 0, 1, 1, 1 if bias is not None else 0)
        matvec(self.format, self._w(), x, y, p, x_dtype, y_dtype, bias, None, stream)

    def apply(self, x, y, rows: int, x_dtype=DType.BF16, y_dtype=DType.F32, bias=None,
              stream=None):
        """Prefill path (compute/matrix.rs:130): Y = X W^T on MFMA."""
        p = Matrix(self.input, self.output, rows, 0, 1, 1, 1 if bias is not None else 0)
        matmul(self.format, self._w(), x, y, p, x_dtype, y_dtype, bias, stream)


class Output(DenseMatrix):
    """lm_head scoring in f32 (Bindings::output, compute/matrix.rs:519-548)."""

    def apply_row(self, x, y, x_dtype=DType.F32, y_dtype=DType.F32, bias=None, rows: int = 1,
                  stream=None):
        super().apply_row(x, y, x_dtype, DType.F32, bias, rows, stream)


class ExpertBank:
    """Routed expert weights (gpt_oss/load.rs:20-40; Experts/ExpertPlan, feed_forward.rs:34-77)."""

    def __init__(self, fmt: int, hidden: int, ffn: int, experts: int, k: int, gate, up, down,
                 gate_bias=None, up_bias=None, down_bias=None,
                 activation=Activation.SWIGLU_CLIPPED, up_bias_one: bool = True):
        self.desc = ExpertsDesc(int(fmt), hidden, ffn, experts, k, int(activation),
                                1 if up_bias_one else 0, _addr(gate), _addr(up), _addr(down),
                                _addr(gate_bias), _addr(up_bias), _addr(down_bias))
        self._keep = (gate, up, down, gate_bias, up_bias, down_bias)
        self._workspace = None

    def workspace_bytes(self, tokens: int) -> int:
        return int(load_library().oco_experts_workspace(ctypes.byref(self.desc), tokens))

    def apply(self, x, x_dtype, ids, probs, tokens: int, out, routed=None, workspace=None,
              stream=None):
        """Bindings::experts (feed_forward.rs:107-275) after the router."""
        need = self.workspace_bytes(tokens)
        if workspace is None:
            if self._workspace is None or self._workspace.nbytes < need:
                self._workspace = DeviceBuffer(max(need, 256))
            workspace = self._workspace
        ws_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else need
        _check(load_library().oco_experts_apply(ctypes.byref(self.desc), _addr(x), int(x_dtype),
                                                _addr(ids), _addr(probs), tokens, _addr(out),
                                                _addr(routed), _addr(workspace), ws_bytes,
                                                _stream(stream)))

    def forward(self, router_w, router_bias, x, x_dtype, tokens: int, out, ids, probs, routed=None,
                workspace=None, stream=None):
        """Bindings::experts (feed_forward.rs:107-275) from the router logits on:
        ids/probs [tokens, k] receive the device's expert selection."""
        need = self.workspace_bytes(tokens)
        if workspace is None:
            if self._workspace is None or self._workspace.nbytes < need:
                self._workspace = DeviceBuffer(max(need, 256))
            workspace = self._workspace
        ws_bytes = workspace.nbytes if isinstance(workspace, DeviceBuffer) else need
        _check(load_library().oco_experts_forward(ctypes.byref(self.desc), _addr(router_w), _addr(router_bias),
                                                  _addr(x), int(x_dtype), tokens, _addr(out), _addr(ids),
                                                  _addr(probs), _addr(routed), _addr(workspace), ws_bytes,
                                                  _stream(stream)))

    def expand(self, x, x_dtype, logits, ids, probs, up_out, act_out, stream=None):
        """expert_expand (projections.metal:78-137) for one token."""
        _check(load_library().oco_expert_expand(ctypes.byref(self.desc), _addr(x), int(x_dtype),
                                                _addr(logits), _addr(ids), _addr(probs),
                                                _addr(up_out), _addr(act_out), _stream(stream)))
