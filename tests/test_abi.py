"""CPU checks of the C-ABI boundary: the library exists, loads, and exports
every symbol include/oco_hip.h declares (no compute calls without a GPU)."""
import ctypes
import os
import re

import oco_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "oco_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(oco_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_operator_surface():
    syms = declared_symbols()
    for need in ["oco_dequant", "oco_matvec", "oco_matmul", "oco_route_select", "oco_router",
                 "oco_route_plan", "oco_experts_apply", "oco_expert_expand", "oco_moe_sum"]:
        assert need in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(oco_amd.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    assert set(declared_symbols()) == set(oco_amd.SIGNATURES)


def test_host_helpers_without_gpu():
    lib = oco_amd.load_library()
    e, b = ctypes.c_uint32(), ctypes.c_uint32()
    for fmt, layout in [(8, (32, 34)), (12, (256, 144)), (14, (256, 210)), (39, (32, 17)),
                        (0, (1, 4)), (30, (1, 2)), (13, (256, 176)), (2, (32, 18)), (3, (32, 20))]:
        assert lib.oco_block_layout(fmt, ctypes.byref(e), ctypes.byref(b)) == 0
        assert (e.value, b.value) == layout == oco_amd.block_layout(fmt)
    assert lib.oco_block_layout(77, ctypes.byref(e), ctypes.byref(b)) == 2
    assert b"77" in lib.oco_last_error()
    assert lib.oco_row_bytes(39, 2880) == 1530
    assert lib.oco_row_bytes(12, 100) == 0
    assert lib.oco_route_plan_words(68, 32) == 6 + 2 * (5 + 32) + 32 * 69 + 32 + 68


def test_argument_validation_without_gpu():
    """Geometry checks fail with OCO_ERR_INVALID before any GPU work (the
    pointers are never dereferenced), and workspace sizes follow the layouts."""
    lib = oco_amd.load_library()
    fake = ctypes.c_void_p(0x1000)
    bad = oco_amd.ExpertsDesc(39, 100, 256, 8, 2, 0, 1, fake, fake, fake, None, None, None)
    rc = lib.oco_experts_apply(ctypes.byref(bad), fake, 0, fake, fake, 4, fake, None, fake, 1 << 30, None)
    assert rc == 1 and b"hidden=100 must be whole blocks" in lib.oco_last_error()
    # ffn is the down projection's reduction length: apply needs whole blocks
    odd = oco_amd.ExpertsDesc(39, 2880, 33, 8, 2, 0, 1, fake, fake, fake, None, None, None)
    rc = lib.oco_experts_apply(ctypes.byref(odd), fake, 0, fake, fake, 4, fake, None, fake, 1 << 30, None)
    assert rc == 1 and b"ffn=33 must be whole blocks" in lib.oco_last_error()
    q4 = oco_amd.ExpertsDesc(12, 2048, 768, 128, 8, 1, 0, fake, fake, fake, None, None, None)
    assert lib.oco_experts_workspace(ctypes.byref(q4), 512) > 512 * 8 * 2048 * 2
    p = oco_amd.Matrix(100, 64, 16, 0, 1, 1, 0)  # k = 100 is not a multiple of 32
    assert lib.oco_matmul(12, fake, fake, 1, fake, 0, None, ctypes.byref(p), None) == 1
    p = oco_amd.Matrix(2880, 5760, 512, 0, 1, 1, 0)
    need = lib.oco_matmul_workspace(39, 1, ctypes.byref(p))
    # per 32 rows and stage of eight 64-wide K steps: two E2M3 terms of 24 B
    # per lane and step, plus one 16-byte scale word per lane (K steps
    # counted to whole stages: 45 -> 48)
    assert need == (512 // 32) * ((2880 // 64 + 7) // 8) * (8 * 64 * 48 + 64 * 16)
    # Q4_K prefill takes the vendor GEMM, whose plan needs a device: none here
    assert lib.oco_matmul_workspace(12, 1, ctypes.byref(p)) == 0
    assert lib.oco_matmul_ws(39, fake, fake, 1, fake, 0, None, ctypes.byref(p), fake, need - 1, None) == 1
    assert b"workspace" in lib.oco_last_error()
    assert lib.oco_route_plan(fake, 64, 32, 8, 0, 0, fake, None) == 1  # tile_rows < 16
    assert lib.oco_moe_sum(fake, 0, fake, fake, 64, 2, 9, None) == 1  # at most 8 routes per token
    assert b"at most 8" in lib.oco_last_error()
    # MXFP4 expert records: 208 bytes per (row, K step of 64) -- four E2M3
    # terms of 24 bytes per block (two blocks) and the scale words, padded
    mx = oco_amd.ExpertsDesc(39, 2880, 2880, 32, 4, 0, 1, fake, fake, fake, None, None, None)
    assert lib.oco_experts_workspace(ctypes.byref(mx), 16) > 16 * 45 * 208 + 64 * 45 * 208
    # the allocation-free entry point takes what fits its 8 MiB array and
    # rejects more before any GPU work
    assert lib.oco_experts_workspace(ctypes.byref(mx), 57) <= 8 << 20 < lib.oco_experts_workspace(ctypes.byref(mx), 58)
    rc = lib.oco_experts_forward_static(ctypes.byref(mx), fake, None, fake, 0, 58, fake, fake, fake, None, None)
    assert rc == 1 and b"scratch" in lib.oco_last_error()


def test_xor32_geometry_at_the_size_limit():
    """The read stream's rounds and grid stay finite and in 32-bit offsets up
    to its limit, and sizes past it are refused before any launch."""
    lib = oco_amd.load_library()
    rounds, grid = ctypes.c_uint64(), ctypes.c_uint64()
    limit = 0xffffffff - 32768
    for words, want_rounds in [(4, 1), (4096, 1), (4100, 2), (2203200, 538), (limit // 4, (limit // 4 * 4 + 16383) // 16384)]:
        assert lib.oco_buffer_xor32_geometry(words, ctypes.byref(rounds), ctypes.byref(grid)) == 0
        assert rounds.value == want_rounds
        assert grid.value == min(rounds.value, 1024)
        # the last round's reads end inside 32-bit offsets
        assert (rounds.value - 1) * 16384 + 16384 <= 1 << 32
    for words in [limit // 4 + 1, (1 << 30), (1 << 32)]:
        assert lib.oco_buffer_xor32_geometry(words, ctypes.byref(rounds), ctypes.byref(grid)) == 1
        assert b"limit" in lib.oco_last_error()
