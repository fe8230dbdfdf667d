"""CPU checks of the C ABI: the library loads and exports every entry point include/*.h declares, the host mirror
keeps the reference's names, and the product path never touches the oracle."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if h.endswith(".h"):
            txt = open(os.path.join(ROOT, "include", h)).read()
            txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
            names |= set(re.findall(r"\b(moex_[a-z0-9_]+)\s*\(", txt))
    return sorted(names)


def test_header_declares_the_reference_entry_points():
    names = _declared()
    for n in ("moex_attn_decode", "moex_attn_fa", "moex_attn_prefill", "moex_kv_alloc", "moex_kv_bytes",
              "moex_attn_gqa", "moex_attn_combine", "moex_attn_decode_heads", "moex_turbo_out", "moex_qk_norm_rope",
              "moex_quantize_rows_i8", "moex_gemv_i8", "moex_gemm_i8"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import ctypes
    import moex_amd
    if not os.path.exists(moex_amd.LIB_PATH):
        pytest.skip("libmoex_attn.so not built (run __graft_entry__.build())")
    L = ctypes.CDLL(moex_amd.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, missing
    assert sorted(moex_amd.EXPORTS) == _declared()


def test_kv_bytes_formula():
    import moex_amd
    if not os.path.exists(moex_amd.LIB_PATH):
        pytest.skip("libmoex_attn.so not built")
    # kernels.cuh:1875: int8 520 B, turbo 240 B per (kv head, position)
    assert moex_amd.kv_bytes(2, 90000, 0) == 2 * 90000 * 520
    assert moex_amd.kv_bytes(2, 262144, 1) == 2 * 262144 * 240


def test_python_mirror_keeps_reference_names():
    import moex_amd
    for n in ("attn_decode", "attn_fa", "attn_prefill", "kv_alloc", "kv_bytes", "attn_gqa", "attn_combine",
              "attn_decode_heads", "turbo_out", "qk_norm_rope", "kv_append", "set_int", "gemv", "gemm",
              "quantize_rows_q4", "quantize_rows_q6"):
        assert callable(getattr(moex_amd, n))


def test_product_never_uses_the_oracle():
    for dirpath, _, files in os.walk(os.path.join(ROOT, "moex_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".hpp", ".h")) or f == "Makefile":
                txt = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in txt.replace("oracle/", ""), f
    # the built library links nothing from oracle/
    import moex_amd
    if os.path.exists(moex_amd.LIB_PATH):
        assert b"liboracle" not in open(moex_amd.LIB_PATH, "rb").read()


def test_gqa_splits_policy():
    """moex_attn_decode fills one workgroup per CU (256 on MI355X, the fallback without a device): per kv head and
    int8 group of up to 4 tokens (one token or a pair alone), or per kv head and turbo token, never above ns"""
    import moex_amd as M
    assert M.gqa_splits(1, 2, 256) == 128
    assert M.gqa_splits(2, 2, 256) == 128
    assert M.gqa_splits(4, 2, 256) == 128
    assert M.gqa_splits(8, 2, 256) == 64
    assert M.gqa_splits(4, 2, 32) == 32
    assert M.gqa_splits(4, 2, 256, turbo=1) == 32
    assert M.gqa_splits(1, 2, 256, turbo=1) == 128
    assert M.gqa_splits(64, 2, 256) == 8


def test_attn_workspace_bytes():
    """The per-stream workspace one attn_fa call takes (for a VRAM audit beside kv_bytes): tile images of
    KV * ceil(max_t / 32) * 37632 B, plus partial rows of split token tiles for short chunks; for chunks of at most
    64 tokens, at least the decode kernels' partials T * H * ns * 1032 B, which int8 chunks take instead (the count
    covers turbo chunks, which take the FA path); full grids add the halves of their paired token tiles,
    KV * (tiles / 2) * 4 wavefront slots of 33280 B, and 8 B of arrival counters per slot. 256 CUs: the fallback
    without a device, MI355X's count."""
    import moex_amd as M
    if not os.path.exists(M.LIB_PATH):
        pytest.skip("libmoex_attn.so not built")
    pairs = 2 * 64 * 4 * (33280 + 8)                                                # 2048 tokens: 128 tiles
    assert M.attn_workspace_bytes(16, 2, 34816, 2048) == 2 * 1088 * 37632 + pairs  # configs[1]
    assert M.attn_workspace_bytes(16, 2, 262144, 2048) == 2 * 8192 * 37632 + pairs  # configs[4]: 617 MB
    assert M.attn_workspace_bytes(16, 2, 40000, 64) == 2 * 1250 * 37632 + 64 * 16 * 32 * 1040  # 32 key pieces
    assert M.attn_workspace_bytes(16, 2, 64, 64) == 64 * 16 * 1 * 1032                # decode kernels, 1 split
    assert M.attn_workspace_bytes(16, 2, 40000, 256) == 2 * 1250 * 37632 + 256 * 16 * 16 * 1040  # 16 pieces
    assert M.attn_workspace_bytes(12, 2, 1000, 64) == 0                            # not a GQA-8 shape
    assert M.workspace_held() == 0
