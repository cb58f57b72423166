"""The C-ABI library loads, exports every symbol include/art_moe.h declares, and
rejects bad arguments on the host (no GPU work is launched by these calls)."""
import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "art_moe.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(art_moe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from art_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail("libart_moe.so not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_expected_entry_points():
    names = _declared()
    assert "art_moe_grouped_gemm" in names and "art_moe_dispatch_plan" in names
    assert len(names) >= 15


def test_every_declared_symbol_is_exported_and_bound(lib):
    from art_amd import _lib
    names = _declared()
    for n in names:
        assert hasattr(lib, n), f"{n} missing from libart_moe.so"
    assert sorted(_lib.SIGNATURES) == names, "ctypes signatures out of sync with the header"


def test_host_only_queries(lib):
    assert lib.art_moe_version() == 100
    assert lib.art_moe_dgrad_swiglu_parts(768) == 6
    assert lib.art_moe_plan_workspace_bytes(8192, 128) >= 128 * 128 * 16
    assert lib.art_moe_plan_workspace_bytes(-1, 128) == 0


def test_invalid_arguments_are_rejected_before_launch(lib):
    from art_amd import _lib
    null = None
    rc = lib.art_moe_router_topk(null, 4, 0, 2, null, null, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG
    assert b"E <= 1024" in lib.art_moe_last_error()
    rc = lib.art_moe_router_topk(null, 4, 8, 9, null, null, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG
    rc = lib.art_moe_router_replay_rows(null, null, 0, null, 0, null, 4, 4, 8, null, null, null,
                                        null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"min(E, 32)" in lib.art_moe_last_error()
    rc = lib.art_moe_router_replay_rows(null, null, 0, null, 0, null, 4, 8, 2, null, null, null,
                                        null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"null pointer" in lib.art_moe_last_error()
    rc = lib.art_moe_grouped_gemm(null, 12, null, null, null, 12, 0, null, 0, 0, null, 0, null, 0,
                                  0, 0, null, 4, 16, 32, 12, 1.0, null, 32, 0, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG
    assert b"multiple of 16" in lib.art_moe_last_error()
    rc = lib.art_moe_fc1_swiglu(null, 64, null, null, null, null, 0, null, 0, null, 0, null, 4, 16,
                                100, 64, null, null, null, null, 0, 0, 0, null, 0, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG
    # fused LoRA projection: partial count of the active tile configuration
    assert lib.art_moe_lora_epilogue_parts(0, 768, _lib.B_BF16) == 6
    assert lib.art_moe_lora_epilogue_parts(1, 768, _lib.B_BF16) == 3
    assert lib.art_moe_lora_epilogue_parts(2, 768, _lib.B_BF16) == 0
    rc = lib.art_moe_sum_parts(null, 0, 16, 16, null, 0, null, 16, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"n_parts >= 1" in lib.art_moe_last_error()
    # fp8 weights: K must be a multiple of 64 (checked before any pointer is used)
    buf = ctypes.create_string_buffer(4096 + 16)
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    rc = lib.art_moe_grouped_gemm(base, 48, null, null, base, 48, 0, base, 64, _lib.B_FP8_ROWSCALE,
                                  null, 0, null, 0, 0, 0, base, 4, 16, 32, 48, 1.0, base, 32, 0,
                                  null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"multiple of 64" in lib.art_moe_last_error()
    # fp8 activations (W8A8): row scales required; A row scales only with fp8 A
    rc = lib.art_moe_grouped_gemm(base, 64, null, null, base, 64, 0, null, 0, _lib.AB_FP8,
                                  null, 0, null, 0, 0, 0, base, 4, 16, 32, 64, 1.0, base, 32, 0,
                                  null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"row scales" in lib.art_moe_last_error()
    rc = lib.art_moe_grouped_gemm(base, 64, null, base, base, 64, 0, null, 0, _lib.B_BF16,
                                  null, 0, null, 0, 0, 0, base, 4, 16, 32, 64, 1.0, base, 32, 0,
                                  null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"AB_FP8" in lib.art_moe_last_error()
    rc = lib.art_moe_quantize_rows_fp8(base, 12, null, null, 0, null, 0, 4, 12, base, 12, base,
                                       null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"K % 8" in lib.art_moe_last_error()
    rc = lib.art_moe_permute(null, null, 4, 2, 12, null, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG
    rc = lib.art_moe_grouped_wgrad(null, 64, null, null, 64, null, null, 4, 100, 64, 12, 1.0,
                                   null, 0, 0, 0, null, 0, 0, 0, 0, 0, null, 0, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG
    assert lib.art_moe_wgrad_workspace_bytes(2048, 128, 2048, 32) == 0
    assert lib.art_moe_wgrad_workspace_bytes(65536, 128, 2048, 32) == (32 + 128) * 2048 * 32 * 4
    rc = lib.art_moe_router_lora_grad(null, null, 8, 8, null, 512, 128, 1.0, null, null, null)
    assert rc == _lib.ART_MOE_ERR_INVALID_ARG and b"(r + 2) * E" in lib.art_moe_last_error()


def test_python_call_raises_valueerror(lib):
    from art_amd import _lib
    with pytest.raises(ValueError, match="router_topk"):
        _lib.call("art_moe_router_topk", None, 4, 0, 2, None, None, None)
