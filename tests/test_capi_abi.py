"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching the device."""

import ctypes
import os
import re

import pytest

import _capi
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ugbsa.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int)\s+(ugbsa_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_capi.LIB_PATH):
        pytest.fail("libugbsa.so is not built (run __graft_entry__.build())")
    return _capi.lib()


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_capi.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_capi.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(raw, name), name
    assert lib.ugbsa_abi_version() == _capi.ABI_VERSION


def test_size_queries(lib):
    # Quest [B, Hk, NB, 2, D]: c3 = 1 * 4 * 2048 * 2 * 128; mean: the two fp16
    # planes, then one fp32 scale (two 16-bit elements) per block
    assert lib.ugbsa_summary_elems(1, 4, 131072, 128, _capi.MODE_QUEST) == 4 * 2048 * 2 * 128
    assert lib.ugbsa_summary_elems(1, 2, 1000, 64, _capi.MODE_MEAN) == 2 * 16 * (2 * 64 + 2)
    # K and V operand copies, then the tile schedule (2 * B * NB int32 = 4 * B * NB bf16,
    # rounded to 16 bytes)
    assert lib.ugbsa_attn_workspace_elems(1, 4, 1000, 128) == 2 * 4 * 16 * 64 * 128 + 64
    assert lib.ugbsa_attn_workspace_elems(2, 2, 131072, 256) == 2 * 2 * 2 * 2048 * 64 * 256 + 4 * 2 * 2048


def test_argument_errors_are_reported_without_launch(lib):
    # null q, odd dtype, bad head split: rejected on the host (UGBSA_EARG/EDTYPE)
    rc = lib.ugbsa_select(None, 0, 0, 0, 1, None, 1, 8, 2, 64, 64, 128, _capi.DTYPE_BF16,
                          _capi.MODE_QUEST, 0.1, 1, 1, 64, None, None, None, None)
    assert rc == -1 and b"null" in lib.ugbsa_last_error()
    rc = lib.ugbsa_block_summary(16, 0, 0, 8, 1, 1, 1, 64, 128, 7, _capi.MODE_MEAN, 16, None)
    assert rc == -3
    rc = lib.ugbsa_block_summary(16, 0, 0, 8, 1, 1, 1, 64, 96, _capi.DTYPE_BF16, _capi.MODE_MEAN, 16, None)
    assert rc == -1 and b"head_dim" in lib.ugbsa_last_error()
    # the summary buffer (whose mean scales are fp32) must be 16-byte aligned
    rc = lib.ugbsa_block_summary(16, 0, 0, 8, 1, 1, 1, 64, 128, _capi.DTYPE_BF16, _capi.MODE_MEAN, 18, None)
    assert rc == -2 and b"planes" in lib.ugbsa_last_error()
    rc = lib.ugbsa_attn_fwd(16, 0, 0, 8, 2, 16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 0, 1,
                            1, 8, 2, 64, 64, 128, _capi.DTYPE_BF16, 1, 1, 64, 0.1,
                            16, 0, 0, 8, 1, 16, 1 << 40, None)
    assert rc == -2 and b"stride" in lib.ugbsa_last_error()
    # a zero or non-finite softmax scale is rejected before any launch
    for bad in (0.0, float("inf"), float("nan")):
        rc = lib.ugbsa_attn_fwd(16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 0, 1,
                                1, 8, 2, 64, 64, 128, _capi.DTYPE_BF16, 1, 1, 64, bad,
                                16, 0, 0, 8, 1, 16, 1 << 40, None)
        assert rc == -1 and b"scale" in lib.ugbsa_last_error(), bad
    rc = lib.ugbsa_router(16, 1, 8, 4, _capi.GRAIN_ROW, _capi.ROUTER_QUANTILE, 0.1, 0, 16,
                          4, 8, 16, 16, 16, None, None)
    assert rc == -1 and b"k_quant" in lib.ugbsa_last_error()
    with pytest.raises(AssertionError):
        _capi.check(rc, "router")
    # one-shot prefill: query length must equal key length
    rc = lib.ugbsa_select(16, 0, 0, 8, 1, 16, 1, 8, 2, 64, 128, 128, _capi.DTYPE_BF16,
                          _capi.MODE_QUEST, 0.1, 1, 1, 64, 16, None, None, None)
    assert rc == -1 and b"query length" in lib.ugbsa_last_error()
    rc = lib.ugbsa_attn_fwd(16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 0, 1,
                            1, 8, 2, 64, 128, 128, _capi.DTYPE_BF16, 1, 1, 64, 0.1,
                            16, 0, 0, 8, 1, 16, 1 << 40, None)
    assert rc == -1 and b"query length" in lib.ugbsa_last_error()
    # a workspace smaller than ugbsa_attn_workspace_elems (K/V copies + tile
    # schedule) is rejected before any launch, by both attention entry points
    # and, below the K/V copies, by the preparation
    need = lib.ugbsa_attn_workspace_elems(1, 2, 64, 128)
    rc = lib.ugbsa_attn_fwd(16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 0, 1,
                            1, 8, 2, 64, 64, 128, _capi.DTYPE_BF16, 1, 1, 64, 0.1,
                            16, 0, 0, 8, 1, 16, need - 1, None)
    assert rc == -1 and b"workspace" in lib.ugbsa_last_error()
    rc = lib.ugbsa_attn_fwd_rows(16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 16, 16, 0, 0, 0,
                                 1, 1, 8, 2, 64, 64, 128, _capi.DTYPE_BF16, 1, 1, 64, 0.1,
                                 16, 0, 0, 8, 1, 16, need - 1, None)
    assert rc == -1 and b"workspace" in lib.ugbsa_last_error()
    copies = 2 * 2 * 1 * 64 * 128
    rc = lib.ugbsa_attn_prepare_kv(16, 0, 0, 8, 1, 16, 0, 0, 8, 1, 1, 2, 64, 128,
                                   _capi.DTYPE_BF16, 64, 16, copies - 1, None)
    assert rc == -1 and b"workspace" in lib.ugbsa_last_error()
    # the static-scratch selector refuses shapes whose one-tile pass exceeds its 2^24 fp32
    rc = lib.ugbsa_select_mask_static(16, 0, 0, 8, 1, 16, 1, 128, 2, 4096 * 64, 4096 * 64, 128,
                                      _capi.DTYPE_BF16, _capi.MODE_QUEST, 0.1, _capi.V1_TOPK, 4,
                                      0, 1, 112, 0.9, None, 16, None, None)
    assert rc == -1 and b"static scratch" in lib.ugbsa_last_error()
    # score dump: rho_k must stay below NB (the reference indexes s(rho_k))
    rc = lib.ugbsa_score_dump(16, 0, 0, 8, 1, 16, 1, 8, 2, 256, 256, 128, _capi.DTYPE_BF16,
                              _capi.MODE_QUEST, 0.1, 2, 4, 16, 16, 16, 16, 16, 16, None, None)
    assert rc == -1 and b"rho_k" in lib.ugbsa_last_error()
