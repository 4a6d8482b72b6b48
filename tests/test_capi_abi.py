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


def declared_prototypes():
    """{name: (return C type, [parameter C types])} from the header's declarations."""
    text = re.sub(r"/\*.*?\*/", " ", open(HEADER).read(), flags=re.S)
    protos = {}
    for ret, name, params in re.findall(
            r"^\s*(const char\*|int64_t|int)\s+(ugbsa_\w+)\(([^)]*)\);", text, re.M):
        params = " ".join(params.split())
        types = []
        if params not in ("", "void"):
            for p in params.split(","):
                # drop the parameter name: the type is everything before it
                types.append(re.sub(r"\s*\b\w+$", "", p.strip()).replace(" *", "*"))
        protos[name] = (ret, types)
    return protos


def _ctype_of(c_type):
    if c_type.endswith("*"):
        return ctypes.c_char_p if c_type == "const char*" else ctypes.c_void_p
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float}[c_type]


def test_binding_signatures_match_header_prototypes():
    # every argument of every entry point has the ctypes class of its C type:
    # an argument added, dropped or retyped on one side fails here on the CPU
    protos = declared_prototypes()
    assert sorted(protos) == declared_symbols()
    for name, (ret, params) in protos.items():
        res, args = _capi.SIGNATURES[name]
        assert res is _ctype_of(ret), (name, ret, res)
        assert len(args) == len(params), (name, len(args), len(params))
        for i, (c_type, a) in enumerate(zip(params, args)):
            want = ctypes.c_void_p if c_type.endswith("*") else _ctype_of(c_type)
            assert a is want, (name, i, c_type, a)


def test_prototype_parser_sees_a_planted_mismatch():
    # the check above rests on the parser: a binding with one argument too few
    # or one 32-bit integer where the header has int64_t must not pass
    protos = declared_prototypes()
    ret, params = protos["ugbsa_attn_workspace_elems"]
    assert ret == "int64_t" and params == ["int"] * 4
    ret, params = protos["ugbsa_router"]
    assert params[7] == "int64_t" and params[0].endswith("*")
    res, args = _capi.SIGNATURES["ugbsa_router"]
    bad = list(args)
    bad[7] = ctypes.c_int
    assert bad[7] is not (ctypes.c_void_p if params[7].endswith("*") else _ctype_of(params[7]))
    assert len(args[:-1]) != len(params)


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
