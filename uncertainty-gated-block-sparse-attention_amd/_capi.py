"""ctypes binding of libugbsa (include/ugbsa.h) — the only route to the kernels.

There is deliberately no CPU or eager-torch fallback: if the shared library
is missing or fails to load, every entry point raises.  Build it with
``python __graft_entry__.py`` (or ``__graft_entry__.build()``) from the
repository root.

Error mapping (mirrors the reference's behaviour): argument and layout
errors raise ``AssertionError`` — the reference asserts shapes / dtype /
device in ``src/triton_block_attn.py:276-277``; HIP launch failures raise
``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os

import torch

LIB_NAME = "libugbsa.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DTYPE_BF16, DTYPE_F16 = 0, 1
MODE_MEAN, MODE_QUEST = 0, 1
GRAIN_CELL, GRAIN_ROW = 0, 1
ROUTER_ABS, ROUTER_QUANTILE = 0, 1
V1_TOPK, V1_BELIEF = 0, 1

# Every symbol include/ugbsa.h declares, with its ctypes signature.
_i, _i64, _f, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
SIGNATURES = {
    "ugbsa_abi_version": (_i, []),
    "ugbsa_last_error": (ctypes.c_char_p, []),
    "ugbsa_summary_elems": (_i64, [_i, _i, _i, _i, _i]),
    "ugbsa_block_summary": (_i, [_p, _i64, _i64, _i64, _i64, _i, _i, _i, _i, _i, _i, _p, _p]),
    "ugbsa_select": (_i, [_p, _i64, _i64, _i64, _i64, _p, _i, _i, _i, _i, _i, _i, _i, _i,
                          _f, _i, _i, _i, _p, _p, _p, _p]),
    "ugbsa_score_dump": (_i, [_p, _i64, _i64, _i64, _i64, _p, _i, _i, _i, _i, _i, _i, _i, _i,
                              _f, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p]),
    "ugbsa_router": (_i, [_p, _i, _i, _i, _i, _i, _f, _i64, _p, _i, _i, _i, _p, _p, _p, _p]),
    "ugbsa_select_mask_workspace_elems": (_i64, [_i, _i, _i, _i]),
    "ugbsa_select_mask": (_i, [_p, _i64, _i64, _i64, _i64, _p, _i, _i, _i, _i, _i, _i, _i, _i,
                               _f, _i, _i, _i, _i, _i, _f, _p, _p, _i64, _p, _p, _p]),
    "ugbsa_select_mask_static": (_i, [_p, _i64, _i64, _i64, _i64, _p, _i, _i, _i, _i, _i, _i,
                                      _i, _i, _f, _i, _i, _i, _i, _i, _f, _p, _p, _p, _p]),
    "ugbsa_router_rows": (_i, [_p, _i, _i, _i, _i, _i, _i, _f, _i64, _i, _p, _p, _p, _p, _p]),
    "ugbsa_keep_kv_idx": (_i, [_p, _i, _i, _i, _i, _i, _p, _p, _p, _p]),
    "ugbsa_attn_fwd_rows": (_i, [_p, _i64, _i64, _i64, _i64,
                                 _p, _i64, _i64, _i64, _i64,
                                 _p, _i64, _i64, _i64, _i64,
                                 _p, _p, _i64, _i64, _i64, _i64,
                                 _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _f,
                                 _p, _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "ugbsa_attn_workspace_elems": (_i64, [_i, _i, _i, _i]),
    "ugbsa_attn_prepare_kv": (_i, [_p, _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64,
                                   _i, _i, _i, _i, _i, _i, _p, _i64, _p]),
    "ugbsa_attn_fwd": (_i, [_p, _i64, _i64, _i64, _i64,
                            _p, _i64, _i64, _i64, _i64,
                            _p, _i64, _i64, _i64, _i64,
                            _p, _i64, _i64, _i64, _i64,
                            _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _f,
                            _p, _i64, _i64, _i64, _i64, _p, _i64, _p]),
}
ABI_VERSION = 4

_LIB = None


def lib():
    """Load libugbsa once; raise loudly if it is absent or stale."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} not found: the HIP extension is not built "
                "(run __graft_entry__.build()); there is no fallback path")
        h = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        if h.ugbsa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} ABI {h.ugbsa_abi_version()} != {ABI_VERSION}; rebuild")
        _LIB = h
    return _LIB


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = lib().ugbsa_last_error().decode(errors="replace")
    if rc < 0:
        raise AssertionError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {rc}: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    """The C ABI's element-format code of a 16-bit torch dtype; the kernels
    run in the caller's dtype as the reference does, bf16 or fp16."""
    assert dtype in (torch.bfloat16, torch.float16), f"bf16 or fp16 required, got {dtype}"
    return DTYPE_F16 if dtype == torch.float16 else DTYPE_BF16


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
