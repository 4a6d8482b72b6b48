"""Score-dump diagnostic of the block selector, computed on MI355X.

Drop-in for the reference's ``src/dump_block_scores.py``: the same
``install_dump_hook(out_path)`` / ``flush_and_teardown()`` API, the same
module-global rebinding of ``sparse_attention._block_select_kv_idx_v2``
(the dispatcher looks that name up at call time), the same shard format and
pickle file::

    {"call_idx": int, "n_blocks": int, "mode_id": int, "budget_blocks": int,
     "g": [B, H, Qt] f32, "r": [B, H, Qt] f32, "sigma": [B, H, Qt] f32,
     "g_rho": [B, H, Qt] f32, "valid": [Qt] bool, "tau_hat": [B, H] f32}

``record`` computes a shard with ``ugbsa_score_dump``: kernel 2 in dump mode
ranks the unforced tile scores rho_k + 1 deep and writes the order-statistic
gaps, and a reduction kernel forms the per-head noise estimate tau_hat — the
per-row score tensor the reference materialises (``[B, H, Qt*64, NB]``) is
never built.  Semantics follow src/dump_block_scores.py:104-207; the selector
output passes through unchanged, and a failure to record is reported and
never raised into the prefill (:92-101).
"""

from __future__ import annotations

import pickle

import torch

import _capi
import sparse_attention

BLOCK = sparse_attention.BLOCK

_STATE = {
    "enabled": False,
    "out_path": None,
    "orig_fn": None,
    "shards": [],
    "call_idx": 0,
}

MODE_LABELS = {0: "topk", 1: "router_mean", 2: "router_quest", 3: "quest", 4: "other"}


def _mode_id(sel) -> int:
    """0=topk, 1=router-mean, 2=router-quest, 3=quest, 4=other (:210-219)."""
    if sel.mode == "topk":
        return 0
    if sel.mode == "router":
        return 2 if sel.router_score == "quest" else 1
    if sel.mode == "quest":
        return 3
    return 4


def install_dump_hook(out_path):
    """Wrap ``sparse_attention._block_select_kv_idx_v2`` so each call records
    one shard (:57-71).  A second install is a no-op."""
    if _STATE["enabled"]:
        print(f"[dump_block_scores] already installed (out={_STATE['out_path']}); "
              f"ignoring install with out={out_path}", flush=True)
        return
    _STATE.update(orig_fn=sparse_attention._block_select_kv_idx_v2, out_path=out_path,
                  shards=[], call_idx=0, enabled=True)
    sparse_attention._block_select_kv_idx_v2 = _wrapped
    print(f"[dump_block_scores] installed, dumping to {out_path}", flush=True)


def flush_and_teardown():
    """Restore the selector and write the shards to ``out_path`` (:74-80)."""
    if not _STATE["enabled"]:
        return
    sparse_attention._block_select_kv_idx_v2 = _STATE["orig_fn"]
    _STATE["enabled"] = False
    _flush()


def _flush():
    if not _STATE["shards"] or _STATE["out_path"] is None:
        return
    with open(_STATE["out_path"], "wb") as f:
        pickle.dump(_STATE["shards"], f, protocol=pickle.HIGHEST_PROTOCOL)
    n_tiles = sum(s["g"].size for s in _STATE["shards"])
    print(f"[dump_block_scores] wrote {len(_STATE['shards'])} calls "
          f"({n_tiles} (B,H,Qt) cells) → {_STATE['out_path']}", flush=True)


def _wrapped(query, key_states, scaling, block_m=64):
    out = _STATE["orig_fn"](query, key_states, scaling, block_m=block_m)
    if _STATE["enabled"]:
        try:
            shard = record(query, key_states, scaling, block_m)
            if shard is not None:
                shard["call_idx"] = _STATE["call_idx"]
                _STATE["shards"].append(shard)
        except Exception as e:   # never crash the prefill
            print(f"[dump_block_scores] WARN record failed at call "
                  f"{_STATE['call_idx']}: {type(e).__name__}: {e}", flush=True)
        _STATE["call_idx"] += 1
    return out


def dump_budgets(budget_blocks, n_blocks):
    """(k_b, rho_k): min(2 * budget_blocks, NB) — without the selector's
    k_min / k_max clamp — and min(2 * k_b, NB) (:150-151)."""
    k_b = min(2 * int(budget_blocks), n_blocks)
    return k_b, min(2 * k_b, n_blocks)


def record(query, key_states, scaling, block_m=64, sel=None, want_tile_score=False):
    """One shard (without ``call_idx``) for a selection call, or None where
    the reference records nothing: no room for a g_rho gap (rho_k <= k_b) or
    no tile with more than rho_k visible blocks (:152-158).

    ``query`` [B, H, M, D] bf16 on the GPU; ``key_states`` [B, H, N, D]
    (repeat_kv'd) or [B, Hk, N, D].  Synchronises to copy the shard to the
    host, as the reference does.  ``want_tile_score`` adds the unforced
    ``tile_score`` [B, H, Qt, NB] (a tensor) for tests.
    """
    sel = sparse_attention.SEL if sel is None else sel
    assert block_m == BLOCK, "selection tiles are 64 rows"
    assert query.is_cuda and query.dtype == torch.bfloat16, "bf16 HIP query required"
    assert key_states.dtype == torch.bfloat16 and key_states.device == query.device
    B, H, M, D = query.shape
    Hk, N = key_states.shape[1], key_states.shape[2]
    assert key_states.shape[0] == B and key_states.shape[3] == D and H % Hk == 0
    nb = (N + BLOCK - 1) // BLOCK
    qt = (M + block_m - 1) // block_m
    k_b, rho_k = dump_budgets(sel.budget_blocks, nb)
    if rho_k <= k_b:
        return None
    last_vis = min((qt - 1) * block_m + block_m - 1, N - 1) // BLOCK + 1   # most visible blocks
    if last_vis <= rho_k:
        return None
    dev = query.device
    lib = _capi.lib()
    mode = _capi.MODE_QUEST if sparse_attention.use_quest(sel) else _capi.MODE_MEAN
    planes = sparse_attention.block_summary(key_states, mode)
    query = sparse_attention._contig_rows(query)
    f32 = dict(dtype=torch.float32, device=dev)
    g, r, sigma, g_rho = (torch.empty(B, H, qt, **f32) for _ in range(4))
    valid = torch.empty(qt, dtype=torch.uint8, device=dev)
    tau = torch.empty(B, H, **f32)
    ts = torch.empty(B, H, qt, nb, **f32) if want_tile_score else None
    _capi.check(lib.ugbsa_score_dump(query.data_ptr(), *query.stride(), planes.data_ptr(),
                                     B, H, Hk, M, N, D, _capi.DTYPE_BF16, mode, float(scaling),
                                     k_b, rho_k, g.data_ptr(), r.data_ptr(), sigma.data_ptr(),
                                     g_rho.data_ptr(), valid.data_ptr(), tau.data_ptr(),
                                     _capi.ptr(ts), _capi.stream_ptr(dev)),
                "score dump")
    shard = {"n_blocks": int(nb), "mode_id": _mode_id(sel),
             "budget_blocks": int(sel.budget_blocks),
             "g": g.cpu().numpy(), "r": r.cpu().numpy(), "sigma": sigma.cpu().numpy(),
             "g_rho": g_rho.cpu().numpy(), "valid": valid.cpu().numpy().astype(bool),
             "tau_hat": tau.cpu().numpy()}
    if want_tile_score:
        shard["tile_score"] = ts
    return shard
