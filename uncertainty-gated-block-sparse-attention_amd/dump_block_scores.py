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

MODE_LABELS = {0: "topk", 1: "router_mean", 2: "router_quest", 3: "quest", 4: "other"}


def _mode_id(sel) -> int:
    """The shard's policy code: 0 topk, 1 router on K-mean, 2 router on Quest,
    3 quest, anything else 4 (src/dump_block_scores.py:210-219)."""
    codes = {("topk", False): 0, ("router", False): 1, ("router", True): 2}
    if sel.mode == "quest":
        return 3
    return codes.get((sel.mode, sel.mode == "router" and sel.router_score == "quest"), 4)


class _DumpSession:
    """One recording session: the selector it wraps, the shards recorded so
    far and where they go.  Only one session is active at a time."""

    def __init__(self, out_path, inner):
        self.out_path = out_path
        self.inner = inner          # the selector function that was bound before
        self.shards = []
        self.calls = 0              # selection calls seen (recorded or not)
        self.active = True          # False once torn down: the recorder only forwards

    def selector(self, query, key_states, scaling, block_m=64):
        """Stands in for ``sparse_attention._block_select_kv_idx_v2``: runs the
        wrapped selector, then records a shard beside it.  The selection is
        returned untouched; a recording failure is printed, not raised."""
        kv_idx = self.inner(query, key_states, scaling, block_m=block_m)
        if not self.active:
            return kv_idx
        try:
            shard = record(query, key_states, scaling, block_m)
        except Exception as err:   # the prefill must go on
            print(f"[dump_block_scores] call {self.calls}: no shard ({type(err).__name__}: {err})",
                  flush=True)
        else:
            if shard is not None:
                shard["call_idx"] = self.calls
                self.shards.append(shard)
        self.calls += 1
        return kv_idx

    def write(self):
        if not self.shards or self.out_path is None:
            return
        with open(self.out_path, "wb") as fh:
            pickle.dump(self.shards, fh, protocol=pickle.HIGHEST_PROTOCOL)
        cells = sum(int(sh["g"].size) for sh in self.shards)
        print(f"[dump_block_scores] {len(self.shards)} shards, {cells} (B,H,Qt) cells -> "
              f"{self.out_path}", flush=True)


_session: _DumpSession | None = None


def install_dump_hook(out_path):
    """Start recording: rebind ``sparse_attention._block_select_kv_idx_v2``
    (the dispatcher looks the name up at call time) to a recorder around the
    current selector (src/dump_block_scores.py:57-71).  While a session is
    active, another install changes nothing."""
    global _session
    if _session is not None:
        print(f"[dump_block_scores] a session writing to {_session.out_path} is active; "
              f"not installing another for {out_path}", flush=True)
        return
    _session = _DumpSession(out_path, sparse_attention._block_select_kv_idx_v2)
    sparse_attention._block_select_kv_idx_v2 = _session.selector
    print(f"[dump_block_scores] recording selection calls for {out_path}", flush=True)


def flush_and_teardown():
    """End the session: bind the selector back and write the shards as one
    pickled list (src/dump_block_scores.py:74-89).  No-op without a session."""
    global _session
    if _session is None:
        return
    session, _session = _session, None
    session.active = False
    sparse_attention._block_select_kv_idx_v2 = session.inner
    session.write()


def dump_budgets(budget_blocks, n_blocks):
    """(k_b, rho_k): min(2 * budget_blocks, NB) — without the selector's
    k_min / k_max clamp — and min(2 * k_b, NB) (:150-151)."""
    k_b = min(2 * int(budget_blocks), n_blocks)
    return k_b, min(2 * k_b, n_blocks)


def record(query, key_states, scaling, block_m=64, sel=None, want_tile_score=False):
    """One shard (without ``call_idx``) for a selection call, or None where
    the reference records nothing: no room for a g_rho gap (rho_k <= k_b) or
    no tile with more than rho_k visible blocks (:152-158).

    ``query`` [B, H, M, D] bf16 or fp16 on the GPU; ``key_states`` [B, H, N, D]
    (repeat_kv'd) or [B, Hk, N, D].  Synchronises to copy the shard to the
    host, as the reference does.  ``want_tile_score`` adds the unforced
    ``tile_score`` [B, H, Qt, NB] (a tensor) for tests.
    """
    sel = sparse_attention.SEL if sel is None else sel
    assert block_m == BLOCK, "selection tiles are 64 rows"
    assert query.is_cuda, "HIP query required"
    _capi.dtype_code(query.dtype)                     # bf16 or fp16, as the model runs
    assert key_states.dtype == query.dtype and key_states.device == query.device
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
                                     B, H, Hk, M, N, D, _capi.dtype_code(query.dtype), mode, float(scaling),
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
