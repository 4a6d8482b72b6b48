"""Block-sparse prefill attention selector + HF dispatch on MI355X.

Drop-in for the v2 path of the reference's ``src/sparse_attention.py``: the
same module-level ``SEL`` / ``PROF`` objects and field names, the same
``_block_select_kv_idx_v2(query, key_states, scaling, block_m=64)`` and
``block_sparse_attention(module, query, key, value, attention_mask, scaling,
dropout=0.0, **kwargs)`` signatures, and the same
``AttentionInterface.register("block_sparse", ...)`` at import.  Selection and
attention run in hand-written gfx950 HIP kernels through ``_capi``:

  kernel 1  ugbsa_block_summary  K-block mean / (min, max)        (:618-646)
  kernel 2  ugbsa_select         scores, tile max, mask, forcing,
                                 top-k, sigma                      (:638-707)
  router    ugbsa_router         row mean, quantile / abs, sentinels (:708-725)
  kernel 3  ugbsa_attn_fwd       block-sparse attention            (triton_block_attn.py)

Everything is asynchronous on the current stream; like the reference, the v2
path syncs the host only when ``SEL.log`` asks for diagnostics.

Differences from the reference, by design:

* Scores are fp32 (bf16 or fp16 inputs — the model's dtype — with fp32 MFMA
  accumulation) rather than rounded to the model dtype, and ``topk`` ties are
  broken by block index (the reference leaves the order unspecified).
  ``kv_idx`` therefore equals the reference selector run on fp32 scores.
* The dispatcher hands the selector and the kernel the un-repeated
  ``[B, Hk, N, D]`` key/value tensors (GQA handled in-kernel) instead of
  ``repeat_kv`` copies; ``_block_select_kv_idx_v2`` accepts either.
* The v1 per-row path (``kernel_v2=False``, and the belief / rollout modes)
  runs on the GPU too: ``_block_select_mask`` (:208-382) through
  ``ugbsa_select_mask`` + ``ugbsa_router_rows`` and ``block_sparse_attn``
  through ``ugbsa_attn_fwd_rows``.  Its keep mask follows the same total tie
  order, so rows with fewer visible blocks than the budget keep the lowest
  invisible blocks (the reference keeps arbitrary ones; attention never
  reads them).
* ``rollout_peek`` (:386-583) is not provided: it is an abandoned research
  mode of the reference, off its v2 path (a depth-1 forward of the model per
  candidate block set).  The dispatcher raises ``NotImplementedError`` for it.
* The sparse branches need one-shot prefill, query length == key length, as
  the reference's launchers assert (``q.shape == k.shape``); a query shorter
  than the keys (a prefill continuing a cache) raises ``AssertionError``
  instead of attending with unshifted positions.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

import _capi
from block_attn import attn_workspace, block_sparse_attn, block_sparse_attn_v2

BLOCK = 64   # tokens per selection block (src/sparse_attention.py:51)


class Selector:
    """Global selector configuration + diagnostics (src/sparse_attention.py:54-138).

    Same fields and defaults as the reference.  The v2 path reads ``mode``,
    ``budget_blocks``, ``k_min``/``k_max``, ``router_mode``, ``router_grain``,
    ``router_tau``, ``router_quantile``, ``router_score``, ``kernel_v2`` and
    ``log``; the remaining knobs belong to the v1 / rollout research modes and
    are kept so harness code that sets them keeps working.
    """

    def __init__(self):
        self.mode = "dense"          # "dense"|"topk"|"belief"|"rollout"|"rollout_peek"|"router"|"quest"
        self.budget_blocks = 32
        self.top_p = 0.9
        self.k_min, self.k_max = 8, 112
        self.explore_bonus = 0.3
        self.ema_alpha = 0.3
        self.router_mode = "abs"     # "abs" | "quantile"
        self.router_grain = "cell"   # "cell" | "row"
        self.router_tau = 0.10
        self.router_quantile = 0.20
        self.router_score = "mean"   # "mean" | "quest"
        self.kernel_v2 = False
        self.peek_swap_w = 2
        self.peek_rows_per_layer = 32
        self.peek_layer_min = 0
        self.peek_layer_max = 999
        self.peek_metric = "peakedness"
        self.peek_xh_threshold = 0.5
        self.model_ref = None
        self.hidden_at = {}
        self.k_pool_at = {}
        self.log = False
        self.reset_log()

    def reset_log(self):
        self.kept_blocks = {}
        self.budget_samples = []
        self.selection_history = None
        self.k_pool_at = {}
        self.router_trigger_rate = []
        self.router_eff_budget = []
        self.router_margin_mean = []


SEL = Selector()


class _Profiler:
    """Event profiler for block_sparse_attention internals (src/sparse_attention.py:141-183).

    Opt-in (``PROF.enabled = True``); buckets ``dense_sdpa``, ``v2_select``,
    ``v2_kernel``; ``summary()`` synchronises and returns calls / total / mean /
    p50 ms per bucket.  Events are HIP events on the current stream.
    """

    def __init__(self):
        self.enabled = False
        self.events = {}

    def reset(self):
        self.events = {}

    def start(self, name):
        if not self.enabled or not torch.cuda.is_available():
            return None
        ev_s = torch.cuda.Event(enable_timing=True)
        ev_e = torch.cuda.Event(enable_timing=True)
        ev_s.record()
        self.events.setdefault(name, []).append((ev_s, ev_e))
        return ev_e

    @staticmethod
    def stop(ev_e):
        if ev_e is not None:
            ev_e.record()

    def summary(self):
        if not self.events:
            return {}
        torch.cuda.synchronize()
        out = {}
        for name, ev_list in self.events.items():
            ms = sorted(s.elapsed_time(e) for s, e in ev_list)
            out[name] = {"calls": len(ms), "total_ms": sum(ms),
                         "mean_ms": sum(ms) / len(ms), "p50_ms": ms[len(ms) // 2]}
        return out


PROF = _Profiler()


def budgets(n_blocks: int, sel: Selector = None):
    """(k_base, k_slots) of the v2 selector — src/sparse_attention.py:688-695."""
    sel = SEL if sel is None else sel
    k_row = int(max(min(sel.k_max, sel.budget_blocks), sel.k_min))
    k_base = min(2 * k_row, n_blocks)
    k_slots = min(2 * k_base, n_blocks) if sel.mode == "router" else k_base
    return k_base, k_slots


@dataclass
class SelectionResult:
    kv_idx: torch.Tensor                 # int32 [B, H, Qt, k_slots]
    k_base: int
    k_slots: int
    sigma: torch.Tensor | None = None     # fp32 [B, H, Qt] per-cell margin
    sigma_eff: torch.Tensor | None = None  # after the row-grain mean
    uncertain: torch.Tensor | None = None  # uint8 [B, H, Qt]
    threshold: torch.Tensor | None = None  # fp32 [1]
    tile_score: torch.Tensor | None = None  # fp32 [B, H, Qt, NB] (if asked)


def select_v2(query, key_states, scaling, block_m=64, sel: Selector = None,
              want_tile_score=False) -> SelectionResult:
    """Run kernels 1, 2 and the router; return kv_idx plus the router state."""
    sel = SEL if sel is None else sel
    assert block_m == BLOCK, "selection tiles are 64 rows"
    assert query.shape[-2] == key_states.shape[-2], (
        "query length must equal key length (one-shot prefill: tile t sees blocks <= t)")
    assert query.is_cuda, "HIP query required"
    _capi.dtype_code(query.dtype)                     # bf16 or fp16, as the model runs
    assert key_states.dtype == query.dtype and key_states.device == query.device
    B, H, M, D = query.shape
    Hk, N = key_states.shape[1], key_states.shape[2]
    assert key_states.shape[0] == B and key_states.shape[3] == D and H % Hk == 0
    dev = query.device
    lib = _capi.lib()
    stream = _capi.stream_ptr(dev)
    query = _contig_rows(query)
    key_states = _contig_rows(key_states)
    n_blocks = (N + BLOCK - 1) // BLOCK
    q_tiles = (M + block_m - 1) // block_m
    k_base, k_slots = budgets(n_blocks, sel)
    mode = _capi.MODE_QUEST if use_quest(sel) else _capi.MODE_MEAN

    planes = block_summary(key_states, mode)
    is_router = sel.mode == "router" and k_base < k_slots
    kv_idx = torch.empty(B, H, q_tiles, k_slots, dtype=torch.int32, device=dev)
    sigma = torch.empty(B, H, q_tiles, dtype=torch.float32, device=dev) if is_router else None
    tile_score = (torch.empty(B, H, q_tiles, n_blocks, dtype=torch.float32, device=dev)
                  if want_tile_score else None)
    _capi.check(lib.ugbsa_select(query.data_ptr(), *query.stride(), planes.data_ptr(),
                                 B, H, Hk, M, N, D, _capi.dtype_code(query.dtype), mode, float(scaling),
                                 k_base, k_slots, block_m, kv_idx.data_ptr(),
                                 _capi.ptr(sigma), _capi.ptr(tile_score), stream),
                "select")
    res = SelectionResult(kv_idx, k_base, k_slots, sigma=sigma, tile_score=tile_score)
    if is_router:
        grain = _capi.GRAIN_ROW if sel.router_grain == "row" else _capi.GRAIN_CELL
        rmode = _capi.ROUTER_QUANTILE if sel.router_mode == "quantile" else _capi.ROUTER_ABS
        k_quant = max(1, int(float(sel.router_quantile) * sigma.numel()))
        res.sigma_eff = torch.empty_like(sigma)
        res.uncertain = torch.empty(sigma.shape, dtype=torch.uint8, device=dev)
        res.threshold = torch.empty(1, dtype=torch.float32, device=dev)
        _capi.check(lib.ugbsa_router(sigma.data_ptr(), B, H, q_tiles, grain, rmode,
                                     float(sel.router_tau), k_quant, kv_idx.data_ptr(),
                                     k_base, k_slots, n_blocks, res.sigma_eff.data_ptr(),
                                     res.uncertain.data_ptr(), res.threshold.data_ptr(), stream),
                    "router")
    return res


def block_summary(key_states, mode):
    """Kernel 1: the K-block summaries of ``mode`` (``_capi.MODE_QUEST`` or
    ``_capi.MODE_MEAN``) as one flat buffer in K's dtype, on the current stream:
    Quest [B, Hk, NB, 2, D] (K-max, K-min); mean the fp16 planes [B, Hk, NB, 2, D]
    then the fp32 block scales [B, Hk, NB] (``block_means`` decodes them)."""
    B, Hk, N, D = key_states.shape
    lib = _capi.lib()
    key_states = _contig_rows(key_states)
    planes = torch.empty(lib.ugbsa_summary_elems(B, Hk, N, D, mode), dtype=key_states.dtype,
                         device=key_states.device)
    _capi.check(lib.ugbsa_block_summary(key_states.data_ptr(), *key_states.stride(), B, Hk, N, D,
                                        _capi.dtype_code(key_states.dtype), mode, planes.data_ptr(),
                                        _capi.stream_ptr(key_states.device)),
                "block summary")
    return planes


def block_means(planes, B, Hk, nb, D):
    """The fp32 block means [B, Hk, NB, D] held by a mean summary buffer of
    ``block_summary``: (hi + lo) * 2^-e per block (hi, lo fp16)."""
    n = B * Hk * nb * 2 * D
    hl = planes[:n].view(torch.float16).view(B, Hk, nb, 2, D).float()
    scale = planes[n:n + 2 * B * Hk * nb].view(torch.float32).view(B, Hk, nb, 1)
    return (hl[..., 0, :] + hl[..., 1, :]) * scale


def use_quest(sel: Selector = None) -> bool:
    """Quest backbone iff mode "quest" or router with router_score "quest"
    (src/sparse_attention.py:627-628)."""
    sel = SEL if sel is None else sel
    return sel.mode == "quest" or (sel.mode == "router" and sel.router_score == "quest")


def _contig_rows(t):
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def _block_select_kv_idx_v2(query, key_states, scaling, block_m=64):
    """v2 selection: kv_idx [B, H, Q_tiles, k_slots] int32, built on the GPU.

    Same contract as src/sparse_attention.py:588-748.  ``key_states`` may be
    the repeat_kv'd [B, H, N, D] tensor (as the reference passes) or the GQA
    [B, Hk, N, D] one.
    """
    res = select_v2(query, key_states, scaling, block_m)
    kv_idx = res.kv_idx
    if SEL.log:
        if res.uncertain is not None:
            SEL.router_trigger_rate.append(float(res.uncertain.float().mean().item()))
        n_blocks = (key_states.shape[-2] + BLOCK - 1) // BLOCK
        last = kv_idx[0, :, -1, :].long().flatten()
        last = last[last < n_blocks]
        kept = torch.zeros(n_blocks, dtype=torch.bool, device=kv_idx.device)
        kept.scatter_(0, last, True)
        layer_idx = len(SEL.kept_blocks)
        SEL.kept_blocks[layer_idx] = kept.cpu()
        SEL.budget_samples.append(float(res.k_slots))
    return kv_idx


@dataclass
class MaskResult:
    keep: torch.Tensor                     # bool [B, H, M, NB]
    k_bud: int
    margin: torch.Tensor | None = None     # fp32 [B, H, M] per-cell margin (router)
    margin_eff: torch.Tensor | None = None  # after the row-grain mean
    uncertain: torch.Tensor | None = None  # uint8 [B, H, M]
    threshold: torch.Tensor | None = None  # fp32 [1]
    scores: torch.Tensor | None = None     # fp32 [B, H, M, NB] ranked scores (if asked)


# Largest per-pass row-score buffer of the v1 selector (fp32 elements, 1 GiB).
_V1_WORKSPACE_ELEMS = 1 << 28


def select_mask_v1(query, key_states, scaling, sel: Selector = None, want_scores=False,
                   layer_idx=None) -> MaskResult:
    """v1 per-row selection on the GPU: keep [B, H, M, NB] bool plus the router state.

    src/sparse_attention.py:208-371 (kernels ``ugbsa_select_mask`` and
    ``ugbsa_router_rows``); the rollout history lives in ``sel.selection_history``
    ([H, NB] fp32 on the device) as in the reference.  Needs M == N (one-shot
    prefill, as the reference's kernel assumes).
    """
    sel = SEL if sel is None else sel
    assert query.is_cuda, "HIP query required"
    _capi.dtype_code(query.dtype)                     # bf16 or fp16, as the model runs
    assert key_states.dtype == query.dtype and key_states.device == query.device
    B, H, M, D = query.shape
    Hk, N = key_states.shape[1], key_states.shape[2]
    assert key_states.shape[0] == B and key_states.shape[3] == D and H % Hk == 0
    assert M == N, "the per-row selector needs Q == K (one-shot prefill)"
    dev = query.device
    lib = _capi.lib()
    stream = _capi.stream_ptr(dev)
    query = _contig_rows(query)
    nb = (N + BLOCK - 1) // BLOCK
    mode = _capi.MODE_QUEST if use_quest(sel) else _capi.MODE_MEAN
    planes = block_summary(key_states, mode)
    if mode == _capi.MODE_MEAN and M > 1 and layer_idx is not None:
        # the mean K of each block, repeat_kv'd, cached for later planners (:230-232)
        kp = block_means(planes, B, Hk, nb, D).repeat_interleave(H // Hk, dim=1)
        sel.k_pool_at[layer_idx] = kp.to(query.dtype)
    k_bud = min(int(max(min(sel.k_max, sel.budget_blocks), sel.k_min)), nb)
    router = sel.mode == "router"
    k_eff = max(1, min(int(sel.budget_blocks), nb - 1)) if router else 0
    belief = sel.mode not in ("topk", "router", "rollout", "quest")
    penalty = None
    if sel.mode == "rollout":
        if sel.selection_history is None or tuple(sel.selection_history.shape) != (H, nb):
            sel.selection_history = torch.zeros(H, nb, dtype=torch.float32, device=dev)
        penalty = (float(sel.explore_bonus) * sel.selection_history.float()).contiguous()
    per_tile = B * H * 64 * nb
    full = lib.ugbsa_select_mask_workspace_elems(B, H, M, N)
    ws_elems = full if want_scores else min(full, max(per_tile, _V1_WORKSPACE_ELEMS // per_tile * per_tile))
    ws = torch.empty(ws_elems, dtype=torch.float32, device=dev)
    keep = torch.empty(B, H, M, nb, dtype=torch.bool, device=dev)
    margin = torch.empty(B, H, M, dtype=torch.float32, device=dev) if router else None
    k_eff_kernel = k_eff if (router and nb > 1) else 0
    _capi.check(lib.ugbsa_select_mask(query.data_ptr(), *query.stride(), planes.data_ptr(),
                                      B, H, Hk, M, N, D, _capi.dtype_code(query.dtype), mode, float(scaling),
                                      _capi.V1_BELIEF if belief else _capi.V1_TOPK, k_bud,
                                      k_eff_kernel, int(sel.k_min), int(sel.k_max),
                                      float(sel.top_p), _capi.ptr(penalty), ws.data_ptr(),
                                      ws_elems, keep.data_ptr(), _capi.ptr(margin), stream),
                "select_mask")
    res = MaskResult(keep, k_bud, margin=margin)
    if want_scores:
        res.scores = ws.view(B, H, -1, nb)[:, :, :M]
    if sel.mode == "rollout":
        # EMA of the last row's selection after forcing (:291-295)
        last = keep[0, :, -1, :].float()
        sel.selection_history = ((1.0 - sel.ema_alpha) * sel.selection_history
                                 + sel.ema_alpha * last)
    if router:
        res.margin_eff = torch.empty_like(margin)
        res.uncertain = torch.empty(B, H, M, dtype=torch.uint8, device=dev)
        res.threshold = torch.empty(1, dtype=torch.float32, device=dev)
        if nb > 1:
            grain = _capi.GRAIN_ROW if sel.router_grain == "row" else _capi.GRAIN_CELL
            rmode = _capi.ROUTER_QUANTILE if sel.router_mode == "quantile" else _capi.ROUTER_ABS
            # rows with more than k_eff visible blocks are eligible (:318-319);
            # n_elig counts rows for row grain and cells for cell grain (:335-336)
            elig_rows = max(0, M - 64 * k_eff)
            n_elig = elig_rows if grain == _capi.GRAIN_ROW else B * H * elig_rows
            k_quant = max(1, int(float(sel.router_quantile) * n_elig)) if n_elig > 0 else 0
            _capi.check(lib.ugbsa_router_rows(margin.data_ptr(), B, H, M, nb, grain, rmode,
                                              float(sel.router_tau), k_quant, k_eff,
                                              keep.data_ptr(), res.margin_eff.data_ptr(),
                                              res.uncertain.data_ptr(), res.threshold.data_ptr(),
                                              stream),
                        "router_rows")
        else:
            # a single block: the only score is both s_top and s_k, so every
            # margin is 0 and no row is eligible
            margin.zero_()
            res.margin_eff.zero_()
            res.uncertain.zero_()
            res.threshold.fill_(float("nan"))
    return res


def _block_select_mask(query, key_states, scaling, layer_idx):
    """v1 selection: keep [B, H, Q, NB] bool, built on the GPU.

    Same contract as src/sparse_attention.py:208-382 (``key_states`` may be
    repeat_kv'd or GQA), including the ``SEL.log`` diagnostics (:355-380).
    """
    res = select_mask_v1(query, key_states, scaling, layer_idx=layer_idx)
    keep = res.keep
    if not SEL.log:
        return keep
    if res.uncertain is not None:
        _log_router_layer(res, keep, query.shape[-2], layer_idx)
    last_rows = keep[0, :, -1, :]                       # [H, NB], the last query row
    SEL.kept_blocks[layer_idx] = last_rows.any(dim=0).cpu()
    SEL.budget_samples.append(last_rows.sum(dim=-1).float().mean().item())
    return keep


def _log_router_layer(res, keep, q_len, layer_idx):
    """One v1 router layer into ``SEL``'s diagnostic lists: the share of
    triggered cells, the mean kept blocks per cell and the mean margin.  On the
    last layer of a prefill (``q_len > 1``; layer count from ``SEL.model_ref``)
    the running means of the three lists are printed on one line, in the
    format the reference's harness logs parse (src/sparse_attention.py:355-375)."""
    series = (SEL.router_trigger_rate, SEL.router_eff_budget, SEL.router_margin_mean)
    values = (res.uncertain.float().mean(), keep.float().sum(dim=-1).mean(), res.margin.mean())
    for dst, val in zip(series, values):
        dst.append(float(val.item()))
    model = SEL.model_ref
    if q_len <= 1 or model is None or layer_idx != len(model.model.layers) - 1:
        return
    trigger, eff_budget, margin = (sum(xs) / len(xs) for xs in series)
    if SEL.router_mode == "quantile":
        knob = "q=%.2f" % SEL.router_quantile
    else:
        knob = "tau=%.3f" % SEL.router_tau
    print("  router[%s/%s]: trigger=%.3f eff_budget=%.1f margin=%.3f %s"
          % (SEL.router_mode, SEL.router_grain, trigger, eff_budget, margin, knob), flush=True)


def install_rollout_hooks(model):
    """Point ``SEL.model_ref`` at ``model`` and stash every decoder layer's
    prefill input in ``SEL.hidden_at[layer]`` (src/sparse_attention.py:189-205).

    Harnesses call this right after loading the model.  ``SEL.model_ref`` is
    what the ``SEL.log`` router summary counts layers from.  The stashed states
    (a reference to each layer's input tensor, no copy; decode steps with one
    query row are skipped) feed only ``rollout_peek``, which this build does
    not provide; they are kept so the call behaves as the reference's, memory
    included."""
    SEL.model_ref = model
    SEL.hidden_at = {}
    for idx, layer in enumerate(model.model.layers):
        layer.register_forward_pre_hook(_HiddenStash(idx), with_kwargs=True)


class _HiddenStash:
    """Forward pre-hook of decoder layer ``idx``: its input hidden state of a
    prefill into ``SEL.hidden_at[idx]``."""

    def __init__(self, idx):
        self.idx = idx

    def __call__(self, module, args, kwargs):
        hs = args[0] if args else kwargs.get("hidden_states")
        if hs is not None and hs.shape[-2] > 1:
            SEL.hidden_at[self.idx] = hs.detach()
        return None


def needle_hit_rate(needle_blocks) -> float:
    """Mean over logged layers of the fraction of ``needle_blocks`` kept for
    the last Q tile (union over heads), read from ``SEL.kept_blocks`` as the
    reference's harness does (src/poc_core.py:77-85).  1.0 when nothing was
    logged or no needle block is given."""
    if not SEL.kept_blocks or not needle_blocks:
        return 1.0
    rates = []
    for kept in SEL.kept_blocks.values():
        hits = sum(1 for b in needle_blocks if b < len(kept) and bool(kept[b]))
        rates.append(hits / len(needle_blocks))
    return sum(rates) / len(rates)


def block_sparse_attention(module, query, key, value, attention_mask,
                           scaling, dropout=0.0, **kwargs):
    """HF attention function (src/sparse_attention.py:751-806).

    query [B, H, S, D]; key / value [B, Hk, S, D] as transformers passes them
    (before repeat_kv).  Dense SDPA for ``mode == "dense"`` or decode (Q == 1);
    the HIP v2 path for topk / router / quest with ``SEL.kernel_v2``; the HIP
    v1 per-row path otherwise (:790-804).  The sparse paths need S_q == S_k.  Returns
    ``(attn_output [B, S, H, D] contiguous, None)``.
    """
    Q = query.shape[-2]
    is_prefill = Q > 1
    H, Hk = query.shape[1], key.shape[1]

    if SEL.mode == "dense" or Q == 1:
        ev = PROF.start("dense_sdpa") if is_prefill else None
        out = F.scaled_dot_product_attention(query, key, value, is_causal=Q > 1,
                                             scale=scaling, enable_gqa=H != Hk)
        PROF.stop(ev)
        return out.transpose(1, 2).contiguous(), None

    # query row i is key position i in the selector's tile visibility and in
    # the kernels' causal mask (one-shot prefill)
    assert key.shape[-2] == Q, (
        f"sparse prefill needs query length == key length (got {Q} vs {key.shape[-2]})")
    if SEL.kernel_v2 and SEL.mode in ("topk", "router", "quest"):
        ev = PROF.start("v2_select") if is_prefill else None
        kv_idx = _block_select_kv_idx_v2(query, key, scaling)   # resolved at call time
        PROF.stop(ev)
        ev = PROF.start("v2_kernel") if is_prefill else None
        B, _, S, D = query.shape
        out = torch.empty(B, S, H, D, dtype=query.dtype, device=query.device)
        ws = attn_workspace(B, Hk, key.shape[-2], D, query.device)
        block_sparse_attn_v2(query, key, value, kv_idx, scale=scaling, block_n=BLOCK,
                             out=out.transpose(1, 2), workspace=ws)
        PROF.stop(ev)
        return out, None

    if SEL.mode == "rollout_peek":
        raise NotImplementedError(
            "SEL.mode 'rollout_peek' is not part of this build: it is an abandoned research "
            "mode of the reference (a model-level planner off the sparse-prefill path); use "
            "'topk', 'quest', 'router', 'belief' or 'rollout'")
    keep = _block_select_mask(query, key, scaling, module.layer_idx)
    B, _, S, D = query.shape
    out = torch.empty(B, S, H, D, dtype=query.dtype, device=query.device)
    ws = attn_workspace(B, Hk, key.shape[-2], D, query.device)
    block_sparse_attn(query, key, value, keep, scale=scaling, block_n=BLOCK,
                      out=out.transpose(1, 2), workspace=ws)
    return out, None


def _register():
    try:
        from transformers import AttentionInterface
    except ImportError:   # the kernels stay usable without transformers
        return False
    AttentionInterface.register("block_sparse", block_sparse_attention)
    return True


REGISTERED = _register()
