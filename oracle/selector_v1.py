"""numpy fp32 restatement of the reference's v1 per-row selector — TEST ORACLE.

Reference: ``src/sparse_attention.py:208-382`` (``_block_select_mask``): a
boolean ``keep [B, H, Q, NB]`` per query row, for the policies ``topk``,
``quest``, ``router`` (per-row margin, eligibility, row/cell grain,
quantile/abs), ``belief`` (top-p softmax mass budget) and ``rollout``
(last-row penalty by an EMA of earlier selections).  The GPU path is held to
these functions; attention over ``keep`` is ``oracle.attention.keep_attention``.

Deliberate definitions where the reference leaves the result unspecified:

* ``topk`` / ``argsort`` tie order: score descending, block ascending (as the
  v2 oracle).  Rows with fewer visible blocks than the budget therefore keep
  the lowest-numbered invisible blocks, where the reference keeps arbitrary
  invisible ones; attention never reads them (causal mask).
* ``mean(dim=1)`` over heads (row grain): sequential fp32 sum over heads,
  then one division by H (ATen's CPU reduction for this layout).
* ``belief`` softmax: max-subtracted exp in fp32 summed sequentially and the
  cumulative mass in fp32 sequentially; budgets that sit within 1e-6 of
  ``top_p`` are near ties (the reference's order of summation is not fixed).

How each function is pinned (tests/test_oracle_selector_v1.py):

* ``row_block_scores``  per-row Quest identity / mean score against float64
                        brute force; -inf exactly outside per-row visibility.
* ``select_mask_v1``    against the golden vectors written from the reference
                        itself (tests/golden/make_golden_v1.py) for every
                        policy, on the reference's own ranked scores (spied),
                        and by hand-built cases (all ties, budget > visible).
* ``router_v1``         against ``sorted`` with +inf for ineligible / NaN
                        cells and the reference's n_elig / k_quant rule.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import selector as S

SPREAD_MIN = np.float32(1e-6)       # clamp(min=1e-6), src/sparse_attention.py:315


@dataclass
class SelectorV1Config:
    """The ``Selector`` fields the v1 path reads (src/sparse_attention.py:58-97)."""
    mode: str = "topk"
    budget_blocks: int = 32
    top_p: float = 0.9
    k_min: int = 8
    k_max: int = 112
    explore_bonus: float = 0.3
    ema_alpha: float = 0.3
    router_mode: str = "abs"
    router_grain: str = "cell"
    router_tau: float = 0.10
    router_quantile: float = 0.20
    router_score: str = "mean"

    @classmethod
    def from_selector(cls, sel) -> "SelectorV1Config":
        return cls(**{f: getattr(sel, f) for f in cls.__dataclass_fields__})

    @property
    def use_quest(self) -> bool:
        # src/sparse_attention.py:223-224
        return self.mode == "quest" or (self.mode == "router" and self.router_score == "quest")


def row_visibility(M: int, N: int, block_n: int = S.BLOCK):
    """visible [M, NB]: block b starts at or before the row's position
    K - Q + i (src/sparse_attention.py:241-243)."""
    nb = (N + block_n - 1) // block_n
    q_global = np.arange(N - M, N)
    return (np.arange(nb) * block_n)[None, :] <= q_global[:, None], q_global


def row_block_scores(q, k, scaling: float, use_quest: bool):
    """block_score [B, H, M, NB] fp32 with -inf outside row visibility.

    src/sparse_attention.py:218-244: the same summaries and score as the v2
    path (Quest two-matmul form or K-mean), per query row, no tile pooling.
    """
    q = S._f32(q)
    B, H, M, D = q.shape
    N = k.shape[2]
    s = S.row_scores(q, k, scaling, use_quest, np.arange(M))
    visible, _ = row_visibility(M, N)
    s[:, :, ~visible] = -np.inf
    return s


def rank_order(scores):
    """Indices of each row sorted by (score desc, block asc)."""
    scores = S._f32(scores)
    key = S.sortable_key(scores).astype(np.int64)
    nb = scores.shape[-1]
    comp = (np.int64(0xFFFFFFFF) - key) * nb + np.arange(nb)
    return np.argsort(comp, axis=-1, kind="stable")


def belief_budget(scores, top_p: float):
    """(cumsum(sorted softmax) < top_p).sum() + 1 per row — :267-269 (before clamp)."""
    s = S._f32(scores)
    order = rank_order(s)
    srt = np.take_along_axis(s, order, axis=-1)
    mx = srt[..., :1]
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp((srt - mx).astype(np.float32)).astype(np.float32)
    z = np.zeros(s.shape[:-1], np.float32)
    for j in range(s.shape[-1]):
        z = (z + e[..., j]).astype(np.float32)
    p = (e / z[..., None]).astype(np.float32)
    c = np.zeros(s.shape[:-1], np.float32)
    cnt = np.zeros(s.shape[:-1], np.int64)
    for j in range(s.shape[-1]):
        c = (c + p[..., j]).astype(np.float32)
        cnt += (c < np.float32(top_p))
    return cnt.astype(np.float32) + np.float32(1.0), c


@dataclass
class MaskSelection:
    keep: np.ndarray                      # bool [B, H, M, NB]
    score_for_sel: np.ndarray             # fp32 [B, H, M, NB] (ranked scores)
    margin: np.ndarray | None = None      # fp32 [B, H, M] per-cell sigma (router)
    margin_score: np.ndarray | None = None  # after the row mean (router)
    eligible: np.ndarray | None = None    # bool [M]
    m_safe: np.ndarray | None = None      # fp32, +inf for ineligible / NaN (quantile)
    threshold: np.float32 | None = None   # quantile threshold (router quantile)
    k_quant: int | None = None
    uncertain: np.ndarray | None = None   # bool [B, H, M]
    budget: np.ndarray | None = None      # fp32 [B, H, M] (belief)
    history: np.ndarray | None = None     # fp32 [H, NB] after the update (rollout)


def router_v1(score_for_sel, visible, cfg: SelectorV1Config):
    """Per-row margin, eligibility, threshold, trigger — :297-354.

    Returns (margin [B,H,M], margin_score, eligible [M], m_safe, thresh,
    k_quant, uncertain [B,H,M]).
    """
    sc = S._f32(score_for_sel)
    B, H, M, nb = sc.shape
    k = int(cfg.budget_blocks)
    k_eff = max(1, min(k, nb - 1))
    order = rank_order(sc)[..., :k_eff + 1]
    vals = np.take_along_axis(sc, order, axis=-1)
    s_top, s_km1, s_k = vals[..., 0], vals[..., k_eff - 1], vals[..., k_eff]
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        spread = np.maximum((s_top - s_k).astype(np.float32), SPREAD_MIN)
        margin = ((s_km1 - s_k).astype(np.float32) / spread).astype(np.float32)
    eligible = visible.sum(axis=-1) > k_eff                       # [M]
    if cfg.router_grain == "row":
        acc = margin[:, 0].copy()
        for h in range(1, H):
            acc = (acc + margin[:, h]).astype(np.float32)
        with np.errstate(invalid="ignore"):
            margin_score = (acc / np.float32(H)).astype(np.float32)[:, None, :]   # [B,1,M]
        elig_score = np.broadcast_to(eligible[None, None, :], (1, 1, M))
    else:
        margin_score = margin
        elig_score = np.broadcast_to(eligible[None, None, :], margin.shape)
    thresh, kq, m_safe = None, None, None
    with np.errstate(invalid="ignore"):
        if cfg.router_mode == "quantile":
            m_safe = np.where(elig_score, margin_score, np.float32(np.inf))
            m_safe = np.where(np.isnan(m_safe), np.float32(np.inf), m_safe).astype(np.float32)
            n_elig = int(elig_score.sum())
            kq = max(1, int(float(cfg.router_quantile) * n_elig)) if n_elig > 0 else 0
            if kq > 0:
                thresh = np.float32(np.sort(m_safe.ravel())[kq - 1])
                unc = (m_safe <= thresh) & elig_score
            else:
                unc = np.zeros(margin_score.shape, bool)
        else:
            unc = (margin_score < np.float32(cfg.router_tau)) & elig_score
    unc = np.broadcast_to(unc, (B, H, M)).copy()
    return margin, margin_score, eligible, m_safe, thresh, kq, unc


def select_mask_v1(q, k, scaling: float, cfg: SelectorV1Config, history=None) -> MaskSelection:
    """``keep`` of ``_block_select_mask`` (src/sparse_attention.py:208-382) in fp32.

    ``k`` may hold H heads (repeat_kv'd) or Hk heads.  ``history`` is the
    rollout EMA state [H, NB] (None or a wrong shape starts from zeros,
    :247-252, :291-295); the updated state is returned in ``MaskSelection.history``.
    """
    q = S._f32(q)
    block_score = row_block_scores(q, k, scaling, cfg.use_quest)
    return select_mask_from_scores(block_score, k.shape[2], cfg, history)


def select_mask_from_scores(block_score, n_keys: int, cfg: SelectorV1Config,
                            history=None) -> MaskSelection:
    """Steps :245-354 on given fp32 block scores [B, H, M, NB] (-inf outside
    visibility) — the part a GPU selector must reproduce bit for bit when fed
    the same scores."""
    block_score = S._f32(block_score)
    B, H, M, nb = block_score.shape
    visible, q_global = row_visibility(M, n_keys)
    res = MaskSelection(keep=None, score_for_sel=block_score)
    if cfg.mode == "rollout":
        if history is None or np.shape(history) != (H, nb):
            history = np.zeros((H, nb), np.float32)
        sfs = block_score.copy()
        penalty = (np.float32(cfg.explore_bonus) * S._f32(history)).astype(np.float32)
        sfs[:, :, -1, :] = (sfs[:, :, -1, :] - penalty[None]).astype(np.float32)
        res.score_for_sel = sfs
    sfs = res.score_for_sel
    order = rank_order(sfs)
    if cfg.mode in ("topk", "router", "rollout", "quest"):
        k_bud = min(int(max(min(cfg.k_max, cfg.budget_blocks), cfg.k_min)), nb)
        top = order[..., :k_bud]
        keep = np.zeros((B, H, M, nb), bool)
        np.put_along_axis(keep, top, True, axis=-1)
    else:   # belief
        budget, _ = belief_budget(block_score, cfg.top_p)
        budget = np.clip(budget, cfg.k_min, cfg.k_max).astype(np.float32)
        res.budget = budget
        rank = np.empty_like(order)
        np.put_along_axis(rank, order, np.arange(nb)[None, None, None, :].repeat(M, 2), axis=-1)
        keep = rank < budget[..., None]
    keep[..., 0] = True
    keep[:, :, np.arange(M), q_global // S.BLOCK] = True
    if cfg.mode == "rollout":
        last = keep[0, :, -1, :].astype(np.float32)
        res.history = (np.float32(1.0 - cfg.ema_alpha) * S._f32(history)
                       + np.float32(cfg.ema_alpha) * last).astype(np.float32)
    if cfg.mode == "router":
        (res.margin, res.margin_score, res.eligible, res.m_safe, res.threshold,
         res.k_quant, res.uncertain) = router_v1(sfs, visible, cfg)
        keep = np.where(res.uncertain[..., None], visible[None, None], keep)
    res.keep = keep
    return res
