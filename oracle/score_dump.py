"""numpy restatement of the reference's score-dump diagnostic — TEST ORACLE.

Reference: ``src/dump_block_scores.py`` — ``_record`` (:104-207) computes,
beside each ``_block_select_kv_idx_v2`` call, per-tile order statistics of
the *unforced* tile scores and a per-head score-noise estimate; ``_mode_id``
(:210-219) labels the backbone.  The GPU path (``ugbsa_score_dump``) is held
to these functions.

Functions and how each is pinned (tests/test_oracle_score_dump.py):

* ``dump_budgets``  k_b = min(2 * budget_blocks, NB) — no k_min/k_max clamp,
                    unlike the selector (:150) — and rho_k = min(2 * k_b, NB)
                    (:151); checked on the boundary cases by hand.
* ``order_stats``   g, r, sigma, g_rho of :161-171 from a descending sort;
                    pinned bit-exactly against Python ``sorted`` per row with
                    explicit IEEE fp32 arithmetic, including the -inf ranks
                    of tiles with few visible blocks (NaN / inf gaps).
* ``pair_rows``     the sampled rows of :182-187; checked by hand at the
                    boundaries (M = 2, M = 1025, M = 1026, large M).
* ``tau_hat``       :188-194; pinned against a float64 brute force over
                    explicit dot products, against 0 for repeated rows, and
                    against the closed form sqrt(mean_blk (delta . s_blk)^2 / 2)
                    for rows in arithmetic progression q_i = a + i * delta
                    (mean backbone: s_blk = Kmean_blk * scaling; Quest with
                    positive rows: s_blk = Kmax_blk * scaling).
* ``score_dump``    the shard (or None when :152-158 return early).
"""

from __future__ import annotations

import numpy as np

from . import selector as S

R_MIN = np.float32(1e-9)    # clamp(min=1e-9), src/dump_block_scores.py:169
N_PAIRS_MAX = 1024          # src/dump_block_scores.py:183

MODE_LABELS = {0: "topk", 1: "router_mean", 2: "router_quest", 3: "quest", 4: "other"}


def mode_id(cfg) -> int:
    """0 topk, 1 router-mean, 2 router-quest, 3 quest, 4 other (:210-219)."""
    if cfg.mode == "topk":
        return 0
    if cfg.mode == "router":
        return 2 if cfg.router_score == "quest" else 1
    if cfg.mode == "quest":
        return 3
    return 4


def dump_budgets(budget_blocks: int, n_blocks: int):
    """(k_b, rho_k) of src/dump_block_scores.py:150-151."""
    k_b = min(2 * int(budget_blocks), n_blocks)
    return k_b, min(2 * k_b, n_blocks)


def tile_n_visible(q_tiles: int, n_keys: int, block_m: int = 64, block_n: int = S.BLOCK):
    """Visible blocks per tile, the row sums of :143-144's mask."""
    last = np.minimum(np.arange(q_tiles) * block_m + block_m - 1, n_keys - 1)
    return last // block_n + 1


def order_stats(T_raw, k_b: int, rho_k: int):
    """(g, r, sigma, g_rho) fp32 [..] from unforced tile scores — :161-171.

    Ranks past the visible blocks hold -inf, so tiles with <= rho_k visible
    blocks yield inf / NaN gaps exactly as the reference's fp32 arithmetic.
    """
    T = np.asarray(T_raw, dtype=np.float32)
    srt = -np.sort(-T, axis=-1)                     # descending, -inf last
    s0, skm1, sk = srt[..., 0], srt[..., k_b - 1], srt[..., k_b]
    srm1, srk = srt[..., rho_k - 1], srt[..., rho_k]
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        g = (skm1 - sk).astype(np.float32)
        r = np.maximum((s0 - sk).astype(np.float32), R_MIN)    # NaN-propagating, as clamp
        sigma = np.clip((g / r).astype(np.float32), np.float32(0), np.float32(2))
        g_rho = (srm1 - srk).astype(np.float32)
    return g, r, sigma, g_rho


def pair_rows(M: int) -> np.ndarray:
    """Lower rows i of the sampled adjacent pairs (i, i + 1) — :183-186."""
    if M < 2:
        return np.zeros(0, dtype=np.int64)
    n_pairs = min(N_PAIRS_MAX, M - 1)
    stride = max(1, (M - 1) // n_pairs)
    return np.minimum(np.arange(n_pairs, dtype=np.int64) * stride, M - 2)


def tau_hat(q, k, scaling: float, use_quest: bool) -> np.ndarray:
    """sqrt(max(0, 0.5 * mean (S[i+1] - S[i])^2)) per (b, h), fp32 — :181-194.

    The mean runs over the sampled pairs and every block (no causal mask);
    summed in float64 here (the reference reduces in fp32 — the GPU test
    compares with a relative tolerance).
    """
    q = np.asarray(q, dtype=np.float32)
    B, H, M = q.shape[:3]
    i0 = pair_rows(M)
    if i0.size == 0:
        return np.zeros((B, H), np.float32)
    lo = S.row_scores(q, k, scaling, use_quest, i0)
    hi = S.row_scores(q, k, scaling, use_quest, i0 + 1)
    diff = (hi - lo).astype(np.float64)
    tau_sq = 0.5 * (diff * diff).mean(axis=(-2, -1))
    return np.sqrt(np.maximum(tau_sq, 0.0)).astype(np.float32)


def score_dump(q, k, scaling: float, cfg: S.SelectorConfig, block_m: int = 64):
    """The shard of ``_record`` (:104-207) without ``call_idx``, or None.

    None where the reference returns early: no room for a g_rho gap
    (rho_k <= k_b, :152-153) or no tile with more than rho_k visible blocks
    (:157-158).
    """
    q = np.asarray(q, dtype=np.float32)
    B, H, M, D = q.shape
    N = k.shape[2]
    nb = (N + S.BLOCK - 1) // S.BLOCK
    qt = (M + block_m - 1) // block_m
    k_b, rho_k = dump_budgets(cfg.budget_blocks, nb)
    if rho_k <= k_b:
        return None
    valid = tile_n_visible(qt, N, block_m) > rho_k
    if not valid.any():
        return None
    T = S.tile_scores(q, k, scaling, cfg.use_quest, block_m, force=False)
    g, r, sigma, g_rho = order_stats(T, k_b, rho_k)
    return {"n_blocks": int(nb), "mode_id": mode_id(cfg),
            "budget_blocks": int(cfg.budget_blocks),
            "g": g, "r": r, "sigma": sigma, "g_rho": g_rho, "valid": valid,
            "tau_hat": tau_hat(q, k, scaling, cfg.use_quest), "tile_score": T}
