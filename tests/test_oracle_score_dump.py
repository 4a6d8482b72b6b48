"""Pins of the score-dump oracle (oracle/score_dump.py) on the CPU.

Each check is independent of the oracle's own formulation: Python ``sorted``
with explicit fp32 arithmetic for the order statistics, float64 dot-product
loops and closed forms for tau_hat, hand-worked row samples and budgets.
"""

import math

import numpy as np
import pytest

from oracle import score_dump as SD
from oracle import selector as S

f32 = np.float32


def test_dump_budgets_no_selector_clamp():
    # the dump doubles budget_blocks directly (src/dump_block_scores.py:150):
    # budget 2 gives k_b 4, where the selector would clamp to k_min = 8 first
    assert SD.dump_budgets(2, 512) == (4, 8)
    assert SD.dump_budgets(32, 512) == (64, 128)
    assert SD.dump_budgets(32, 100) == (64, 100)     # rho_k capped at NB
    assert SD.dump_budgets(64, 100) == (100, 100)    # no gap: rho_k <= k_b


def brute_stats(row, k_b, rho_k):
    s = sorted((float(x) for x in row), reverse=True)
    s0, skm1, sk, srm1, srk = (f32(s[i]) for i in (0, k_b - 1, k_b, rho_k - 1, rho_k))
    with np.errstate(invalid="ignore", over="ignore"):
        g = f32(skm1 - sk)
        r = f32(s0 - sk)
        r = r if (math.isnan(r) or r >= f32(1e-9)) else f32(1e-9)
        sg = f32(g / r)
        if not math.isnan(sg):
            sg = min(max(sg, f32(0)), f32(2))
        grho = f32(srm1 - srk)
    return g, r, sg, grho


def test_order_stats_against_sorted():
    rng = np.random.default_rng(7)
    nb, k_b, rho_k = 24, 4, 8
    T = rng.standard_normal((3, 5, nb)).astype(np.float32)
    T[0, 0, 3] = T[0, 0, 5]                       # a tie
    n_vis = np.array([24, 9, 8, 5, 1])            # rows with -inf tails
    for t, nv in enumerate(n_vis):
        T[:, t, nv:] = -np.inf
    got = SD.order_stats(T, k_b, rho_k)
    for b in range(3):
        for t in range(5):
            want = brute_stats(T[b, t], k_b, rho_k)
            for name, arr, w in zip(("g", "r", "sigma", "g_rho"), got, want):
                v = arr[b, t]
                assert (np.isnan(v) and np.isnan(w)) or v == w, (name, b, t, v, w)
    # tiles with <= rho_k visible blocks: s(rho_k) = -inf, so g_rho = +inf or NaN
    assert np.isfinite(got[3][0, 1]) and np.isinf(got[3][0, 2]) and np.isnan(got[3][0, 3])
    # tile with 5 visible blocks: s(k_b) is finite, s(rho_k - 1) is -inf
    assert np.isfinite(got[0][0, 3]) and np.isnan(got[3][0, 3])


def test_pair_rows_by_hand():
    assert SD.pair_rows(1).size == 0
    assert SD.pair_rows(2).tolist() == [0]
    assert SD.pair_rows(100).tolist() == list(range(99))
    assert SD.pair_rows(1025).tolist() == list(range(1024))
    i = SD.pair_rows(1026)                            # stride (1025 // 1024) = 1
    assert i.size == 1024 and i[-1] == 1023
    i = SD.pair_rows(8192)                            # stride 8191 // 1024 = 7
    assert i.size == 1024 and i[1] == 7 and i[-1] == 1023 * 7 and i[-1] + 1 < 8192


def brute_tau(q, k, scaling, quest):
    q = q.astype(np.float64)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    nb = (N + 63) // 64
    kp = np.zeros((B, Hk, nb * 64, D))
    kp[:, :, :N] = k
    blk = kp.reshape(B, Hk, nb, 64, D)
    out = np.zeros((B, H))
    for b in range(B):
        for h in range(H):
            kh = h // (H // Hk)
            acc, n = 0.0, 0
            for i in SD.pair_rows(M):
                for j in range(nb):
                    def score(row):
                        x = q[b, h, row]
                        if quest:
                            return sum(max(x[d] * blk[b, kh, j, :, d].max(),
                                           x[d] * blk[b, kh, j, :, d].min()) for d in range(D)) * scaling
                        return float(x @ blk[b, kh, j].mean(axis=0)) * scaling
                    d = score(i + 1) - score(i)
                    acc += d * d
                    n += 1
            out[b, h] = math.sqrt(0.5 * acc / n)
    return out


@pytest.mark.parametrize("quest", [False, True])
def test_tau_hat_brute_force(quest):
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 4, 40, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 150, 8)).astype(np.float32)   # ragged last block
    got = SD.tau_hat(q, k, 0.35, quest)
    want = brute_tau(q, k, 0.35, quest)
    np.testing.assert_allclose(got, want, rtol=2e-6)


def test_tau_hat_repeated_rows_is_zero():
    rng = np.random.default_rng(3)
    row = rng.standard_normal(16).astype(np.float32)
    q = np.broadcast_to(row, (1, 2, 300, 16)).copy()
    k = rng.standard_normal((1, 1, 300, 16)).astype(np.float32)
    for quest in (False, True):
        assert np.all(SD.tau_hat(q, k, 0.25, quest) == 0)
    assert np.all(SD.tau_hat(q[:, :, :1], k, 0.25, True) == 0)    # M < 2


@pytest.mark.parametrize("quest", [False, True])
def test_tau_hat_arithmetic_progression_closed_form(quest):
    # q_i = a + i * delta: S[i + 1] - S[i] = (delta . s_blk) for every pair,
    # s_blk = Kmean_blk * scaling (mean) or Kmax_blk * scaling (Quest, q > 0)
    rng = np.random.default_rng(5)
    D, M = 8, 200
    a = np.full(D, 4.0)
    delta = rng.integers(1, 4, D) / 64.0
    q = (a + np.arange(M)[:, None] * delta)[None, None].astype(np.float32)
    k = rng.standard_normal((1, 1, 256, D)).astype(np.float32)
    blocks = k.reshape(1, 1, 4, 64, D).astype(np.float64)
    s = blocks.max(axis=3) if quest else blocks.mean(axis=3)
    step = (s[0, 0] @ delta) * 0.5
    want = math.sqrt(0.5 * np.mean(step ** 2))
    got = SD.tau_hat(q, k, 0.5, quest)[0, 0]
    assert abs(got - want) <= 1e-5 * want


def test_raw_scores_are_forced_scores_before_forcing():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 2, 300, 16)).astype(np.float32)
    k = rng.standard_normal((1, 1, 300, 16)).astype(np.float32)
    for quest in (False, True):
        raw = S.tile_scores(q, k, 0.25, quest, force=False)
        forced = S.tile_scores(q, k, 0.25, quest)
        vis, self_blk = S.tile_visibility(5, 300, 5)
        mask = np.ones_like(raw, dtype=bool)
        mask[..., 0] = False
        mask[:, :, np.arange(5), self_blk] = False
        assert np.array_equal(raw[mask], forced[mask])
        assert np.all(np.isfinite(raw[:, :, vis])) and np.all(raw[:, :, ~vis] == -np.inf)


def test_score_dump_early_returns():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 2, 512, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 512, 16)).astype(np.float32)   # NB = 8
    cfg = S.SelectorConfig(mode="router", budget_blocks=4)          # k_b = 8 = NB
    assert SD.score_dump(q, k, 0.25, cfg) is None
    cfg.budget_blocks = 2                                            # rho_k = 8 = NB
    assert SD.score_dump(q, k, 0.25, cfg) is None
    cfg.budget_blocks = 1                                            # k_b 2, rho_k 4
    shard = SD.score_dump(q, k, 0.25, cfg)
    assert shard["valid"].tolist() == [False] * 4 + [True] * 4
    assert shard["mode_id"] == 1 and shard["g"].shape == (1, 2, 8)
