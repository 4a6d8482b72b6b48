"""Pins the numpy selector oracle: reference golden vectors + independent math."""

import math
from fractions import Fraction

import numpy as np
import pytest

from conftest import load_golden
from oracle import selector as S

GOLDEN_SMALL = ["a", "b_ragged", "c_full"]


def cfg_from_fields(fields):
    known = S.SelectorConfig.__dataclass_fields__
    return S.SelectorConfig(**{k: v for k, v in fields.items() if k in known})


def unique_slot_mismatches(kv_ref, kv_new, T):
    """Slots whose reference score is unique in its row must hold the same block."""
    bad = 0
    nb = T.shape[-1]
    for idx in np.ndindex(*T.shape[:-1]):
        row = T[idx]
        vals, counts = np.unique(row, return_counts=True)
        once = set(vals[counts == 1].tolist())
        for j, blk in enumerate(kv_ref[idx]):
            if blk < nb and float(row[blk]) in once and kv_new[idx][j] != blk:
                bad += 1
    return bad


@pytest.mark.parametrize("name", GOLDEN_SMALL)
def test_golden_selection_on_reference_scores(name):
    """Given the reference's own fp32 tile scores, the oracle's selection is the
    reference's: same sets, same slot order where scores are untied, same
    margins handed to kthvalue, bit-identical threshold."""
    _, pols = load_golden(name)
    assert len(pols) == 9
    for pol, rec in pols.items():
        cfg = cfg_from_fields(rec["fields"])
        T = rec["tile_score"]
        sel = S.select_from_tile_scores(T, cfg)
        nb = T.shape[-1]
        assert sel.kv_idx.shape == rec["kv_idx"].shape, pol
        assert (S.canonical_sets(sel.kv_idx, sel.k_base, nb)
                == S.canonical_sets(rec["kv_idx"], sel.k_base, nb)), pol
        assert unique_slot_mismatches(rec["kv_idx"], sel.kv_idx, T) == 0, pol
        # sentinel columns: exactly the extra slots of non-triggered tiles
        if sel.uncertain is not None:
            ref_sent = (rec["kv_idx"][..., sel.k_base:] == nb).all(-1)
            assert np.array_equal(ref_sent, ~sel.uncertain), pol
        if "kth_in" in rec:
            assert np.array_equal(rec["kth_in"].ravel(), sel.sigma_eff.ravel(),
                                  equal_nan=True), pol
            assert int(rec["kth_k"]) == S.quantile_rank(cfg.router_quantile,
                                                        sel.sigma_eff.size)
            a, b = np.float32(rec["kth_out"]), sel.threshold
            assert (np.isnan(a) and np.isnan(b)) or a.view(np.uint32) == b.view(np.uint32), pol


@pytest.mark.parametrize("name", GOLDEN_SMALL)
def test_golden_selection_on_own_scores(name):
    """From the bf16 inputs, the oracle's fp32 scores sit within 1e-6 of the
    reference's, and its kv_idx sets equal the reference's."""
    inp, pols = load_golden(name)
    for pol, rec in pols.items():
        cfg = cfg_from_fields(rec["fields"])
        sel = S.select_kv_idx_v2(inp["q"], inp["k"], float(inp["scaling"]), cfg)
        T = rec["tile_score"]
        fin = np.isfinite(T)
        assert np.array_equal(fin, np.isfinite(sel.tile_score))
        assert np.abs(T[fin] - sel.tile_score[fin]).max() <= 1e-6, pol
        nb = T.shape[-1]
        assert (S.canonical_sets(sel.kv_idx, sel.k_base, nb)
                == S.canonical_sets(rec["kv_idx"], sel.k_base, nb)), pol


def test_golden_c1_full_config():
    """BASELINE configs[0] (S=8192, 8/2 heads, D=128, fp32) regenerated from
    the seeded generator; both router backbones."""
    import hashlib
    import synth
    inp, pols = load_golden("c1")
    cfg = synth.CONFIGS["c1"]
    q, k, _ = synth.make_layer(cfg, 0)
    q, k = q.numpy(), k.numpy()
    h = hashlib.sha256()
    h.update(q.tobytes())
    h.update(k.tobytes())
    assert h.hexdigest() == str(inp["input_sha256"]), "generator drifted"
    for pol, rec in pols.items():
        c = S.SelectorConfig(**cfg.sel_fields())
        c.router_score = pol.split("_")[1]
        own = S.select_kv_idx_v2(q, k, cfg.scaling, c)
        fromT = S.select_from_tile_scores(rec["tile_score"], c)
        nb = rec["tile_score"].shape[-1]
        ref_sets = S.canonical_sets(rec["kv_idx"], fromT.k_base, nb)
        assert ref_sets == S.canonical_sets(fromT.kv_idx, fromT.k_base, nb)
        assert ref_sets == S.canonical_sets(own.kv_idx, own.k_base, nb)
        assert fromT.threshold.view(np.uint32) == np.float32(rec["kth_out"]).view(np.uint32)
        assert fromT.uncertain.mean() == 0.25


def test_budgets_match_config_table():
    # (budget_blocks, NB) -> (k_base, k_slots) for c1..c5 under router
    table = {(8, 128): (16, 32), (32, 512): (64, 128), (64, 2048): (128, 256),
             (48, 1024): (96, 192)}
    for (bud, nb), want in table.items():
        assert S.budgets(S.SelectorConfig(mode="router", budget_blocks=bud), nb) == want
    assert S.budgets(S.SelectorConfig(mode="topk", budget_blocks=200), 4096) == (224, 224)
    assert S.budgets(S.SelectorConfig(mode="topk", budget_blocks=1), 4096) == (16, 16)
    assert S.budgets(S.SelectorConfig(mode="router", budget_blocks=32), 40) == (40, 40)


def test_block_summaries_bruteforce():
    rng = np.random.default_rng(0)
    k = rng.standard_normal((1, 2, 150, 8)).astype(np.float32)   # ragged: 150 = 2*64 + 22
    kmin, kmax = S.block_summaries(k, True)
    kmean = S.block_summaries(k, False)
    for h in range(2):
        for blk in range(3):
            rows = list(k[0, h, blk * 64:(blk + 1) * 64])
            rows += [np.zeros(8, np.float32)] * (64 - len(rows))    # F.pad zeros
            rows = np.array(rows)
            assert np.array_equal(kmin[0, h, blk], rows.min(0))
            assert np.array_equal(kmax[0, h, blk], rows.max(0))
            np.testing.assert_allclose(kmean[0, h, blk], rows.astype(np.float64).sum(0) / 64,
                                       rtol=0, atol=2e-7)


def test_quest_identity_and_upper_bound():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 2, 128, 16)).astype(np.float32)
    k = rng.standard_normal((1, 1, 128, 16)).astype(np.float32)
    sc = 16 ** -0.5
    T = S.tile_scores(q, k, sc, True)
    kmin, kmax = S.block_summaries(k, True)
    for h in range(2):
        for t in range(2):
            for blk in range(t + 1):
                rows = q[0, h, t * 64:(t + 1) * 64].astype(np.float64)
                per_row = np.maximum(rows * kmax[0, 0, blk], rows * kmin[0, 0, blk]).sum(1) * sc
                forced = blk == 0 or blk == t
                if not forced:
                    assert abs(per_row.max() - T[0, h, t, blk]) <= 1e-5
                # Quest upper bound: >= the best exact q.k in the block, per row
                exact = rows @ k[0, 0, blk * 64:(blk + 1) * 64].astype(np.float64).T * sc
                assert (per_row + 1e-5 >= exact.max(1)).all()


def test_tile_max_visibility_forcing_bruteforce():
    rng = np.random.default_rng(2)
    M = 200                                            # ragged Q: 4 tiles, last has 8 rows
    q = rng.standard_normal((1, 1, M, 8)).astype(np.float32)
    k = rng.standard_normal((1, 1, M, 8)).astype(np.float32)
    sc = 0.3
    T = S.tile_scores(q, k, sc, False)
    kmean = S.block_summaries(k, False)
    qp = np.zeros((256, 8), np.float32)
    qp[:M] = q[0, 0]
    for t in range(4):
        last = min(t * 64 + 63, M - 1)
        for blk in range(4):
            if blk == 0 or blk == last // 64:
                assert T[0, 0, t, blk] == S.FMAX
            elif blk * 64 > last:
                assert T[0, 0, t, blk] == -np.inf
            else:
                want = max(float(np.float32(qp[r] @ kmean[0, 0, blk]) * np.float32(sc))
                           for r in range(t * 64, t * 64 + 64))     # padded rows score 0
                assert abs(T[0, 0, t, blk] - want) <= 1e-6


def test_topk_order_total():
    rng = np.random.default_rng(3)
    T = rng.integers(-3, 3, size=(5, 40)).astype(np.float32)   # many ties
    T[0, 5] = np.nan
    T[1, :10] = -np.inf
    vals, idx = S.topk_order(T, 17)
    for r in range(5):
        def key(i):
            x = T[r, i]
            return (0 if np.isnan(x) else 1, -x if not np.isnan(x) else 0, i)
        want = sorted(range(40), key=key)[:17]
        assert idx[r].tolist() == want


def _round_subnormal(fr: Fraction) -> float:
    """Round a non-negative Fraction to the fp32 grid below 2**-126 (quantum 2**-149), ties to even."""
    units = fr * (2 ** 149)
    n = units.numerator // units.denominator
    rem = units - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    assert n <= 2 ** 23
    return math.ldexp(n, -149)


def test_sigma_fmax_quirk_bitexact():
    rng = np.random.default_rng(4)
    kb = 3
    for _ in range(300):
        a = np.float32(rng.uniform(-2, 2))
        gap = np.float32(10.0 ** rng.uniform(-7, 0.5))
        c = np.float32(a - gap)
        vals = np.array([S.FMAX, 5, a, c], np.float32)
        sig = S.sigma_margin(vals[None], kb)[0]
        g = Fraction(float(np.float32(a - c)))
        want = _round_subnormal(g / Fraction(float(S.FMAX)))
        assert float(sig) == want
    # documented probe values: gap 1e-6 -> 2 quanta
    vals = np.array([S.FMAX, 1.0, np.float32(0.5), np.float32(0.5) - np.float32(1e-6)], np.float32)
    assert float(S.sigma_margin(vals[None], 3)[0]) / S.sigma_quantum() == 2.0


def test_sigma_nan_rows_are_early_tiles():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 64 * 12, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 64 * 12, 8)).astype(np.float32)
    cfg = S.SelectorConfig(mode="router", budget_blocks=2, k_min=1, router_mode="quantile",
                           router_grain="cell", router_score="mean")
    sel = S.select_kv_idx_v2(q, k, 0.3, cfg)
    assert sel.k_base == 4 and sel.k_slots == 8
    nan_tiles = np.isnan(sel.sigma[0, 0])
    assert nan_tiles.tolist() == [t <= sel.k_base - 1 for t in range(12)]
    assert not sel.uncertain[..., :sel.k_base].any()   # NaN never triggers


def test_kth_smallest_nan_last_and_replication():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(50).astype(np.float32)
    x[[3, 9, 11]] = np.nan
    for kq in (1, 7, 47, 48, 50):
        want = sorted(x.tolist(), key=lambda v: (math.isnan(v), v))[kq - 1]
        got = S.kth_smallest(x, kq)
        assert (math.isnan(want) and np.isnan(got)) or got == np.float32(want)
    # row grain: a [B, H, Qt] expand of a per-tile mean -> sorted_unique[(kq-1)//H]
    base = rng.standard_normal(20).astype(np.float32)
    rep = np.broadcast_to(base[None, None], (1, 7, 20))
    for kq in (1, 8, 35, 140):
        assert S.kth_smallest(rep, kq) == np.sort(base)[(kq - 1) // 7]
    assert S.quantile_rank(0.25, 57344) == 14336 and S.quantile_rank(0.0, 10) == 1


def test_router_abs_mode_triggers_all_finite():
    """Appendix quirk: sigma is ~1e-40, so abs mode with tau=0.1 triggers every finite cell."""
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 2, 64 * 10, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 64 * 10, 8)).astype(np.float32)
    cfg = S.SelectorConfig(mode="router", budget_blocks=2, k_min=1, router_mode="abs")
    sel = S.select_kv_idx_v2(q, k, 0.3, cfg)
    assert np.array_equal(sel.uncertain, ~np.isnan(sel.sigma))


def test_tile_scores_at_equals_full_tensor_rows():
    # the subset form used by the long-context spot checks (ragged last tile)
    rng = np.random.default_rng(21)
    q = rng.standard_normal((1, 4, 700, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 700, 16)).astype(np.float32)
    tiles = [0, 3, 10]
    for quest in (False, True):
        for force in (False, True):
            full = S.tile_scores(q, k, 0.3, quest, force=force)
            sub = S.tile_scores_at(q, k, 0.3, quest, tiles, force=force)
            assert np.array_equal(sub, full[:, :, tiles]), (quest, force)
    kv = S.topk_order(full, 4)[1]                     # [1, 4, 11, 4]
    base_sub, extra_sub = S.canonical_sets(kv[:, :, tiles], 2, 11, tiles=tiles)
    base_all, extra_all = S.canonical_sets(kv, 2, 11)
    pick = [h * 11 + t for h in range(4) for t in tiles]
    assert base_sub == [base_all[i] for i in pick]
    assert extra_sub == [extra_all[i] for i in pick]
