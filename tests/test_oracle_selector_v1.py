"""Pins of the v1 per-row selector oracle (oracle/selector_v1.py).

Against the golden vectors written from the reference's own
``_block_select_mask`` (tests/golden/make_golden_v1.py): on the scores the
reference ranked, the oracle's keep mask is identical except where the
reference's unspecified tie order picks other blocks of the same score (the
rows' cut ties, including -inf blocks of rows with fewer visible blocks than
the budget); the router's kthvalue input, rank and threshold, the rollout
history and ``_compute_kv_idx`` are bit-identical; the oracle's own scores
match the reference's within 1e-5.  Hand-built cases pin the tie order.
"""

import ast
import os

import numpy as np
import pytest

from conftest import GOLDEN, bf16_bits_to_f32
from oracle import attention as OA
from oracle import selector_v1 as V1

CASES = ["a", "b_ragged", "c_clamp"]


def load_v1(name):
    z = np.load(os.path.join(GOLDEN, f"selector_v1_{name}.npz"))
    inp = {k: z[k] for k in z.files if "/" not in k}
    scores = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith("scores/")}
    pols = {}
    for key in z.files:
        if "/" in key and not key.startswith("scores/"):
            pol, rest = key.split("/", 1)
            pols.setdefault(pol, {})[rest] = z[key]
    for rec in pols.values():
        rec["fields"] = dict(ast.literal_eval(str(rec["fields"])))
    q = bf16_bits_to_f32(inp["q_bf16"])
    k = bf16_bits_to_f32(inp["k_bf16"])
    return q, k, float(inp["scaling"]), scores, pols


def ranked(scores, rec, layer):
    r = scores[str(rec["scores"]).split("/")[1]].copy()
    rows_key = f"L{layer}/ranked_rows"
    if rows_key in rec:
        r[:, :, rec[rows_key]] = rec[f"L{layer}/ranked_at_rows"]
    return r


def unpack_keep(bits, nb):
    return np.unpackbits(bits, axis=-1)[..., :nb].astype(bool)


def cut_values(scores, counts):
    """Per row: the counts-th largest score (the top-k / rank < budget cut)."""
    srt = -np.sort(-scores, axis=-1)
    c = np.clip(np.asarray(counts, np.int64) - 1, 0, scores.shape[-1] - 1)
    c = np.broadcast_to(c, scores.shape[:-1])
    return np.take_along_axis(srt, c[..., None], axis=-1)[..., 0]


def assert_keep_equal_up_to_ties(keep_a, keep_b, scores, counts, uncertain=None):
    diff = keep_a != keep_b
    rows = diff.any(axis=-1)
    if uncertain is not None:
        assert not (rows & uncertain).any(), "uncertain rows must equal the visible mask"
    if not rows.any():
        return 0
    cut = cut_values(scores, counts)
    bad = diff & (scores != cut[..., None])
    assert not bad.any(), f"{int(bad.any(axis=-1).sum())} rows differ beyond cut ties"
    return int(rows.sum())


@pytest.mark.parametrize("name", CASES)
def test_v1_oracle_on_reference_scores(name):
    q, k, scaling, scores, pols = load_v1(name)
    M, N = q.shape[2], k.shape[2]
    nb = (N + 63) // 64
    visible, _ = V1.row_visibility(M, N)
    for pol, rec in pols.items():
        cfg = V1.SelectorV1Config(**{f: v for f, v in rec["fields"].items()
                                     if f in V1.SelectorV1Config.__dataclass_fields__})
        layers = 2 if cfg.mode == "rollout" else 1
        history = None
        base = ranked(scores, rec, 0)
        for layer in range(layers):
            sel = V1.select_mask_from_scores(base, N, cfg, history)
            ref_ranked = ranked(scores, rec, layer)
            assert np.array_equal(sel.score_for_sel, ref_ranked), (pol, layer)
            keep_ref = unpack_keep(rec[f"L{layer}/keep_bits"], nb)
            if cfg.mode == "belief":
                counts = sel.budget
            else:
                counts = min(int(max(min(cfg.k_max, cfg.budget_blocks), cfg.k_min)), nb)
            n = assert_keep_equal_up_to_ties(sel.keep, keep_ref, sel.score_for_sel, counts,
                                             sel.uncertain)
            print(f"{name}/{pol}/L{layer}: {n} rows differ only by cut ties")
            if cfg.mode == "router" and cfg.router_mode == "quantile":
                assert np.array_equal(sel.m_safe.ravel(), rec[f"L{layer}/kth_in"].ravel())
                assert sel.k_quant == int(rec[f"L{layer}/kth_k"])
                assert sel.threshold == rec[f"L{layer}/kth_out"]
            if cfg.mode == "rollout":
                assert np.array_equal(sel.history, rec[f"L{layer}/history"]), (pol, layer)
                history = sel.history
            # _compute_kv_idx on the reference's own mask
            kv, mk = OA.compute_kv_idx(keep_ref, 64)
            assert mk == int(rec[f"L{layer}/max_kept"])
            assert np.array_equal(kv, rec[f"L{layer}/kv_idx"])
        # SEL.log diagnostics, recomputed from the reference's masks
        for layer in range(layers):
            keep_ref = unpack_keep(rec[f"L{layer}/keep_bits"], nb)
            last = keep_ref[0, :, -1, :]
            assert np.array_equal(rec["log/kept_blocks"][layer], last.any(axis=0))
            assert rec["log/budget_samples"][layer] == pytest.approx(last.sum(-1).mean())
        if cfg.mode == "router":
            sel = V1.select_mask_from_scores(base, N, cfg)
            keep_ref = unpack_keep(rec["L0/keep_bits"], nb)
            assert rec["log/router_trigger_rate"][0] == pytest.approx(sel.uncertain.mean())
            assert rec["log/router_eff_budget"][0] == pytest.approx(keep_ref.sum(-1).mean())
            mm = rec["log/router_margin_mean"][0]
            assert (np.isnan(mm) and np.isnan(sel.margin).any()) or \
                mm == pytest.approx(float(sel.margin.astype(np.float64).mean()), rel=1e-5)


@pytest.mark.parametrize("name", CASES)
def test_v1_oracle_scores_from_scratch(name):
    q, k, scaling, scores, pols = load_v1(name)
    for backbone, ref in scores.items():
        got = V1.row_block_scores(q, k, scaling, backbone == "quest")
        fin = np.isfinite(ref)
        assert np.array_equal(fin, np.isfinite(got))
        assert np.abs(got[fin] - ref[fin]).max() <= 1e-5, backbone


def test_v1_tie_order_and_short_rows_by_hand():
    # all scores tie: the budget takes the lowest blocks, then sink / own block
    M = N = 640
    nb = 10
    s = np.zeros((1, 1, M, nb), np.float32)
    visible, qg = V1.row_visibility(M, N)
    s[:, :, ~visible] = -np.inf
    cfg = V1.SelectorV1Config(mode="topk", budget_blocks=3, k_min=1)
    keep = V1.select_mask_from_scores(s, N, cfg).keep[0, 0]
    # row 639 (all 10 visible): blocks 0, 1, 2 plus its own block 9
    assert np.nonzero(keep[639])[0].tolist() == [0, 1, 2, 9]
    # row 70 (blocks 0, 1 visible): both, plus the lowest invisible block 2
    assert np.nonzero(keep[70])[0].tolist() == [0, 1, 2]
    # belief on equal scores: mass 1/n per block, budget = #(cumsum < p) + 1
    cfg = V1.SelectorV1Config(mode="belief", top_p=0.5, k_min=1, k_max=112)
    sel = V1.select_mask_from_scores(s, N, cfg)
    assert sel.budget[0, 0, 639] == 5.0      # cumsum 0.1..0.4 < 0.5, 0.5 is not
    assert np.nonzero(sel.keep[0, 0, 639])[0].tolist() == [0, 1, 2, 3, 4, 9]


def test_v1_router_quantile_rule_by_hand():
    # row grain: n_elig counts rows, the kth value runs over B * M entries,
    # ineligible rows and NaN margins rank as +inf
    rng = np.random.default_rng(4)
    M = N = 512
    s = rng.standard_normal((1, 2, M, 8)).astype(np.float32)
    visible, _ = V1.row_visibility(M, N)
    s[:, :, ~visible] = -np.inf
    cfg = V1.SelectorV1Config(mode="router", budget_blocks=3, k_min=1, router_mode="quantile",
                              router_grain="row", router_quantile=0.5)
    sel = V1.select_mask_from_scores(s, N, cfg)
    elig = visible.sum(-1) > 3                      # rows 192 .. 511
    assert np.array_equal(sel.eligible, elig) and sel.k_quant == int(0.5 * elig.sum())
    m = sel.margin_score[0, 0]
    assert np.isinf(sel.m_safe[0, 0][~elig]).all()
    want = np.float32(sorted(np.where(elig, m, np.inf))[sel.k_quant - 1])
    assert sel.threshold == want
    assert np.array_equal(sel.uncertain[0, 0], (m <= want) & elig)
    unc_rows = np.nonzero(sel.uncertain[0, 0])[0]
    assert np.array_equal(sel.keep[0, 1, unc_rows], visible[unc_rows])
