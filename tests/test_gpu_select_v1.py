"""GPU parity of the v1 per-row path (kernel_v2=False) against the oracle
(oracle/selector_v1.py, oracle/attention.py).

Bars:
* selection on the kernel's own fp32 row scores — keep, margins, the row-mean
  margins, threshold, trigger flags and the rollout history bit-identical to
  the oracle on those scores (belief: budgets equal unless the cumulative
  mass sits within 1e-5 of top_p);
* kernel row scores vs oracle scores from the same bf16 inputs — |dS| <=
  1e-5 * max(1, |S|) (fp32 sums of up to 2 * 256 products, in other orders);
* keep vs the reference's own masks (golden vectors): differing blocks only
  at the row's cut score (ties, and near ties within twice the row's measured
  kernel-vs-reference score gap, at least 1e-6);
* _compute_kv_idx / row masks exact; attention over a keep mask within
  max-abs 2e-2 / mean-abs 2e-3 of the fp32 oracle (head_dim 64/128/256,
  GQA, 64- and 32-row tiles, through the HF dispatcher).
"""

import numpy as np
import pytest
import torch

import sparse_attention as sa
import synth
from block_attn import _compute_kv_idx, block_sparse_attn, keep_kv_idx
from oracle import attention as OA
from oracle import selector_v1 as V1
from parity import score_gap_tol
from test_oracle_selector_v1 import CASES, load_v1, ranked, unpack_keep

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
MAX_ABS, MEAN_ABS = 2e-2, 2e-3

POLICIES = {
    "topk": dict(mode="topk"),
    "quest": dict(mode="quest"),
    "router_quest_row_q": dict(mode="router", router_score="quest", router_grain="row",
                               router_mode="quantile", router_quantile=0.25),
    "router_mean_cell_q": dict(mode="router", router_score="mean", router_grain="cell",
                               router_mode="quantile", router_quantile=0.3),
    "router_mean_row_abs": dict(mode="router", router_score="mean", router_grain="row",
                                router_mode="abs", router_tau=0.3),
    "router_quest_cell_abs": dict(mode="router", router_score="quest", router_grain="cell",
                                  router_mode="abs", router_tau=0.2),
    "belief": dict(mode="belief"),
    "belief_p05": dict(mode="belief", top_p=0.5),
    "rollout": dict(mode="rollout"),
}


def make_sel(**fields):
    s = sa.Selector()
    for k, v in fields.items():
        setattr(s, k, v)
    return s


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return a.shape == b.shape and bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


def belief_near_tie_rows(scores, top_p, tol=1e-5):
    """Rows whose sorted cumulative softmax mass passes within tol of top_p."""
    s = np.asarray(scores, np.float64)
    srt = -np.sort(-s, axis=-1)
    e = np.exp(srt - srt[..., :1])
    c = np.cumsum(e / e.sum(-1, keepdims=True), axis=-1)
    return (np.abs(c - top_p) <= tol).any(axis=-1)


def check_on_kernel_scores(res, sel, N, history=None):
    """Kernel selection == oracle selection on the kernel's own row scores."""
    T = res.scores.cpu().numpy()
    cfg = V1.SelectorV1Config.from_selector(sel)
    o = V1.select_mask_from_scores(T, N, cfg, history)
    keep = res.keep.cpu().numpy()
    diff = (keep != o.keep).any(-1)
    if cfg.mode == "belief":
        assert not (diff & ~belief_near_tie_rows(T, cfg.top_p)).any(), "belief budgets"
    else:
        assert not diff.any(), f"{int(diff.sum())} rows differ"
    if cfg.mode == "router":
        assert same_bits(res.margin.cpu().numpy(), o.margin), "margin bits"
        eff = res.margin_eff.cpu().numpy()
        want_eff = np.broadcast_to(o.margin_score, eff.shape)
        assert same_bits(eff, want_eff), "row-mean margin bits"
        assert np.array_equal(res.uncertain.cpu().numpy().astype(bool), o.uncertain)
        if cfg.router_mode == "quantile" and o.threshold is not None:
            assert res.threshold.cpu().numpy()[0] == o.threshold
    return o


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("policy", sorted(POLICIES))
def test_v1_select_exact_on_kernel_scores(hip_lib, D, policy):
    print(f"[case] v1 select D={D} policy={policy}", flush=True)
    # ragged (NB 32), aligned (NB 64), and NB 21 (keep rows not a multiple of 8 bytes)
    S = {64: 2000, 128: 4096, 256: 1300}[D]
    q, k, _ = synth.make_layer(synth.CONFIGS["c1"], 7, S=S, D=D, dtype=torch.bfloat16)
    sel = make_sel(budget_blocks=5, k_min=2, k_max=12, **POLICIES[policy])
    qd, kd = q.to(DEV), k.to(DEV)
    history = None
    for layer in range(2 if policy == "rollout" else 1):
        res = sa.select_mask_v1(qd, kd, D ** -0.5, sel=sel, want_scores=True)
        torch.cuda.synchronize()
        o = check_on_kernel_scores(res, sel, S, history)
        if policy == "rollout":
            assert same_bits(sel.selection_history.cpu().numpy(), o.history)
            history = o.history
    # kernel row scores vs the oracle's own
    cfg = V1.SelectorV1Config.from_selector(sel)
    T_or = V1.row_block_scores(q.float().numpy(), k.float().numpy(), D ** -0.5, cfg.use_quest)
    T_k = res.scores.cpu().numpy()
    fin = np.isfinite(T_or)
    assert np.array_equal(fin, np.isfinite(T_k))
    assert (np.abs(T_or[fin] - T_k[fin]) <= 1e-5 * np.maximum(1.0, np.abs(T_or[fin]))).all()


@pytest.mark.parametrize("name", CASES)
def test_v1_select_vs_reference_golden(hip_lib, name):
    """The reference's own keep masks, reproduced on the GPU up to cut ties."""
    print(f"[case] v1 golden {name}", flush=True)
    q, k, scaling, scores, pols = load_v1(name)
    qd = torch.from_numpy(q).to(torch.bfloat16).to(DEV)
    kd = torch.from_numpy(k).to(torch.bfloat16).to(DEV)
    N = k.shape[2]
    nb = (N + 63) // 64
    for pol, rec in pols.items():
        sel = make_sel(**rec["fields"])
        layers = 2 if sel.mode == "rollout" else 1
        for layer in range(layers):
            res = sa.select_mask_v1(qd, kd, scaling, sel=sel, want_scores=True)
            torch.cuda.synchronize()
            # the kernel's row scores against the reference's (before the
            # rollout penalty, which the kernel applies inside its ranking):
            # checked first, so that the cut-tie window below, twice the
            # measured gap, cannot be widened by a badly wrong row
            raw = scores[str(rec["scores"]).split("/")[1]]
            k_sc = res.scores.cpu().numpy()
            fin = np.isfinite(raw)
            assert np.array_equal(fin, np.isfinite(k_sc)), f"{pol}: finite pattern"
            assert (np.abs(raw[fin] - k_sc[fin]) <= 1e-5 * np.maximum(1.0, np.abs(raw[fin]))).all(), \
                f"{pol}: kernel row scores off the reference's"
            ref_sc = ranked(scores, rec, layer)
            keep_ref = unpack_keep(rec[f"L{layer}/keep_bits"], nb)
            keep = res.keep.cpu().numpy()
            if sel.mode == "router":
                # trigger decisions equal the reference's except where the
                # row's margin sits at the threshold
                unc = res.uncertain.cpu().numpy().astype(bool)
                o = V1.select_mask_from_scores(ref_sc, N, V1.SelectorV1Config.from_selector(sel))
                flip = unc != o.uncertain
                if flip.any():
                    m = res.margin_eff.cpu().numpy()[flip]
                    thr = res.threshold.cpu().numpy()[0]
                    assert np.all(np.abs(m - thr) <= 1e-5), f"{pol}: trigger flips off the threshold"
                rows = ~(unc | o.uncertain)
            else:
                rows = np.ones(keep.shape[:3], bool)
            diff = (keep != keep_ref) & rows[..., None]
            if sel.mode == "belief":
                # rows whose budget itself sits at a near tie of the mass
                diff &= ~belief_near_tie_rows(ref_sc, sel.top_p)[..., None]
                cfg = V1.SelectorV1Config.from_selector(sel)
                counts = V1.select_mask_from_scores(ref_sc, N, cfg).budget.astype(np.int64)
            else:
                counts = np.full(keep.shape[:3], min(int(max(min(sel.k_max, sel.budget_blocks),
                                                              sel.k_min)), nb))
            bad_rows = diff.any(-1)
            if bad_rows.any():
                srt = -np.sort(-ref_sc, axis=-1)
                cut = np.take_along_axis(srt, np.minimum(counts, nb)[..., None] - 1, axis=-1)[..., 0]
                # within twice the row's measured score gap (at least the
                # contract's 1e-6 tie window) of the cut
                tol = score_gap_tol(raw, k_sc).reshape(ref_sc.shape[:-1])
                with np.errstate(invalid="ignore"):
                    near = np.abs(ref_sc - cut[..., None]) <= tol[..., None]
                near |= np.isinf(ref_sc) & np.isinf(cut[..., None])
                assert not (diff & ~near).any(), f"{pol}/L{layer}: blocks differ off the cut"
            print(f"  {pol}/L{layer}: {int(bad_rows.sum())} rows differ at cut ties", flush=True)


@pytest.mark.parametrize("policy", ["topk", "belief", "rollout", "router_quest_row_q",
                                    "router_mean_cell_q"])
@pytest.mark.parametrize("tiles_per_pass", [1, 3])
def test_v1_multipass_equals_single_pass(hip_lib, monkeypatch, policy, tiles_per_pass):
    """Above its workspace bound the per-row selector scores rows in passes of
    whole 64-row tiles (ugbsa_select_mask: rows_t0 / rows_t1 offsets into the
    row-score buffer).  Forced down to 1 or 3 tiles per pass, with a ragged
    last tile, every output equals the single-pass run bit for bit."""
    print(f"[case] v1 multipass {policy} x{tiles_per_pass}", flush=True)
    cfg = synth.CONFIGS["c1"]
    S, D = 64 * 9 + 23, 128
    q, k, _ = synth.make_layer(cfg, 5, S=S, dtype=torch.bfloat16)
    qd, kd = q.to(DEV), k.to(DEV)
    B, H, nb = q.shape[0], q.shape[1], (S + 63) // 64
    fields = dict(budget_blocks=3, k_min=1, **POLICIES[policy])

    def run(ws_elems):
        sel = make_sel(**fields)
        res = []
        for _ in range(2 if policy == "rollout" else 1):   # the history feeds the next call
            if ws_elems is None:
                r = sa.select_mask_v1(qd, kd, D ** -0.5, sel=sel, want_scores=True)
            else:
                monkeypatch.setattr(sa, "_V1_WORKSPACE_ELEMS", ws_elems)
                r = sa.select_mask_v1(qd, kd, D ** -0.5, sel=sel)
            torch.cuda.synchronize()
            res.append(r)
        return res, sel

    one, sel1 = run(None)
    many, seln = run(B * H * 64 * nb * tiles_per_pass)
    for a, b in zip(one, many):
        assert torch.equal(a.keep, b.keep)
        for f in ("margin", "margin_eff", "uncertain", "threshold"):
            x, y = getattr(a, f), getattr(b, f)
            assert (x is None) == (y is None), f
            if x is not None:
                assert same_bits(x.cpu().numpy(), y.cpu().numpy()), f
    if policy == "rollout":
        assert same_bits(sel1.selection_history.cpu().numpy(), seln.selection_history.cpu().numpy())


def test_v1_compute_kv_idx_and_rowmask(hip_lib):
    print("[case] v1 compute_kv_idx", flush=True)
    g = torch.Generator().manual_seed(3)
    # NB a multiple of 8 (8-byte row reads, one or two 512-block spans) and not
    for (M, nb, bm) in ((1000, 16, 64), (512, 8, 32), (4096, 64, 64), (700, 11, 64),
                        (640, 600, 64), (300, 1032, 32)):
        keep = torch.rand(2, 3, M, nb, generator=g) < 0.15
        keep[..., 0] = True
        kd = keep.to(DEV)
        kv, mk = _compute_kv_idx(kd, bm)
        want_kv, want_mk = OA.compute_kv_idx(keep.numpy(), bm)
        assert mk == want_mk and np.array_equal(kv.cpu().numpy(), want_kv)
        kvf, rm, mk2 = keep_kv_idx(kd, bm)
        assert mk2 == mk
        rm = rm.cpu().numpy().view(np.uint64)
        kvf = kvf.cpu().numpy()
        kp = np.zeros((2, 3, -(-M // bm) * bm, nb), bool)
        kp[:, :, :M] = keep.numpy()
        tiles = kp.reshape(2, 3, -1, bm, nb)
        # every listed block's row mask: bit r set where tile row r keeps it
        weights = (np.uint64(1) << np.arange(bm, dtype=np.uint64))
        want_rm = (tiles.transpose(0, 1, 2, 4, 3).astype(np.uint64) * weights).sum(-1)
        blk = np.minimum(kvf, nb - 1)
        got = np.take_along_axis(want_rm, blk.astype(np.int64), axis=-1)
        got[kvf == nb] = 0
        assert np.array_equal(rm, got.astype(np.uint64))


@pytest.mark.parametrize("D,Hq,Hk,bm", [(64, 4, 2, 64), (128, 4, 1, 64), (256, 2, 1, 64),
                                        (128, 2, 2, 32)])
def test_v1_attention_over_keep(hip_lib, D, Hq, Hk, bm):
    print(f"[case] v1 attention D={D} Hq={Hq} Hk={Hk} block_m={bm}", flush=True)
    g = torch.Generator().manual_seed(D + Hq)
    S = 1500
    q = torch.randn(1, Hq, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, Hk, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, Hk, S, D, generator=g).to(torch.bfloat16)
    nb = (S + 63) // 64
    keep = torch.rand(1, Hq, S, nb, generator=g) < 0.3
    keep[..., 0] = True
    rows = torch.arange(S)
    keep[:, :, rows, rows // 64] = True
    out = block_sparse_attn(q.to(DEV), k.to(DEV), v.to(DEV), keep.to(DEV), D ** -0.5, block_m=bm)
    torch.cuda.synchronize()
    ref = OA.keep_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                            keep.numpy(), D ** -0.5)
    err = np.abs(out.float().cpu().numpy() - ref)
    print(f"  max|d|={err.max():.3e} mean|d|={err.mean():.3e}", flush=True)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS


class _Module:
    num_key_value_groups, layer_idx = 4, 0


@pytest.mark.parametrize("policy", ["topk", "router_quest_row_q", "belief", "rollout"])
def test_v1_dispatcher_end_to_end(hip_lib, policy):
    """block_sparse_attention with kernel_v2=False: the keep of the GPU
    selector (checked against the oracle) and attention over it."""
    check_v1_dispatcher(policy, torch.bfloat16)


@pytest.mark.parametrize("policy", ["topk", "router_quest_row_q"])
def test_v1_dispatcher_end_to_end_fp16(hip_lib, policy):
    """The per-row path on an fp16 layer: row scores, keep and row-masked
    attention in fp16."""
    check_v1_dispatcher(policy, torch.float16)


def check_v1_dispatcher(policy, dtype):
    print(f"[case] v1 dispatcher {policy} {dtype}", flush=True)
    cfg = synth.CONFIGS["c1"]
    q, k, v = synth.make_layer(cfg, 2, S=2048, dtype=dtype)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    saved = dict(vars(sa.SEL))
    try:
        sa.SEL.__init__()
        sa.SEL.kernel_v2 = False
        sa.SEL.log = True
        for f, val in dict(budget_blocks=4, k_min=2, **POLICIES[policy]).items():
            setattr(sa.SEL, f, val)
        hist0 = None
        out, none = sa.block_sparse_attention(_Module(), qd, kd, vd, None, cfg.scaling)
        assert none is None and out.shape == (1, 2048, 8, 128) and out.is_contiguous()
        assert out.dtype == dtype
        if policy == "rollout":
            hist1 = sa.SEL.selection_history.clone()
            sa.SEL.selection_history = hist0
        res = sa.select_mask_v1(qd, kd, cfg.scaling, want_scores=True)
        torch.cuda.synchronize()
        check_on_kernel_scores(res, sa.SEL, 2048)
        if policy == "rollout":
            assert torch.equal(sa.SEL.selection_history, hist1)
        ref = OA.keep_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                res.keep.cpu().numpy(), cfg.scaling)
        err = np.abs(out.transpose(1, 2).float().cpu().numpy() - ref)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS
        last = res.keep[0, :, -1, :]
        assert torch.equal(sa.SEL.kept_blocks[0], last.any(0).cpu())
        assert sa.SEL.budget_samples[0] == pytest.approx(float(last.sum(-1).float().mean()))
        if policy.startswith("router"):
            assert sa.SEL.router_trigger_rate[0] == pytest.approx(float(res.uncertain.float().mean()))
    finally:
        sa.SEL.__dict__.update(saved)
