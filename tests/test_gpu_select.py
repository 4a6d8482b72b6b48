"""GPU parity of kernels 1, 2 and the router against the CPU oracle.

Bars:
* block summaries — Quest planes bit-exact (min/max of bf16 with F.pad zeros);
  mean planes: scaled fp16 hi + lo within 2^-23 of the kernel's fp32 mean,
  itself within the fp32 summation bound of the exact mean;
* selection on the kernel's own fp32 tile scores — kv_idx, sigma, sigma_eff,
  trigger flags and threshold bit-identical to the oracle run on those scores;
* kernel scores vs oracle scores from the same bf16 inputs — max |dT| <= 1e-5;
* kv_idx vs the oracle from scratch and vs the reference's golden vectors —
  equal except rows explained by near ties (tests/parity.py).
"""

import numpy as np
import pytest
import torch

import _capi
import sparse_attention as sa
import synth
from conftest import load_golden
from block_attn import block_sparse_attn_v2
from oracle import attention as OA
from oracle import selector as OS
from parity import (check_mean_planes, f32np, same_float_bits, score_gap_tol, summation_bound,
                    unexplained_differences)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def make_sel(**fields):
    s = sa.Selector()
    s.kernel_v2 = True
    for k, v in fields.items():
        setattr(s, k, v)
    return s


def run_summary(k, mode):
    """Kernel 1 on k (bf16, device): the flat summary buffer."""
    lib = _capi.lib()
    B, Hk, N, D = k.shape
    planes = torch.empty(lib.ugbsa_summary_elems(B, Hk, N, D, mode), dtype=torch.bfloat16, device=DEV)
    _capi.check(lib.ugbsa_block_summary(k.data_ptr(), *k.stride(), B, Hk, N, D, _capi.DTYPE_BF16,
                                        mode, planes.data_ptr(), _capi.stream_ptr(DEV)), "summary")
    torch.cuda.synchronize()
    return planes


@pytest.mark.parametrize("D", [64, 128, 256])
def test_block_summary(hip_lib, D):
    print(f"[case] block_summary D={D}", flush=True)
    g = torch.Generator().manual_seed(D)
    k = torch.randn(2, 3, 1000, D, generator=g)                          # ragged last block
    # blocks of very different magnitudes (each block's own scale), an
    # all-zero block and one of mixed signs around zero
    k *= torch.pow(2.0, torch.randint(-30, 31, (2, 3, 16, 1), generator=g).float()
                   ).repeat_interleave(64, 2)[:, :, :1000]
    k[1, 2, 128:192] = 0
    k[0, 1, 64:128] = torch.tensor([1.0, -1.0]).repeat(32).view(64, 1)
    k = k.to(torch.bfloat16)
    kd = k.to(DEV)
    B, Hk, N, _ = k.shape
    nb = (N + 63) // 64
    kmin, kmax = OS.block_summaries(k.float().numpy(), True)
    pq = run_summary(kd, _capi.MODE_QUEST).view(B, Hk, nb, 2, D).float().cpu().numpy()
    assert np.array_equal(pq[..., 0, :], kmax) and np.array_equal(pq[..., 1, :], kmin)
    rec = check_mean_planes(run_summary(kd, _capi.MODE_MEAN), k)
    # the decoder the v1 path uses agrees with the test's own
    means = sa.block_means(run_summary(kd, _capi.MODE_MEAN), B, Hk, nb, D).double().cpu().numpy()
    assert np.allclose(means, rec, rtol=2.0 ** -22, atol=0)


POLICIES = {
    "topk": dict(mode="topk"),
    "quest": dict(mode="quest"),
    "router_quest_row_q": dict(mode="router", router_score="quest", router_grain="row",
                               router_mode="quantile", router_quantile=0.25),
    "router_mean_row_q": dict(mode="router", router_score="mean", router_grain="row",
                              router_mode="quantile", router_quantile=0.25),
    "router_quest_cell_q": dict(mode="router", router_score="quest", router_grain="cell",
                                router_mode="quantile", router_quantile=0.25),
    "router_mean_cell_abs": dict(mode="router", router_score="mean", router_grain="cell",
                                 router_mode="abs"),
    "router_quest_row_q090": dict(mode="router", router_score="quest", router_grain="row",
                                  router_mode="quantile", router_quantile=0.90),
}


def gpu_vs_oracle_on_kernel_scores(q, k, scaling, sel):
    res = sa.select_v2(q.to(DEV), k.to(DEV), scaling, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    T = res.tile_score.cpu().numpy()
    ocfg = OS.SelectorConfig.from_selector(sel)
    o = OS.select_from_tile_scores(T, ocfg)
    assert np.array_equal(res.kv_idx.cpu().numpy(), o.kv_idx), "kv_idx differs on the same scores"
    if o.sigma is not None:
        assert same_float_bits(res.sigma.cpu().numpy(), o.sigma), "sigma bits"
        assert same_float_bits(res.sigma_eff.cpu().numpy(), o.sigma_eff), "sigma_eff bits"
        assert np.array_equal(res.uncertain.cpu().numpy().astype(bool), o.uncertain)
        if o.threshold is not None:
            thr = res.threshold.cpu().numpy()[0]
            assert (np.isnan(thr) and np.isnan(o.threshold)) or same_float_bits(thr, o.threshold)
    return res, o


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("policy", sorted(POLICIES))
def test_select_exact_on_kernel_scores(hip_lib, D, policy):
    print(f"[case] select D={D} policy={policy}", flush=True)
    cfg = synth.CONFIGS["c1"]
    S = 2000 if D != 128 else 4096                       # ragged and aligned
    q, k, _ = synth.make_layer(cfg, 3, S=S, D=D, dtype=torch.bfloat16)
    sel = make_sel(budget_blocks=4, k_min=1, **POLICIES[policy])
    res, o = gpu_vs_oracle_on_kernel_scores(q, k, D ** -0.5, sel)
    # scores agree with the oracle's independent fp32 scores
    T_or = OS.tile_scores(q.float().numpy(), k.float().numpy(), D ** -0.5,
                          OS.SelectorConfig.from_selector(sel).use_quest)
    T_k = res.tile_score.cpu().numpy()
    fin = np.isfinite(T_or)
    assert np.array_equal(fin, np.isfinite(T_k))
    assert np.abs(T_or[fin] - T_k[fin]).max() <= 1e-5


@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("policy", ["quest", "router_mean_row_q"])
def test_select_pair_blocks_batch_and_ragged_groups(hip_lib, D, policy):
    """Select workgroups take consecutive (tile, query head) pairs of one (b,
    KV head): with B = 2, Hk = 3 and 5 query heads per KV head over 15 tiles
    (75 pairs per KV head), workgroups span two tiles and the last one of each
    (b, KV head) holds fewer pairs than waves.  kv_idx and sigma bit-exact on
    the kernel's own scores; the scores within the fp32 summation-order
    bound of the oracle's."""
    print(f"[case] select pair blocks D={D} policy={policy}", flush=True)
    g = torch.Generator().manual_seed(D)
    B, H, Hk, S = 2, 15, 3, 900
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    sel = make_sel(budget_blocks=2, k_min=1, **POLICIES[policy])
    res, _ = gpu_vs_oracle_on_kernel_scores(q, k, D ** -0.5, sel)
    quest = OS.SelectorConfig.from_selector(sel).use_quest
    T_or = OS.tile_scores(q.float().numpy(), k.float().numpy(), D ** -0.5, quest)
    T_k = res.tile_score.cpu().numpy()
    fin = np.isfinite(T_or)
    assert np.array_equal(fin, np.isfinite(T_k))
    # unit-normal inputs give scores of ~30, where the fp32 summation order
    # alone moves a score by more than the synthetic layers' 1e-5
    tol = summation_bound(q.float().numpy(), k.float().numpy(), D ** -0.5, quest)
    assert (np.abs(T_or[fin] - T_k[fin]) <= tol[fin]).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("policy", ["topk", "router_mean_row_q"])
def test_select_mean_planes_wide_magnitudes(hip_lib, dtype, D, policy):
    """K-mean scoring with Q tiles and K blocks whose magnitudes span many
    octaves (bf16: 2^-20 .. 2^20 per tile / block, rows within a tile over
    2^-8 .. 1; fp16: 2^-6 .. 2^6), so that the per-block plane scales and the
    per-tile Q scales move far from 1 and differ between neighbours: kv_idx /
    sigma bit-exact on the kernel's own scores, and the scores within the
    fp32 summation-order bound of the oracle's (relative to the terms' size)."""
    print(f"[case] select wide magnitudes dtype={dtype} D={D} policy={policy}", flush=True)
    g = torch.Generator().manual_seed(D + (7 if dtype == torch.float16 else 0))
    B, H, Hk, S = 1, 4, 2, 1500
    span = 20 if dtype == torch.bfloat16 else 6
    nb = (S + 63) // 64
    tile_sc = torch.pow(2.0, torch.randint(-span, span + 1, (B, H, nb, 1), generator=g).float())
    row_sc = torch.pow(2.0, torch.randint(-8, 1, (B, H, nb * 64, 1), generator=g).float())
    blk_sc = torch.pow(2.0, torch.randint(-span, span + 1, (B, Hk, nb, 1), generator=g).float())
    q = torch.randn(B, H, S, D, generator=g) * (tile_sc.repeat_interleave(64, 2) * row_sc)[:, :, :S]
    k = torch.randn(B, Hk, S, D, generator=g) * blk_sc.repeat_interleave(64, 2)[:, :, :S]
    q, k = q.to(dtype), k.to(dtype)
    sel = make_sel(budget_blocks=3, k_min=1, **POLICIES[policy])
    res, _ = gpu_vs_oracle_on_kernel_scores(q, k, D ** -0.5, sel)
    T_or = OS.tile_scores(q.float().numpy(), k.float().numpy(), D ** -0.5, False)
    T_k = res.tile_score.cpu().numpy()
    fin = np.isfinite(T_or)
    assert np.array_equal(fin, np.isfinite(T_k))
    tol = summation_bound(q.float().numpy(), k.float().numpy(), D ** -0.5, False)
    d = np.abs(T_or[fin].astype(np.float64) - T_k[fin])
    assert (d <= tol[fin]).all(), (d.max(), (d / tol[fin]).max())
    print(f"  max |dT| / bound = {(d / tol[fin]).max():.3f}", flush=True)


@pytest.mark.parametrize("name", ["a", "b_ragged", "c_full"])
def test_select_vs_reference_golden(hip_lib, name):
    """The reference's own kv_idx (fp32 CPU run) reproduced on the GPU."""
    print(f"[case] golden {name}", flush=True)
    inp, pols = load_golden(name)
    q = torch.from_numpy(inp["q"]).to(torch.bfloat16)   # exact: inputs are bf16 values
    k = torch.from_numpy(inp["k"]).to(torch.bfloat16)
    for pol, rec in pols.items():
        fields = {f: v for f, v in rec["fields"].items()}
        sel = make_sel(**fields)
        res, o = gpu_vs_oracle_on_kernel_scores(q, k, float(inp["scaling"]), sel)
        T_ref = rec["tile_score"]
        fin = np.isfinite(T_ref)
        assert np.abs(T_ref[fin] - res.tile_score.cpu().numpy()[fin]).max() <= 1e-5, pol
        ref = OS.select_from_tile_scores(T_ref, OS.SelectorConfig.from_selector(sel))
        n_diff, bad = unexplained_differences(
            res.kv_idx.cpu().numpy(), rec["kv_idx"], T_ref, ref.k_base, ref.k_slots,
            trig_a=None if res.uncertain is None else res.uncertain.cpu().numpy(),
            trig_b=ref.uncertain,
            sig_a=None if res.sigma_eff is None else res.sigma_eff.cpu().numpy(),
            sig_b=ref.sigma_eff,
            thr_a=None if res.threshold is None else res.threshold.cpu().numpy()[0],
            thr_b=ref.threshold, tol=score_gap_tol(T_ref, res.tile_score.cpu().numpy()))
        assert not bad, f"{pol}: {len(bad)} unexplained rows of {n_diff} differing"


def test_select_c1_full_config(hip_lib):
    """BASELINE configs[0] layer (S=8192, 8/2 heads, D=128) in bf16 on the GPU."""
    print("[case] select c1 full", flush=True)
    cfg = synth.CONFIGS["c1"]
    q, k, _ = synth.make_layer(cfg, 0, dtype=torch.bfloat16)
    sel = make_sel(**cfg.sel_fields())
    res, o = gpu_vs_oracle_on_kernel_scores(q, k, cfg.scaling, sel)
    assert res.kv_idx.shape == (1, 8, 128, 32)
    orc = OS.select_kv_idx_v2(q.float().numpy(), k.float().numpy(), cfg.scaling,
                              OS.SelectorConfig.from_selector(sel))
    n_diff, bad = unexplained_differences(
        res.kv_idx.cpu().numpy(), orc.kv_idx, orc.tile_score, orc.k_base, orc.k_slots,
        res.uncertain.cpu().numpy(), orc.uncertain, res.sigma_eff.cpu().numpy(),
        orc.sigma_eff, res.threshold.cpu().numpy()[0], orc.threshold,
        tol=score_gap_tol(orc.tile_score, res.tile_score.cpu().numpy()))
    assert not bad, f"{len(bad)} unexplained rows of {n_diff}"
    assert float(res.uncertain.float().mean()) == 0.25
    # attention over the kernel's kv_idx at the full layer shape: every head
    # and tile against the fp32 oracle
    _, _, v = synth.make_layer(cfg, 0, dtype=torch.bfloat16)
    out = block_sparse_attn_v2(q.to(DEV), k.to(DEV), v.to(DEV), res.kv_idx, cfg.scaling)
    ref = OA.gathered_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                res.kv_idx.cpu().numpy(), cfg.scaling)
    err = np.abs(out.float().cpu().numpy() - ref)
    print(f"  c1 attention: max {err.max():.2e} mean {err.mean():.2e}", flush=True)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3


def test_select_c2_full_config(hip_lib):
    """BASELINE configs[1] layer: S=32768, 28/4 heads, D=128, router-on-Quest 64 -> 128."""
    print("[case] select c2 full", flush=True)
    cfg = synth.CONFIGS["c2"]
    q, k, _ = synth.make_layer(cfg, 0)
    sel = make_sel(**cfg.sel_fields())
    res, o = gpu_vs_oracle_on_kernel_scores(q, k, cfg.scaling, sel)
    assert res.kv_idx.shape == (1, 28, 512, 128) and (res.k_base, res.k_slots) == (64, 128)
    # oracle scores from scratch for one KV group (7 query heads)
    ocfg = OS.SelectorConfig.from_selector(sel)
    T_or = OS.tile_scores(q[:, :7].float().numpy(), k[:, :1].float().numpy(), cfg.scaling, True)
    T_k = res.tile_score[:, :7].cpu().numpy()
    fin = np.isfinite(T_or)
    assert np.abs(T_or[fin] - T_k[fin]).max() <= 1e-5
    # every head and tile: the kernel's ranking against a stable sort of its
    # own scores on the GPU (ties and the -inf tail in ascending block order)
    srt_v, srt_i = torch.sort(res.tile_score[0].to(DEV), dim=-1, descending=True, stable=True)
    kv_dev = res.kv_idx[0]
    assert torch.equal(kv_dev[..., :res.k_base], srt_i[..., :res.k_base].int())
    unc_dev = res.uncertain[0].bool()
    assert torch.equal(kv_dev[..., res.k_base:][unc_dev],
                       srt_i[..., res.k_base:res.k_slots][unc_dev].int())
    del srt_v, srt_i
    # from-scratch selection of those heads under the kernel's trigger flags
    k_base, k_slots = res.k_base, res.k_slots
    _, idx_or = OS.topk_order(T_or, k_slots)
    kv_or = idx_or.astype(np.int32)
    trig = res.uncertain[:, :7].cpu().numpy().astype(bool)
    kv_or[..., k_base:][~trig] = T_or.shape[-1]
    n_diff, bad = unexplained_differences(res.kv_idx[:, :7].cpu().numpy(), kv_or, T_or, k_base,
                                          k_slots, tol=score_gap_tol(T_or, T_k))
    print(f"  c2 group 0: {n_diff} of {kv_or.shape[1] * kv_or.shape[2]} tiles differ, "
          f"unexplained {len(bad)}", flush=True)
    assert not bad
    # trigger fraction: kq = int(0.25 * 28 * 512) = 3584 -> 128 tiles of 448 eligible
    trig_tiles = res.uncertain[0, 0].cpu().numpy().astype(bool)
    assert trig_tiles.sum() >= 128 and not trig_tiles[:64].any()


def test_router_kernel_edge_cases(hip_lib):
    """Row/cell grain, NaN threshold, abs mode on hand-built sigma arrays."""
    print("[case] router edges", flush=True)
    lib = _capi.lib()
    rng = np.random.default_rng(0)
    B, H, Qt, kb, ks, nb = 2, 3, 40, 4, 8, 64
    for grain in (_capi.GRAIN_ROW, _capi.GRAIN_CELL):
        for rmode, qfrac in ((_capi.ROUTER_QUANTILE, 0.3), (_capi.ROUTER_QUANTILE, 0.99),
                             (_capi.ROUTER_ABS, 0.0)):
            sig = (rng.integers(0, 50, (B, H, Qt)) * OS.sigma_quantum()).astype(np.float32)
            sig[:, :, :5] = np.nan
            kv = np.tile(np.arange(ks, dtype=np.int32), (B, H, Qt, 1))
            tau = 20 * OS.sigma_quantum()
            sd = torch.from_numpy(sig).to(DEV)
            kvd = torch.from_numpy(kv).to(DEV)
            eff = torch.empty_like(sd)
            unc = torch.empty(sd.shape, dtype=torch.uint8, device=DEV)
            thr = torch.empty(1, device=DEV)
            kq = max(1, int(qfrac * sig.size))
            _capi.check(lib.ugbsa_router(sd.data_ptr(), B, H, Qt, grain, rmode, tau, kq,
                                         kvd.data_ptr(), kb, ks, nb, eff.data_ptr(),
                                         unc.data_ptr(), thr.data_ptr(), _capi.stream_ptr(DEV)),
                        "router")
            torch.cuda.synchronize()
            want_eff = OS.head_mean(sig) if grain == _capi.GRAIN_ROW else sig
            assert same_float_bits(eff.cpu().numpy(), want_eff)
            if rmode == _capi.ROUTER_QUANTILE:
                want_thr = OS.kth_smallest(want_eff, kq)
                got = thr.cpu().numpy()[0]
                assert (np.isnan(want_thr) and np.isnan(got)) or got == want_thr
                with np.errstate(invalid="ignore"):
                    want_unc = want_eff <= want_thr
            else:
                with np.errstate(invalid="ignore"):
                    want_unc = want_eff < np.float32(tau)
            assert np.array_equal(unc.cpu().numpy().astype(bool), want_unc)
            want_kv = kv.copy()
            want_kv[..., kb:][~want_unc] = nb
            assert np.array_equal(kvd.cpu().numpy(), want_kv)


@pytest.mark.parametrize("case", ["random", "all_ties", "few_values"])
def test_select_streaming_rows_exact(hip_lib, case):
    """Rows past 4096 blocks select by streaming candidates (bounded LDS):
    kv_idx / sigma bit-identical to the oracle on the kernel's own scores,
    including rows where most scores tie (cut ties go to the lowest block)."""
    print(f"[case] select streaming {case}", flush=True)
    nb = 4097
    S = nb * 64
    g = torch.Generator().manual_seed(77)
    q = torch.randn(1, 2, S, 64, generator=g)
    k = torch.randn(1, 1, S, 64, generator=g)
    if case == "all_ties":
        q.zero_()                                     # every unforced score is 0
    elif case == "few_values":
        q = torch.randint(-1, 2, q.shape, generator=g).float() * 0.5
        k = torch.randint(-1, 2, k.shape, generator=g).float()
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    for fields in (dict(mode="quest", budget_blocks=32),
                   dict(mode="router", router_score="quest", budget_blocks=32,
                        router_grain="row", router_mode="quantile", router_quantile=0.25)):
        sel = make_sel(**fields)
        res, o = gpu_vs_oracle_on_kernel_scores(q, k, 0.125, sel)
        if case == "all_ties":
            kv = res.kv_idx[0, 0, -1].cpu().numpy()
            assert kv[0] == 0 and kv[1] == nb - 1 and list(kv[2:64]) == list(range(1, 63))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("policy", ["topk", "router_mean_row_q"])
@pytest.mark.parametrize("nb", [3000, 4097])
def test_select_long_rows_mean_planes_d256(hip_lib, policy, dtype, nb):
    """Long rows at head_dim 256 with the mean planes (16.6 KiB plane
    chunks): 3000 blocks keep the row in LDS (12 KiB per wave) and the
    launcher stages the chunks through one buffer (a second barrier per
    chunk), so that two workgroups share a CU; 4097 blocks stream their
    candidates.  kv_idx / sigma bit-identical to the oracle on the kernel's
    own scores."""
    print(f"[case] select long rows D=256 nb={nb} policy={policy} dtype={dtype}", flush=True)
    S = nb * 64
    g = torch.Generator().manual_seed(78)
    q = torch.randn(1, 2, S, 256, generator=g).to(dtype)
    k = torch.randn(1, 1, S, 256, generator=g).to(dtype)
    sel = make_sel(budget_blocks=32, **POLICIES[policy])
    res, _ = gpu_vs_oracle_on_kernel_scores(q, k, 256 ** -0.5, sel)
    assert res.kv_idx.shape[-1] == (128 if policy.startswith("router") else 64)


@pytest.mark.parametrize("S", [1, 37, 64, 65, 130, 200])
@pytest.mark.parametrize("policy", ["topk", "router_quest_row_q", "router_mean_cell_abs"])
def test_tiny_shapes_select_and_attention(hip_lib, S, policy):
    """One or a few key blocks (S from 1 token to 4 blocks, ragged): budgets
    clamp to NB (k_base = k_slots = NB, the router then has nothing to add and
    is skipped, as the reference's k_base < k_slots test does), selection is
    bit-exact on the kernel's own scores and the attention over its kv_idx
    matches the oracle; a single token attends to itself only."""
    print(f"[case] tiny S={S} policy={policy}", flush=True)
    g = torch.Generator().manual_seed(S)
    B, H, Hk, D = 1, 4, 2, 128
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16)
    sel = make_sel(budget_blocks=1, k_min=1, **POLICIES[policy])
    nb = (S + 63) // 64
    k_base, k_slots = sa.budgets(nb, sel)
    assert k_base == min(2, nb) and k_slots == (min(2 * k_base, nb) if sel.mode == "router" else k_base)
    res, _ = gpu_vs_oracle_on_kernel_scores(q, k, D ** -0.5, sel)
    assert (res.sigma is None) == (k_base == k_slots or sel.mode != "router")
    kv = res.kv_idx
    out = block_sparse_attn_v2(q.to(DEV), k.to(DEV), v.to(DEV), kv, D ** -0.5)
    ref = OA.gathered_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                kv.cpu().numpy(), D ** -0.5)
    err = np.abs(f32np(out) - ref)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    if S == 1:
        assert torch.equal(out[0, :, 0].cpu(), v[0].repeat_interleave(H // Hk, dim=0)[:, 0])
