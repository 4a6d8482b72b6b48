"""GPU parity of the fp16 path: kernels 1-3 and the dispatcher on fp16 inputs.

The reference runs its selector and block_sparse_attn_v2 in the model's dtype
(src/sparse_attention.py:588-748, src/triton_block_attn.py:267-298), so an
fp16 model reaches this path with fp16 q / k / v.  Bars, as for bf16:

* Quest planes exact (K-max / K-min of fp16 values); mean planes (scaled
  fp16 hi + lo, the same format as for bf16) within 2^-23 of the kernel's
  fp32 mean, itself within the fp32 summation bound of the exact mean;
* selection on the kernel's own fp32 tile scores bit-identical to the oracle;
  kernel scores within the fp32 summation-order bound of the oracle's fp32
  scores from the same fp16 values (products of two fp16 values are exact in
  fp32; only the order of the additions differs — see summation_bound);
* attention within max-abs 2e-2 / mean-abs 2e-3 of the fp32 oracle, and —
  since P is rounded to fp16 (11 significant bits) rather than bf16 (8) — at
  least 3x closer to it on average than the bf16 kernel on the same values
  rounded to bf16, which a bf16 fallback inside the fp16 path would fail.
"""

import numpy as np
import pytest
import torch

import _capi
import sparse_attention as sa
import synth
from block_attn import block_sparse_attn_v2
from oracle import attention as OA
from oracle import selector as OS
from parity import check_mean_planes, f32np, same_float_bits, summation_bound

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
MAX_ABS, MEAN_ABS = 2e-2, 2e-3


class _Module:
    num_key_value_groups = 7
    layer_idx = 0


def qkv(seed, B, H, Hk, M, N, D, dtype=torch.float16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, M, D, generator=g) * scale).to(dtype)
    k = (torch.randn(B, Hk, N, D, generator=g) * scale).to(dtype)
    v = (torch.randn(B, Hk, N, D, generator=g) * scale).to(dtype)
    return q, k, v


def err_stats(out, ref):
    e = np.abs(f32np(out) - ref)
    return float(e.max()), float(e.mean())


def run_summary(k, mode):
    """Kernel 1 on k (fp16, device): the flat summary buffer."""
    lib = _capi.lib()
    B, Hk, N, D = k.shape
    planes = torch.empty(lib.ugbsa_summary_elems(B, Hk, N, D, mode), dtype=k.dtype, device=DEV)
    _capi.check(lib.ugbsa_block_summary(k.data_ptr(), *k.stride(), B, Hk, N, D, _capi.DTYPE_F16,
                                        mode, planes.data_ptr(), _capi.stream_ptr(DEV)), "summary")
    torch.cuda.synchronize()
    return planes


@pytest.mark.parametrize("D", [64, 128, 256])
def test_block_summary_f16(hip_lib, D):
    print(f"[case] fp16 block_summary D={D}", flush=True)
    g = torch.Generator().manual_seed(D + 7)
    k = (torch.randn(2, 3, 1000, D, generator=g) * 0.3).to(torch.float16)   # ragged last block
    k[0, 0, :64, :8] = 1e-4                        # small means beside large ones in a block
    k[1, 0, 64:128] = 6e-5                         # a block of fp16 subnormal-range values
    kd = k.to(DEV)
    B, Hk, N, _ = k.shape
    nb = (N + 63) // 64
    kmin, kmax = OS.block_summaries(k.float().numpy(), True)
    pq = run_summary(kd, _capi.MODE_QUEST).view(B, Hk, nb, 2, D).float().cpu().numpy()
    assert np.array_equal(pq[..., 0, :], kmax) and np.array_equal(pq[..., 1, :], kmin)
    check_mean_planes(run_summary(kd, _capi.MODE_MEAN), k)


POLICIES = {
    "topk": dict(mode="topk"),
    "quest": dict(mode="quest"),
    "router_quest_row_q": dict(mode="router", router_score="quest", router_grain="row",
                               router_mode="quantile", router_quantile=0.25),
    "router_mean_cell_q": dict(mode="router", router_score="mean", router_grain="cell",
                               router_mode="quantile", router_quantile=0.25),
}


def make_sel(**fields):
    s = sa.Selector()
    s.kernel_v2 = True
    for k, v in fields.items():
        setattr(s, k, v)
    return s


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("policy", sorted(POLICIES))
def test_select_f16_exact_on_kernel_scores(hip_lib, D, policy):
    print(f"[case] fp16 select D={D} policy={policy}", flush=True)
    cfg = synth.CONFIGS["c1"]
    S = 2000 if D != 128 else 4096
    q, k, _ = synth.make_layer(cfg, 5, S=S, D=D, dtype=torch.float16)
    sel = make_sel(budget_blocks=4, k_min=1, **POLICIES[policy])
    res = sa.select_v2(q.to(DEV), k.to(DEV), D ** -0.5, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    T_k = res.tile_score.cpu().numpy()
    ocfg = OS.SelectorConfig.from_selector(sel)
    o = OS.select_from_tile_scores(T_k, ocfg)
    assert np.array_equal(res.kv_idx.cpu().numpy(), o.kv_idx), "kv_idx differs on the same scores"
    if o.sigma is not None:
        assert same_float_bits(res.sigma.cpu().numpy(), o.sigma)
        assert same_float_bits(res.sigma_eff.cpu().numpy(), o.sigma_eff)
        assert np.array_equal(res.uncertain.cpu().numpy().astype(bool), o.uncertain)
    T_or = OS.tile_scores(q.float().numpy(), k.float().numpy(), D ** -0.5, ocfg.use_quest)
    fin = np.isfinite(T_or)
    assert np.array_equal(fin, np.isfinite(T_k))
    tol = summation_bound(q.float().numpy(), k.float().numpy(), D ** -0.5, ocfg.use_quest)
    assert (np.abs(T_or[fin] - T_k[fin]) <= tol[fin]).all()
    print(f"  max|dT|={np.abs(T_or[fin] - T_k[fin]).max():.2e} (bar {tol[fin].min():.1e}.."
          f"{tol[fin].max():.1e})", flush=True)


def random_kv_idx(gen, B, H, qt, nb, slots, block_m=64):
    kv = torch.full((B, H, qt, slots), nb, dtype=torch.int32)
    for t in range(qt):
        self_blk = min((t * block_m + block_m - 1) // 64, nb - 1)
        for bh in range(B * H):
            b, h = divmod(bh, H)
            n_pick = int(torch.randint(0, slots - 1, (1,), generator=gen))
            pick = torch.randint(0, nb, (n_pick,), generator=gen)
            row = torch.unique(torch.cat([torch.tensor([0, self_blk]), pick]))[:slots]
            kv[b, h, t, :row.numel()] = row.to(torch.int32)
    return kv


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("block_m", [64, 32])
def test_attention_f16(hip_lib, D, block_m):
    print(f"[case] fp16 attention D={D} block_m={block_m}", flush=True)
    B, H, Hk, M = 2, 8, 2, 1000
    q, k, v = qkv(D + block_m + 1, B, H, Hk, M, M, D)
    g = torch.Generator().manual_seed(11)
    nb, qt = (M + 63) // 64, (M + block_m - 1) // block_m
    kv_idx = random_kv_idx(g, B, H, qt, nb, 6, block_m).to(DEV)
    out = block_sparse_attn_v2(q.to(DEV), k.to(DEV), v.to(DEV), kv_idx, D ** -0.5, block_m=block_m)
    assert out.dtype == torch.float16
    ref = OA.gathered_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                kv_idx.cpu().numpy(), D ** -0.5, block_m=block_m)
    mx, mean = err_stats(out, ref)
    print(f"  fp16: max|d|={mx:.3e} mean|d|={mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS
    # the same values in bf16 through the bf16 kernel: P (and the output) lose
    # three more bits, so its error against its own oracle is several times larger
    qb, kb, vb = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    outb = block_sparse_attn_v2(qb.to(DEV), kb.to(DEV), vb.to(DEV), kv_idx, D ** -0.5,
                                block_m=block_m)
    refb = OA.gathered_attention(qb.float().numpy(), kb.float().numpy(), vb.float().numpy(),
                                 kv_idx.cpu().numpy(), D ** -0.5, block_m=block_m)
    mxb, meanb = err_stats(outb, refb)
    print(f"  bf16: max|d|={mxb:.3e} mean|d|={meanb:.3e}", flush=True)
    assert mean * 3 < meanb


def test_attention_f16_large_scores(hip_lib):
    """Scores of a few hundred (|q|, |k| ~ 8 at head_dim 128): the online
    softmax moves its offsets and rescales O, all within fp16's range since
    P <= 2^8."""
    print("[case] fp16 attention large scores", flush=True)
    q, k, v = qkv(3, 1, 4, 4, 512, 512, 128, scale=8.0)
    kv_idx = torch.arange(8, dtype=torch.int32).view(1, 1, 1, 8).expand(1, 4, 8, 8).contiguous()
    out = block_sparse_attn_v2(q.to(DEV), k.to(DEV), v.to(DEV), kv_idx.to(DEV), 128 ** -0.5)
    ref = OA.causal_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), 128 ** -0.5)
    mx, mean = err_stats(out, ref)
    print(f"  max|d|={mx:.3e} mean|d|={mean:.3e}", flush=True)
    assert np.isfinite(f32np(out)).all()
    assert mx <= MAX_ABS * 8 and mean <= MEAN_ABS * 8       # |v| ~ 8: the bar scaled with it


@pytest.mark.parametrize("policy", ["quest", "router_quest"])
def test_dispatcher_f16(hip_lib, policy):
    """block_sparse_attention (HF hook) on fp16 tensors: fp16 output equal to
    the oracle's attention over the kv_idx the oracle selects on the kernel's
    own scores."""
    print(f"[case] fp16 dispatcher {policy}", flush=True)
    cfg = synth.CONFIGS["c2"]
    q, k, v = synth.make_layer(cfg, 2, S=2048, dtype=torch.float16)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    saved = dict(vars(sa.SEL))
    try:
        sa.SEL.kernel_v2 = True
        sa.SEL.budget_blocks = 8
        sa.SEL.router_grain, sa.SEL.router_mode, sa.SEL.router_quantile = "row", "quantile", 0.25
        sa.SEL.mode = "router" if policy.startswith("router") else policy
        sa.SEL.router_score = "quest"
        out, none = sa.block_sparse_attention(_Module(), qd, kd, vd, None, cfg.scaling)
        assert none is None and out.dtype == torch.float16 and out.shape == (1, 2048, 28, 128)
        res = sa.select_v2(qd, kd, cfg.scaling, want_tile_score=True)
        torch.cuda.synchronize()
        o = OS.select_from_tile_scores(res.tile_score.cpu().numpy(),
                                       OS.SelectorConfig.from_selector(sa.SEL))
        assert np.array_equal(o.kv_idx, res.kv_idx.cpu().numpy())
        heads = [0, 9, 27]
        ref = OA.gathered_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                    o.kv_idx, cfg.scaling, heads=heads)
        mx, mean = err_stats(out.transpose(1, 2)[:, heads], ref[:, heads])
        print(f"  max|d|={mx:.3e} mean|d|={mean:.3e}", flush=True)
        assert mx <= MAX_ABS and mean <= MEAN_ABS
    finally:
        sa.SEL.__dict__.update(saved)


def test_mixed_formats_rejected(hip_lib):
    q, k, v = qkv(1, 1, 2, 2, 128, 128, 64)
    kv_idx = torch.zeros(1, 2, 2, 1, dtype=torch.int32, device=DEV)
    with pytest.raises(AssertionError):
        block_sparse_attn_v2(q.to(DEV), k.to(DEV).to(torch.bfloat16), v.to(DEV), kv_idx, 0.125)
    with pytest.raises(AssertionError):
        block_sparse_attn_v2(q.to(DEV).float(), k.to(DEV).float(), v.to(DEV).float(), kv_idx, 0.125)
