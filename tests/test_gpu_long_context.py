"""Long contexts (256K and 1M tokens, up to 16384 key blocks) on the GPU.

The Qwen2.5-7B-1M layer shape (28 / 4 heads, D=128) with router-on-Quest,
budget 64 (k_base 128, k_slots 256), q = 0.25, row grain — the configuration
of BASELINE configs[2] at 2x and 8x its length.  The oracle cannot score a
[28, 16384, 16384] tile tensor on the CPU, so the checks are the ones that
hold at any size plus spot checks of sampled tiles:

* every tile's slots 0 / 1 are the forced sink and self blocks; the base slots
  hold distinct visible blocks; sentinel NB fills slots >= k_base exactly on
  the tiles the router did not trigger;
* the router: the threshold is the k_quant-th smallest head-mean sigma (NaN
  last, H-fold replication) and the trigger flags are sigma_eff <= threshold,
  recomputed on the host from the kernel's own sigma;
* sampled tiles of sampled heads: kv_idx equal to the oracle's selection on
  the oracle's scores except for near ties, and the attention output within
  max-abs 2e-2 / mean-abs 2e-3 of the oracle over the kernel's kv_idx.
"""

import time

import numpy as np
import pytest
import torch

import sparse_attention as sa
import synth
from block_attn import attn_workspace, block_sparse_attn_v2
from oracle import attention as OA
from oracle import selector as OS
from parity import same_float_bits, score_gap_tol, unexplained_differences

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def sel_c3(budget=64):
    s = sa.Selector()
    s.kernel_v2 = True
    s.mode, s.router_score = "router", "quest"
    s.budget_blocks = budget
    s.router_mode, s.router_grain, s.router_quantile = "quantile", "row", 0.25
    return s


@pytest.mark.parametrize("S", [262144, 1048576])
def test_long_context_select_and_attention(hip_lib, S):
    print(f"[case] long context S={S}", flush=True)
    cfg = synth.CONFIGS["c3"]
    q, k, v = synth.make_layer_fast(cfg, 0, S=S)
    torch.cuda.synchronize()
    sel = sel_c3()
    nb = S // 64
    scaling = cfg.scaling
    t0 = time.perf_counter()
    # tile scores kept for the sampled-tile checks below (1M: 30 GB of fp32)
    res = sa.select_v2(q, k, scaling, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    out = torch.empty_like(q)
    block_sparse_attn_v2(q, k, v, res.kv_idx, scale=scaling, out=out,
                         workspace=attn_workspace(1, 4, S, 128, DEV))
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    print(f"  select {1e3 * (t1 - t0):.1f} ms, attention {1e3 * (t2 - t1):.1f} ms "
          f"(first call, includes launch setup)", flush=True)
    k_base, k_slots = res.k_base, res.k_slots
    assert (k_base, k_slots) == (128, 256) and res.kv_idx.shape == (1, 28, nb, k_slots)

    kv = res.kv_idx[0].cpu().numpy()                         # [H, Qt, k_slots]
    unc = res.uncertain[0].cpu().numpy().astype(bool)        # [H, Qt]
    t = np.arange(nb)
    # forced sink and self block lead every tile with t >= 1
    assert (kv[:, 1:, 0] == 0).all() and (kv[:, 1:, 1] == t[None, 1:]).all()
    # base slots: distinct visible blocks (tiles with more than k_base visible)
    base = kv[:, k_base:, :k_base]
    assert (base <= t[None, k_base:, None]).all() and (base >= 0).all()
    srt = np.sort(base, axis=-1)
    assert (np.diff(srt, axis=-1) > 0).all()
    # extra slots: sentinels exactly where the router did not trigger
    extra = kv[:, :, k_base:]
    assert ((extra == nb).all(axis=-1) == ~unc).all()
    trig = unc[:, k_slots:]
    ex = extra[:, k_slots:][trig]
    assert (ex < nb).all() and (np.diff(np.sort(ex, axis=-1), axis=-1) > 0).all()

    # three heads, every tile: the kernel's ranking against a stable sort of its
    # own scores on the GPU (ties and the -inf tail in ascending block order)
    for h in (0, 13, 27):
        srt_v, srt_i = torch.sort(res.tile_score[0, h], dim=-1, descending=True, stable=True)
        assert torch.equal(res.kv_idx[0, h, :, :k_base], srt_i[:, :k_base].int()), h
        trig_h = res.uncertain[0, h].bool()
        assert torch.equal(res.kv_idx[0, h, :, k_base:][trig_h], srt_i[:, k_base:k_slots][trig_h].int())
        vals_h = srt_v[:, :k_base + 1].cpu().numpy()[None, None]
        assert same_float_bits(res.sigma[0, h].cpu().numpy()[None, None],
                               OS.sigma_margin(vals_h, k_base)), h
        del srt_v, srt_i

    # router decisions recomputed on the host from the kernel's sigma
    sig = res.sigma.cpu().numpy()
    eff = OS.head_mean(sig)
    assert np.array_equal(eff.view(np.uint32), res.sigma_eff.cpu().numpy().view(np.uint32))
    kq = OS.quantile_rank(0.25, eff.size)
    thr = OS.kth_smallest(eff, kq)
    assert res.threshold.cpu().numpy()[0] == thr
    with np.errstate(invalid="ignore"):
        assert np.array_equal(unc, (eff <= thr)[0])
    assert not unc[:, :k_base].any()                  # NaN sigma: tiles t < k_base

    # spot checks: sampled tiles of two heads of KV group 1
    rng = np.random.default_rng(S)
    tiles = sorted(set([nb - 1, nb // 2, k_base, k_base - 1] + rng.integers(0, nb, 4).tolist()))
    kg = k[:, 1:2].float().cpu().numpy()
    vg = v[:, 1:2].float().cpu().numpy()
    ocfg = OS.SelectorConfig.from_selector(sel)
    for h in (7, 13):
        qh = q[:, h:h + 1].float().cpu().numpy()
        T = OS.tile_scores_at(qh, kg, scaling, True, tiles)          # [1, 1, n, NB]
        vals, idx = OS.topk_order(T, k_slots)
        kv_or = idx.astype(np.int32)
        kv_k = kv[h][tiles][None, None]
        trig_k = unc[h][tiles][None, None]
        kv_or[..., k_base:][~trig_k] = nb        # the oracle rows under the kernel's trigger
        T_k = res.tile_score[:, h:h + 1, tiles].cpu().numpy()
        fin = np.isfinite(T)
        assert np.array_equal(fin, np.isfinite(T_k)) and np.abs(T[fin] - T_k[fin]).max() <= 1e-5
        n_diff, bad = unexplained_differences(kv_k, kv_or, T, k_base, k_slots, tiles=tiles,
                                              tol=score_gap_tol(T, T_k))
        print(f"  head {h}: {n_diff} of {len(tiles)} sampled tiles differ, all near ties",
              flush=True)
        assert not bad
        ref = OA.gathered_attention(qh, kg, vg, kv[h][None, None], scaling, tiles=tiles)
        got = out[:, h:h + 1].float().cpu().numpy()
        for tt in tiles:
            rows = slice(64 * tt, 64 * tt + 64)
            err = np.abs(got[0, 0, rows] - ref[0, 0, rows])
            assert err.max() <= 2e-2 and err.mean() <= 2e-3, (h, tt, err.max(), err.mean())
