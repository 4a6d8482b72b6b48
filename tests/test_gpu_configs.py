"""BASELINE configs[2..4] at their full layer shapes on the GPU.

c3  Qwen2.5-7B-1M at 128K (28 / 4 heads, D=128), router-on-Quest 128 -> 256;
c4  Qwen2.5-14B at 64K (40 / 8 heads, D=128, 5 % outlier K channels at 4x),
    both backbones (K-mean top-k, Quest) with and without the router, 96 (-> 192);
c5  Qwen3.6-style at 128K (16 / 2 heads, D=256, QK-Norm), router-on-K-mean
    128 -> 256.

The CPU oracle cannot rank a full [H, Qt, NB] tile tensor of these layers
inside a GPU test (c3: 57344 rows of 2048 blocks), so each layer is checked
the way that holds at any size, and on samples where a full check does not fit:

* kernel 2's own fp32 tile scores of two sampled heads, all tiles: the
  oracle's top-k of those rows reproduces the kernel's base slots exactly,
  and (router) its sigma margins bit for bit;
* the same on every head and tile, with a stable descending torch.sort of
  the kernel's scores on the GPU as the independent ranking (ties and the
  -inf tail in ascending block order, as the contract's total order): base
  and extra slots equal slot for slot, and sigma recomputed from the sorted
  values in IEEE fp32 on the host equal bit for bit;
* the router on the kernel's sigma of every head: the head mean, the
  k_quant-th smallest threshold and the trigger flags recomputed on the host
  bit for bit; sentinel NB exactly on the untriggered tiles, and the oracle's
  slots k_base .. k_slots on the triggered tiles of the sampled heads;
* sampled tiles: kernel scores within 1e-5 of the oracle's scores from the
  bf16 inputs, kv_idx equal to the oracle's from-scratch selection except
  near ties, and the attention output within max-abs 2e-2 / mean-abs 2e-3 of
  the fp32 oracle over the kernel's kv_idx;
* the attention of the whole layer under its real launch schedule: an output
  buffer pre-filled with NaN is finite everywhere afterwards (every row of
  every head written), and one query head of every KV group matches the fp32
  oracle on every tile (the oracle run over tile chunks on a thread pool).

Inputs come from ``synth.make_layer_fast`` (seeded, on the device), the same
generator bench.py times.
"""

import numpy as np
import pytest
import torch

import sparse_attention as sa
import synth
from block_attn import block_sparse_attn_v2
from oracle import attention as OA
from oracle import selector as OS
from parity import (check_attention_rows, oracle_heads, same_float_bits, score_gap_tol,
                    unexplained_differences)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

C4_POLICIES = {
    "topk_mean": dict(mode="topk"),
    "quest": dict(mode="quest"),
    "router_mean": dict(mode="router", router_score="mean"),
    "router_quest": dict(mode="router", router_score="quest"),
}

CASES = [("c3", None), ("c5", None)] + [("c4", p) for p in sorted(C4_POLICIES)]


def selector_for(cfg, policy):
    s = sa.Selector()
    s.kernel_v2 = True
    for f, val in cfg.sel_fields().items():
        setattr(s, f, val)
    if policy is not None:
        for f, val in C4_POLICIES[policy].items():
            setattr(s, f, val)
    return s


@pytest.fixture(scope="module")
def layers():
    cache = {}

    def get(name):
        if name not in cache:
            cache.clear()
            torch.cuda.empty_cache()
            cache[name] = synth.make_layer_fast(synth.CONFIGS[name], 0, device=DEV)
        return cache[name]
    yield get
    cache.clear()


@pytest.mark.parametrize("name,policy", CASES, ids=[f"{n}-{p}" if p else n for n, p in CASES])
def test_full_config_layer(hip_lib, layers, name, policy):
    print(f"[case] full config {name} policy={policy}", flush=True)
    cfg = synth.CONFIGS[name]
    q, k, v = layers(name)
    sel = selector_for(cfg, policy)
    ocfg = OS.SelectorConfig.from_selector(sel)
    nb = cfg.S // 64
    grp = cfg.Hq // cfg.Hkv
    res = sa.select_v2(q, k, cfg.scaling, sel=sel, want_tile_score=True)
    out = block_sparse_attn_v2(q, k, v, res.kv_idx, cfg.scaling)
    torch.cuda.synchronize()
    k_base, k_slots = res.k_base, res.k_slots
    router = sel.mode == "router"
    assert k_base == 2 * cfg.budget_blocks
    assert k_slots == (2 * k_base if router else k_base)
    assert res.kv_idx.shape == (1, cfg.Hq, nb, k_slots)

    kv = res.kv_idx[0].cpu().numpy()                              # [H, Qt, k_slots]
    t = np.arange(nb)
    assert (kv[:, 1:, 0] == 0).all() and (kv[:, 1:, 1] == t[None, 1:]).all()
    base = kv[:, k_base:, :k_base]
    assert (base >= 0).all() and (base <= t[None, k_base:, None]).all()
    assert (np.diff(np.sort(base, axis=-1), axis=-1) > 0).all()

    # full rows of two heads (different KV groups): the oracle's top-k and
    # sigma on the kernel's own scores
    heads = (1, cfg.Hq - 2)
    T_k = res.tile_score[0, list(heads)].cpu().numpy()[None]      # [1, 2, Qt, NB]
    vals, idx = OS.topk_order(T_k, k_slots)
    assert np.array_equal(kv[list(heads)][..., :k_base], idx[0, ..., :k_base])
    if router:
        sig = res.sigma.cpu().numpy()                             # [1, H, Qt]
        assert same_float_bits(sig[:, list(heads)], OS.sigma_margin(vals, k_base))
        eff = OS.head_mean(sig) if sel.router_grain == "row" else sig
        assert same_float_bits(eff, res.sigma_eff.cpu().numpy())
        kq = OS.quantile_rank(sel.router_quantile, eff.size)
        thr = OS.kth_smallest(eff, kq)
        assert same_float_bits(res.threshold.cpu().numpy()[0], thr)
        unc = res.uncertain[0].cpu().numpy().astype(bool)
        with np.errstate(invalid="ignore"):
            assert np.array_equal(unc, (eff <= thr)[0])
        assert unc.sum() >= kq                     # ties at the threshold all trigger
        extra = kv[:, :, k_base:]
        assert ((extra == nb).all(axis=-1) == ~unc).all()
        for j, h in enumerate(heads):
            assert np.array_equal(extra[h][unc[h]], idx[0, j][unc[h]][:, k_base:])

    # every head and tile: the kernel's ranking against a stable sort of its
    # own scores (an implementation independent of the kernel's radix select)
    T_all = res.tile_score[0]                                      # [H, Qt, NB] on the GPU
    srt_v, srt_i = torch.sort(T_all, dim=-1, descending=True, stable=True)
    kv_dev = res.kv_idx[0]
    assert torch.equal(kv_dev[..., :k_base], srt_i[..., :k_base].int())
    if router:
        unc_dev = res.uncertain[0].bool()
        assert torch.equal(kv_dev[..., k_base:][unc_dev], srt_i[..., k_base:k_slots][unc_dev].int())
        vals_all = srt_v[..., :k_base + 1].cpu().numpy()[None]   # [1, H, Qt, k_base + 1]
        assert same_float_bits(res.sigma.cpu().numpy(), OS.sigma_margin(vals_all, k_base))
    del T_all, srt_v, srt_i

    # sampled tiles: independent oracle scores, selection from scratch, attention
    rng = np.random.default_rng(cfg.index)
    tiles = sorted(set([0, 1, k_base - 1, k_base, nb // 2, nb - 1]
                       + rng.integers(0, nb, 4).tolist()))
    for h in heads:
        g = h // grp
        qh = q[:, h:h + 1].float().cpu().numpy()
        kg = k[:, g:g + 1].float().cpu().numpy()
        vg = v[:, g:g + 1].float().cpu().numpy()
        T_or = OS.tile_scores_at(qh, kg, cfg.scaling, ocfg.use_quest, tiles)
        T_kt = res.tile_score[:, h:h + 1, tiles].cpu().numpy()
        fin = np.isfinite(T_or)
        assert np.array_equal(fin, np.isfinite(T_kt))
        assert np.abs(T_or[fin] - T_kt[fin]).max() <= 1e-5
        _, idx_or = OS.topk_order(T_or, k_slots)
        kv_or = idx_or.astype(np.int32)
        kv_kt = kv[h][tiles][None, None]
        if router:
            trig = unc[h][tiles][None, None]
            kv_or[..., k_base:][~trig] = nb        # the oracle rows under the kernel's trigger
        n_diff, bad = unexplained_differences(kv_kt, kv_or, T_or, k_base, k_slots, tiles=tiles,
                                              tol=score_gap_tol(T_or, T_kt))
        print(f"  head {h}: {n_diff} of {len(tiles)} sampled tiles differ, "
              f"unexplained {len(bad)}", flush=True)
        assert not bad
        ref = OA.gathered_attention(qh, kg, vg, kv[h][None, None], cfg.scaling, tiles=tiles)
        got = out[:, h:h + 1].float().cpu().numpy()
        for tt in tiles:
            rows = slice(64 * tt, 64 * tt + 64)
            err = np.abs(got[0, 0, rows] - ref[0, 0, rows])
            assert err.max() <= 2e-2 and err.mean() <= 2e-3, (h, tt, err.max(), err.mean())
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("name", ["c3", "c4", "c5"])
def test_full_config_attention_every_tile(hip_lib, layers, name):
    """The real attention schedule of a full layer (c3: 19 generation
    launches over 28 heads; c4: 40 heads at 64K; c5: 32 launches, 16 heads,
    per-XCD tile runs) writes every output row: the buffer starts as NaN and
    must be finite everywhere after the call.  One query head of every KV
    group (a different position in each group) is compared with the fp32
    oracle over the kernel's kv_idx on every tile."""
    print(f"[case] full config {name}: attention every row / every tile", flush=True)
    cfg = synth.CONFIGS[name]
    q, k, v = layers(name)
    sel = selector_for(cfg, None)
    grp = cfg.Hq // cfg.Hkv
    res = sa.select_v2(q, k, cfg.scaling, sel=sel)
    out = torch.full_like(q, float("nan"))
    block_sparse_attn_v2(q, k, v, res.kv_idx, cfg.scaling, out=out)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all(), "rows left unwritten"
    heads = [g * grp + g % grp for g in range(cfg.Hkv)]
    ref = oracle_heads(q, k, v, res.kv_idx, cfg.scaling, heads)
    for h in heads:
        mx, mn = check_attention_rows(out[0, h].float().cpu().numpy(), ref[h], f"{name} head {h}")
        print(f"  {name} head {h}: max-abs {mx:.2e} mean-abs {mn:.2e}", flush=True)
