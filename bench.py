#!/usr/bin/env python
"""Sparse-prefill benchmark on one MI355X (BASELINE.json metric).

A step is one sparse prefill attention layer over inputs already resident in
HBM: K-block summaries -> fused select (scores, tile max, top-k, sigma) ->
router (quantile, sentinels) -> K/V operand layout -> block-sparse attention.
``value`` is ms/layer at BASELINE configs[1] (Qwen2.5-7B-1M layer, 32K,
router-on-Quest 64 -> 128); the 128K layers (configs[2], 28 of them), one
layer each of configs[3] and configs[4] (head_dim 256) and the dense
comparators are reported in the same line.  Inputs are synthetic (seeded
N(0,1) with planted needle blocks, synth.py), drawn on the GPU.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "uncertainty-gated-block-sparse-attention_amd")
sys.path.insert(0, PKG)

PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E


# Selector policies of BASELINE configs[3]: the backbone (K-mean or Quest)
# with and without the router; the budget comes from the config.
POLICIES = {
    "topk_mean": dict(mode="topk"),
    "quest": dict(mode="quest"),
    "router_mean": dict(mode="router", router_score="mean"),
    "router_quest": dict(mode="router", router_score="quest"),
}


def policy_name(sel) -> str:
    if sel.mode == "router":
        return f"router-on-{sel.router_score}"
    return "quest" if sel.mode == "quest" else f"{sel.mode} (K-mean)"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="c2")
    p.add_argument("--policy", choices=sorted(POLICIES), default=None,
                   help="override the config's selector policy (configs[3] runs both "
                        "backbones, K-mean and Quest, each with and without the router)")
    p.add_argument("--c3-layers", type=int, default=28,
                   help="stacked independent 128K layers for the configs[2] sweep (0 = skip)")
    p.add_argument("--no-c5", action="store_true",
                   help="skip the single configs[3] and configs[4] layers of the default line")
    p.add_argument("--dtype", choices=("bf16", "fp16"), default="bf16",
                   help="element format of Q/K/V (every BASELINE config is bf16)")
    p.add_argument("--no-dense", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=20.0,
                   help="target CPU work of the bounded baseline sample")
    p.add_argument("--path", choices=("v2", "v1"), default="v2",
                   help="v2: per-tile selection (the headline); v1: the per-row path "
                        "(kernel_v2=False: per-row keep mask, keep-masked attention)")
    p.add_argument("--list-overlap", action="store_true",
                   help="print how much the emitted kv_idx lists share: visited (tile, block) "
                        "slots against distinct (KV head, block) pairs over a KV group's heads "
                        "and windows of consecutive tiles (one layer, no timing)")
    p.add_argument("--pmc-run", action="store_true",
                   help="untimed driver for rocprofv3 --pmc: --steps layers of the workload, "
                        "then two copies of a 1 GiB tensor (counter calibration)")
    return p.parse_args()


class LayerRunner:
    """Preallocated buffers + the five launches of one sparse prefill layer."""

    def __init__(self, cfg, q, k, v, sel_fields=None):
        import torch
        import _capi
        import sparse_attention as sa
        self.torch, self.capi, self.lib = torch, _capi, _capi.lib()
        self.cfg = cfg
        self.q, self.k, self.v = q, k, v
        B, H, S, D = q.shape
        Hk = k.shape[1]
        self.B, self.H, self.Hk, self.S, self.D = B, H, Hk, S, D
        sel = sa.Selector()
        for f, val in (sel_fields or cfg.sel_fields()).items():
            setattr(sel, f, val)
        self.sel = sel
        self.NB = self.Qt = (S + 63) // 64
        self.k_base, self.k_slots = sa.budgets(self.NB, sel)
        quest = sel.mode == "quest" or (sel.mode == "router" and sel.router_score == "quest")
        self.mode = _capi.MODE_QUEST if quest else _capi.MODE_MEAN
        self.router = sel.mode == "router" and self.k_base < self.k_slots
        dev = q.device
        self.dt = _capi.dtype_code(q.dtype)
        self.planes = torch.empty(self.lib.ugbsa_summary_elems(B, Hk, S, D, self.mode),
                                  dtype=q.dtype, device=dev)
        self.kv_idx = torch.empty(B, H, self.Qt, self.k_slots, dtype=torch.int32, device=dev)
        self.sigma = torch.empty(B, H, self.Qt, dtype=torch.float32, device=dev)
        self.sigma_eff = torch.empty_like(self.sigma)
        self.unc = torch.empty(B, H, self.Qt, dtype=torch.uint8, device=dev)
        self.thr = torch.empty(1, dtype=torch.float32, device=dev)
        self.ws = torch.empty(self.lib.ugbsa_attn_workspace_elems(B, Hk, S, D),
                              dtype=q.dtype, device=dev)
        self.out = torch.empty_like(q)
        self.k_quant = max(1, int(float(sel.router_quantile) * B * H * self.Qt))
        self.grain = _capi.GRAIN_ROW if sel.router_grain == "row" else _capi.GRAIN_CELL
        self.rmode = _capi.ROUTER_QUANTILE if sel.router_mode == "quantile" else _capi.ROUTER_ABS
        self.names = ["summary", "select", "router", "prepare_kv", "attention"]

    def step(self, ev=None):
        """One layer; ev: list of 6 events recorded between the launches."""
        c, L, s = self.capi, self.lib, self.capi.stream_ptr(self.q.device)
        q, k, v = self.q, self.k, self.v
        B, H, Hk, S, D = self.B, self.H, self.Hk, self.S, self.D
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        c.check(L.ugbsa_block_summary(k.data_ptr(), *k.stride(), B, Hk, S, D, self.dt,
                                      self.mode, self.planes.data_ptr(), s), "summary")
        rec(1)
        c.check(L.ugbsa_select(q.data_ptr(), *q.stride(), self.planes.data_ptr(), B, H, Hk, S, S, D,
                               self.dt, self.mode, float(self.cfg.scaling), self.k_base,
                               self.k_slots, 64, self.kv_idx.data_ptr(),
                               self.sigma.data_ptr() if self.router else None, None, s), "select")
        rec(2)
        if self.router:
            c.check(L.ugbsa_router(self.sigma.data_ptr(), B, H, self.Qt, self.grain, self.rmode,
                                   float(self.sel.router_tau), self.k_quant, self.kv_idx.data_ptr(),
                                   self.k_base, self.k_slots, self.NB, self.sigma_eff.data_ptr(),
                                   self.unc.data_ptr(), self.thr.data_ptr(), s), "router")
        rec(3)
        c.check(L.ugbsa_attn_prepare_kv(k.data_ptr(), *k.stride(), v.data_ptr(), *v.stride(),
                                        B, Hk, S, D, self.dt, 64, self.ws.data_ptr(),
                                        self.ws.numel(), s),
                "prepare_kv")
        rec(4)
        self.attention(self.kv_idx)
        rec(5)

    def attention(self, kv_idx):
        c, L, s = self.capi, self.lib, self.capi.stream_ptr(self.q.device)
        q, k, o = self.q, self.k, self.out
        c.check(L.ugbsa_attn_fwd(q.data_ptr(), *q.stride(), k.data_ptr(), *k.stride(),
                                 None, 0, 0, 0, 1, kv_idx.data_ptr(), *kv_idx.stride(),
                                 self.B, self.H, self.Hk, self.S, self.S, self.D, self.dt,
                                 kv_idx.shape[2], kv_idx.shape[3], 64, float(self.cfg.scaling),
                                 o.data_ptr(), *o.stride(), self.ws.data_ptr(), self.ws.numel(), s),
                "attention")

    def attended_flops(self, kv_idx=None, exact=False) -> float:
        """Attention FLOPs over the visited (tile, block) pairs of kv_idx.
        Executed (default): 4 * 64 * 64 * D per visit, the diagonal block in
        full, as the kernel computes it.  exact: only the (row, key) pairs the
        causal mask keeps, 4 * D each — 64 * 65 / 2 = 2080 pairs on the
        diagonal block (the layer shapes are whole blocks)."""
        torch = self.torch
        kv = self.kv_idx if kv_idx is None else kv_idx
        t = torch.arange(kv.shape[2], device=kv.device).view(1, 1, -1, 1)
        ok = (kv >= 0) & (kv < self.NB) & (kv <= t)
        visits = float(ok.sum().item())
        if not exact:
            return visits * 4.0 * 64 * 64 * self.D
        diag = float((ok & (kv == t)).sum().item())
        return ((visits - diag) * 64 * 64 + diag * 64 * 65 / 2) * 4.0 * self.D

    def select_bytes(self) -> dict:
        """Algorithmic HBM bytes of kernels 1 and 2 (one launch each)."""
        B, H, Hk, S, D, NB = self.B, self.H, self.Hk, self.S, self.D, self.NB
        planes = self.lib.ugbsa_summary_elems(B, Hk, S, D, self.mode) * 2
        k1 = B * Hk * S * D * 2 + planes
        k2 = B * H * S * D * 2 + planes + B * H * self.Qt * self.k_slots * 4 + B * H * self.Qt * 4
        return {"summary": k1, "select": k2}

    def select_flops(self) -> float:
        """Scoring FLOPs over causally visible blocks, one summary contraction
        per backbone (Quest 2, mean 1), as BASELINE counts them."""
        n_sum = 2 if self.mode == self.capi.MODE_QUEST else 1
        vis = self.Qt * (self.Qt + 1) // 2
        return 2.0 * self.D * 64 * self.B * self.H * n_sum * vis


def warm_clocks(fn, torch, seconds=1.0):
    """Run fn until `seconds` of wall time have passed: MI355X clocks ramp
    over a few hundred milliseconds of sustained work, so a handful of
    warm-up steps alone under-reports steady-state speed."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()


def timed(fn, steps, warmup, torch):
    warm_clocks(fn, torch, 0.5)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, (time.perf_counter() - t0) * 1e3 / steps


def run_layer_bench(runner, steps, warmup, torch):
    """Timed region of `steps` layers; returns ms/step and per-kernel mean ms."""
    warm_clocks(runner.step, torch)
    for _ in range(warmup):
        runner.step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(6)] for _ in range(steps)]
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        runner.step(evs[i])
    end.record()
    torch.cuda.synchronize()
    total = start.elapsed_time(end) / steps
    per = {}
    for j, name in enumerate(runner.names):
        per[name] = sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps
    return total, per


def dense_sdpa_ms(q, k, v, scaling, torch, steps=3):
    """torch SDPA causal bf16 on the repeat_kv'd heads (the reference's dense path)."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    rep = q.shape[1] // k.shape[1]
    kr = k.repeat_interleave(rep, dim=1)
    vr = v.repeat_interleave(rep, dim=1)
    for backend in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel([backend]):
                fn = lambda: F.scaled_dot_product_attention(q, kr, vr, is_causal=True, scale=scaling)
                ms, _ = timed(fn, steps, 1, torch)
            return ms, backend.name
        except RuntimeError:
            continue
    return None, None


def dense_kernel3_ms(runner, torch, steps=3):
    """The build's kernel 3 on a full causal kv_idx (case A) — the MFMA dense comparator."""
    B, H, Qt = runner.B, runner.H, runner.Qt
    full = torch.arange(Qt, dtype=torch.int32, device=runner.q.device).view(1, 1, 1, Qt)
    full = full.expand(B, H, Qt, Qt).contiguous()
    ms, _ = timed(lambda: runner.attention(full), steps, 1, torch)
    flops = 4.0 * B * H * runner.D * 64 * 64 * Qt * (Qt + 1) / 2
    del full
    return ms, flops


def cpu_model() -> str:
    """The host CPU's model name, with its family / model / stepping numbers
    from /proc/cpuinfo (a virtualised host may report a generic name)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, val = (x.strip() for x in line.split(":", 1))
                info.setdefault(key, val)
            elif info:
                break                                   # first processor only
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    ids = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(ids)})" if ids else name


def cpu_baseline(cfg, q, k, v, kv_idx, budget_s):
    """The CPU oracle (numpy fp32) on the same layer: the v2 selector over
    every KV group and masked dense attention (reference_attn cost) over every
    head, timed in full when the config is BASELINE configs[0] or [1] (about
    35 s at configs[1]); longer layers stop after budget_s of attention and
    scale by the heads done."""
    from threadpoolctl import threadpool_info, threadpool_limits
    sys.path.insert(0, ROOT)
    from oracle import attention as OA
    from oracle import selector as OS
    import sparse_attention as sa

    grp = cfg.Hq // cfg.Hkv
    full = cfg.index <= 1
    sel = sa.Selector()
    for f, val in cfg.sel_fields().items():
        setattr(sel, f, val)
    ocfg = OS.SelectorConfig.from_selector(sel)
    qn = q.float().cpu().numpy()
    kn = k.float().cpu().numpy()
    vn = v.float().cpu().numpy()
    # BLAS threads: the cores of this process's affinity mask, capped by the
    # host's per-job thread setting (OMP_NUM_THREADS) where one is given
    affinity = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    n_threads = min(affinity, int(cap)) if cap.isdigit() and int(cap) > 0 else affinity
    limits = threadpool_limits(limits=n_threads, user_api="blas")
    t0 = time.perf_counter()
    if full:
        OS.select_kv_idx_v2(qn, kn, cfg.scaling, ocfg)
        sel_s = time.perf_counter() - t0
    else:
        OS.select_kv_idx_v2(qn[:, :grp], kn[:, :1], cfg.scaling, ocfg)
        sel_s = (time.perf_counter() - t0) * cfg.Hkv
    qt = kv_idx.shape[2]
    kv_np = kv_idx.cpu().numpy()
    t0 = time.perf_counter()
    heads_done = 0
    for h in range(cfg.Hq):
        kh = h // grp
        OA.masked_tile_attention(qn[:, h:h + 1], kn[:, kh:kh + 1], vn[:, kh:kh + 1],
                                 kv_np[:, h:h + 1], cfg.scaling)
        heads_done += 1
        if not full and time.perf_counter() - t0 > budget_s:
            break
    att_sample_s = time.perf_counter() - t0
    att_s = att_sample_s / heads_done * cfg.Hq
    threads = max((p.get("num_threads", 1) for p in threadpool_info()
                   if p.get("user_api") == "blas"), default=1)
    limits.restore_original_limits()
    if full:
        sample = (f"numpy fp32 oracle on the whole {cfg.name} layer: v2 selector over all "
                  f"{cfg.Hkv} KV groups ({sel_s:.1f} s) and masked dense attention "
                  f"(reference_attn cost, all {qt} tiles of all {cfg.Hq} heads, {att_s:.1f} s); "
                  f"CPU: {cpu_model()}")
    else:
        sample = (f"numpy fp32 oracle on {cfg.name}: v2 selector for 1 of {cfg.Hkv} KV groups "
                  f"({sel_s / cfg.Hkv:.1f} s, x{cfg.Hkv}); masked dense attention (reference_attn "
                  f"cost, all {qt} tiles) for {heads_done} of {cfg.Hq} heads "
                  f"({att_sample_s:.1f} s, x{cfg.Hq / heads_done:.2f}); CPU: {cpu_model()}")
    return {
        "value": round((sel_s + att_s) * 1e3, 1),
        "unit": "ms/layer",
        "cores": int(threads),
        "kind": "port",
        "sample": sample,
        "affinity_cores": affinity,
        "blas_threads": int(threads),
        "cpu_model": cpu_model(),
        "select_ms": round(sel_s * 1e3, 1),
        "attention_ms": round(att_s * 1e3, 1),
    }


def traffic_profile(cfg_name):
    """The committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of a workload
    (a config at its own policy, or "c4_<policy>" for configs[3]'s others)."""
    return os.path.join("profiles", f"attn_fwd_{cfg_name}_traffic.md")


def measured_traffic(cfg_name):
    """HBM bytes per attention launch (all launches of one layer) from the
    committed FETCH_SIZE / WRITE_SIZE summary of this workload, calibrated
    against a 1 GiB copy; None if the workload has no summary."""
    try:
        for line in open(os.path.join(ROOT, traffic_profile(cfg_name))):
            if line.startswith(f"traffic_bytes attn_fwd_pipe_kernel {cfg_name}:"):
                return float(line.split(":")[1])
    except OSError:
        pass
    return None


def policy_key(cfg, fields) -> str | None:
    """The POLICIES key of a selector field set on cfg (None if none fits)."""
    for key, pol in POLICIES.items():
        if all(fields.get(f) == v for f, v in pol.items()) and (
                pol["mode"] != "router" or fields.get("router_score", "mean") == pol["router_score"]):
            return key
    return None


def kernel12_rates(runner, per) -> dict:
    """Achieved HBM GB/s of kernels 1 (summary) and 2 (select) on their
    algorithmic bytes, with the fraction of the 8 TB/s peak, and kernel 2's
    scoring MFMA fraction."""
    b = runner.select_bytes()
    gbs = {k_: b[k_] / (per[k_] * 1e-3) / 1e9 for k_ in ("summary", "select")}
    return {"hbm_gbs": {k_: round(v_, 1) for k_, v_ in gbs.items()},
            "hbm_frac": {k_: round(v_ / PEAK_HBM_GBS, 4) for k_, v_ in gbs.items()},
            "algorithmic_bytes": b,
            "select_mfma_frac": round(runner.select_flops() / (per["select"] * 1e-3) / 1e12
                                      / PEAK_BF16_TFLOPS, 4)}


def attention_kernel_label(D, NB, elem="ElemBf16"):
    """The attn_fwd_pipe_kernel<E, D, NT, QLDS, SB, OA> instance launch_attn_fwd
    runs for 64-row tiles (csrc/attn_fwd.hip)."""
    if D == 256:
        return f"attn_fwd_pipe_kernel<{elem}, 256, 4, true, true, true>"
    return f"attn_fwd_pipe_kernel<{elem}, {D}, 4, false, false, false>"


def roofline(cfg_name, D, NB, tflops, fp16=False):
    """cfg_name: the workload whose committed traffic summary applies (None
    when the selector policy or the element format differs from the ones the
    summary was taken on: bf16)."""
    if fp16:
        cfg_name = None
    return {
        "bound": "mfma",
        "kernel": attention_kernel_label(D, NB, "ElemF16" if fp16 else "ElemBf16"),
        "achieved": round(tflops, 1),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
        "traffic": measured_traffic(cfg_name) if cfg_name else None,
        "traffic_source": (traffic_profile(cfg_name) + " (rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                           "calibrated by a 1 GiB copy)"
                           if cfg_name and measured_traffic(cfg_name) is not None else None),
    }



def traffic_name(cfg, fields):
    """The traffic summary that applies to cfg under the selector fields:
    the config's own ("c4") at its default policy, "c4_<policy>" otherwise."""
    if fields == cfg.sel_fields():
        return cfg.name
    key = policy_key(cfg, fields)
    return f"{cfg.name}_{key}" if key else None


def in_dtype(args, torch):
    """torch dtype of the synthetic Q/K/V (--dtype)."""
    return torch.float16 if args.dtype == "fp16" else torch.bfloat16


def single_layer_block(cfg, args, torch, synth, dev, policy=None, layer=None, dense=True):
    """One layer of cfg at its default policy (or POLICIES[policy]): ms/layer,
    per-kernel ms, attended TFLOP/s, roofline, kernel 1-2 HBM rates and (with
    dense) the dense ratio.  layer: (q, k, v) already drawn for cfg."""
    fields = cfg.sel_fields()
    if policy is not None:
        fields.update(POLICIES[policy])
    if layer is None:
        layer = synth.make_layer_fast(cfg, 0, device=dev, dtype=in_dtype(args, torch))
    r = LayerRunner(cfg, *layer, sel_fields=fields)
    torch.cuda.synchronize()
    ms, per = run_layer_bench(r, max(3, args.steps // 2), 1, torch)
    fl = r.attended_flops()
    ex = r.attended_flops(exact=True)
    tf = fl / (per["attention"] * 1e-3) / 1e12
    out = {"ms_per_layer": round(ms, 3),
           "kernels_ms": {k_: round(v_, 3) for k_, v_ in per.items()},
           "attended_tflop": round(fl / 1e12, 3), "attended_tflops": round(tf, 1),
           "causal_exact_tflop": round(ex / 1e12, 3),
           "causal_exact_tflops": round(ex / (per["attention"] * 1e-3) / 1e12, 1),
           "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4),
           "roofline": roofline(traffic_name(cfg, fields), cfg.D, r.NB, tf,
                                args.dtype == "fp16"),
           **kernel12_rates(r, per)}
    out["policy"] = policy_name(r.sel)
    if r.router:
        out["trigger_rate"] = round(float(r.unc.float().mean().item()), 4)
    if dense and not args.no_dense:
        sd, _ = dense_sdpa_ms(r.q, r.k, r.v, cfg.scaling, torch, steps=2)
        k3, k3f = dense_kernel3_ms(r, torch, steps=2)
        best = min(x for x in (sd, k3) if x is not None)
        out.update({"dense_sdpa_ms": None if sd is None else round(sd, 2),
                    "dense_kernel3_ms": round(k3, 2),
                    "dense_kernel3_tflops": round(k3f / (k3 * 1e-3) / 1e12, 1),
                    "ratio_sparse_vs_dense": round(ms / best, 4)})
    del r
    return out


def pmc_run(cfg, steps, torch, synth, dev, dtype, policy=None):
    q, k, v = synth.make_layer_fast(cfg, 0, device=dev, dtype=dtype)
    fields = cfg.sel_fields()
    if policy is not None:
        fields.update(POLICIES[policy])
    runner = LayerRunner(cfg, q, k, v, sel_fields=fields)
    for _ in range(steps):
        runner.step()
    torch.cuda.synchronize()
    src = torch.empty(1 << 29, dtype=torch.int16, device=dev).fill_(1)   # 1 GiB
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc run done", flush=True)


def list_overlap(runner, torch):
    """Visited slots of the layer's kv_idx (block < NB and <= t) against the
    number of distinct (b, KV head, window, block) tuples over the KV group's
    query heads and windows of w consecutive tiles: how many of the visits a
    cache that kept every block for one window would serve."""
    runner.step()
    torch.cuda.synchronize()
    kv = runner.kv_idx.long()
    B, H, Qt, _ = kv.shape
    NB, Hk = runner.NB, runner.Hk
    grp = H // Hk
    t = torch.arange(Qt, device=kv.device).view(1, 1, Qt, 1)
    ok = (kv >= 0) & (kv < NB) & (kv <= t)
    res = {"visits": int(ok.sum())}
    for w in (1, 2, 4, 8, 16):
        seen = torch.zeros(B * Hk * ((Qt + w - 1) // w) * NB, dtype=torch.bool, device=kv.device)
        win = (torch.arange(Qt, device=kv.device) // w).view(1, Qt, 1)
        nwin = (Qt + w - 1) // w
        for h in range(H):
            g = h // grp
            bidx = torch.arange(B, device=kv.device).view(B, 1, 1)
            key = ((bidx * Hk + g) * nwin + win) * NB + kv[:, h].clamp(0, NB - 1)
            seen[key[ok[:, h]]] = True
        res[f"union_w{w}"] = int(seen.sum())
        res[f"visits_per_union_w{w}"] = round(res["visits"] / max(1, res[f"union_w{w}"]), 2)
    return res


def run_v1(args, cfg, q, k, v, torch):
    """The v1 per-row path on one layer (SEL.kernel_v2 = False,
    src/sparse_attention.py:790-804): per-row selection + router
    (select_mask_v1), keep -> kv_idx + row masks, keep-masked attention.
    The compaction syncs once for MAX_KEPT, as the reference does."""
    import sparse_attention as sa
    from block_attn import attn_workspace, block_sparse_attn, keep_kv_idx
    sel = sa.Selector()
    for f, val in cfg.sel_fields().items():
        setattr(sel, f, val)
    B, H, S, D = q.shape
    ws = attn_workspace(B, k.shape[1], S, D, q.device)
    out = torch.empty_like(q)
    state = {}

    def step(ev=None):
        rec = (lambda i: ev[i].record()) if ev is not None else (lambda i: None)
        rec(0)
        res = sa.select_mask_v1(q, k, cfg.scaling, sel=sel)
        rec(1)
        block_sparse_attn(q, k, v, res.keep, cfg.scaling, out=out, workspace=ws)
        rec(2)
        state["res"] = res

    warm_clocks(step, torch)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    sel_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    attn_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    res = state["res"]
    kv, _, max_kept = keep_kv_idx(res.keep, 64, want_rowmask=False)
    t = torch.arange(kv.shape[2], device=kv.device).view(1, 1, -1, 1)
    visited = ((kv[..., :max_kept] < kv.shape[-1]) & (kv[..., :max_kept] <= t)).sum().item()
    flops = float(visited) * 4.0 * 64 * 64 * D
    return {
        "metric": "v1 per-row sparse prefill ms/layer (kernel_v2=False); executed TFLOP/s",
        "value": round(sel_ms + attn_ms, 4), "unit": "ms/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(sel_ms + attn_ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": args.dtype,
        "data": "synthetic (seeded N(0,1) Q/K/V with planted needle blocks, synth.make_layer_fast on the GPU)",
        "config": {"workload": f"{cfg.name} shape, v1 {cfg.mode}-on-{cfg.router_score} "
                               f"budget {cfg.budget_blocks} per row, q={cfg.router_quantile} "
                               f"{cfg.router_grain}-grain", "seq_len": cfg.S, "global_batch": cfg.B},
        "kernels_ms": {"select_rows_and_router": round(sel_ms, 4),
                       "compaction_and_attention": round(attn_ms, 4)},
        "max_kept": int(max_kept),
        "mean_kept_per_row": round(float(res.keep.float().sum(-1).mean().item()), 2),
        "trigger_rate": (round(float(res.uncertain.float().mean().item()), 4)
                         if res.uncertain is not None else None),
        "executed_tflop": round(flops / 1e12, 4),
        "executed_tflops": round(flops / (attn_ms * 1e-3) / 1e12, 1),
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported in this build "
              "(the hot path would shard by KV-head group; only the one-GPU share is built "
              "and measured)", file=sys.stderr)
        sys.exit(2)
    import torch
    import synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = synth.CONFIGS[args.config]
    if args.pmc_run:
        pmc_run(cfg, args.steps, torch, synth, dev, in_dtype(args, torch), args.policy)
        return
    t_gen = time.perf_counter()
    q, k, v = synth.make_layer_fast(cfg, 0, device=dev, dtype=in_dtype(args, torch))
    gen_s = time.perf_counter() - t_gen
    if args.path == "v1":
        print(json.dumps(run_v1(args, cfg, q, k, v, torch)), flush=True)
        return
    fields = cfg.sel_fields()
    if args.policy is not None:
        fields.update(POLICIES[args.policy])
    runner = LayerRunner(cfg, q, k, v, sel_fields=fields)
    if args.list_overlap:
        print(json.dumps({"config": cfg.name, "policy": policy_name(runner.sel),
                          **list_overlap(runner, torch)}), flush=True)
        return
    ms_step, per = run_layer_bench(runner, args.steps, args.warmup, torch)
    attn_flops = runner.attended_flops()
    exact_flops = runner.attended_flops(exact=True)
    attn_tflops = attn_flops / (per["attention"] * 1e-3) / 1e12
    select_ms = per["summary"] + per["select"] + per["router"]
    res = {
        "metric": "sparse prefill ms/layer at 32K/128K vs dense; attended TFLOP/s; % MFMA peak",
        "value": round(ms_step, 4),
        "unit": "ms/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded N(0,1) Q/K/V with planted needle blocks, synth.make_layer_fast on the GPU)",
        "config": {"workload": f"{cfg.name}: BASELINE configs[{cfg.index}] — one causal prefill "
                               f"attention layer, B={cfg.B} Hq={cfg.Hq} Hkv={cfg.Hkv} S={cfg.S} "
                               f"D={cfg.D}, {policy_name(runner.sel)} "
                               f"k_base={runner.k_base} k_slots={runner.k_slots} "
                               f"q={cfg.router_quantile} {cfg.router_grain}-grain",
                   "seq_len": cfg.S, "global_batch": cfg.B},
        "kernels_ms": {k_: round(v_, 4) for k_, v_ in per.items()},
        "select_ms": round(select_ms, 4),
        "attended_tflop": round(attn_flops / 1e12, 4),
        "attended_tflops": round(attn_tflops, 1),
        "causal_exact_tflop": round(exact_flops / 1e12, 4),
        "causal_exact_tflops": round(exact_flops / (per["attention"] * 1e-3) / 1e12, 1),
        "trigger_rate": round(float(runner.unc.float().mean().item()), 4) if runner.router else None,
        **kernel12_rates(runner, per),
        "roofline": roofline(traffic_name(cfg, fields), cfg.D,
                             runner.NB, attn_tflops, args.dtype == "fp16"),
        "gen_s": round(gen_s, 1),
    }
    if not args.no_dense:
        sd_ms, backend = dense_sdpa_ms(q, k, v, cfg.scaling, torch)
        k3_ms, k3_flops = dense_kernel3_ms(runner, torch)
        dense_best = min(x for x in (sd_ms, k3_ms) if x is not None)
        res["dense"] = {"sdpa_ms": None if sd_ms is None else round(sd_ms, 3), "sdpa_backend": backend,
                        "kernel3_full_ms": round(k3_ms, 3),
                        "kernel3_full_tflops": round(k3_flops / (k3_ms * 1e-3) / 1e12, 1),
                        "ratio_sparse_vs_dense": round(ms_step / dense_best, 4)}
    kv_for_cpu = runner.kv_idx.clone()
    del runner
    if args.c3_layers > 0 and args.config != "c3":
        c3 = synth.CONFIGS["c3"]
        layers = []
        for layer in range(args.c3_layers):
            lq, lk, lv = synth.make_layer_fast(c3, layer, device=dev, dtype=in_dtype(args, torch))
            layers.append(LayerRunner(c3, lq, lk, lv))
        torch.cuda.synchronize()
        sweep_steps = max(1, min(args.steps, 3))

        def sweep():
            for r in layers:
                r.step()
        ms_sweep, _ = timed(sweep, sweep_steps, 1, torch)
        r0 = layers[0]
        ms1, per3 = run_layer_bench(r0, max(3, args.steps // 2), 1, torch)
        fl3 = r0.attended_flops()
        ex3 = r0.attended_flops(exact=True)
        tf3 = fl3 / (per3["attention"] * 1e-3) / 1e12
        c3res = {"layers": args.c3_layers, "ms_per_layer": round(ms_sweep / args.c3_layers, 3),
                 "single_layer_ms": round(ms1, 3),
                 "kernels_ms": {k_: round(v_, 3) for k_, v_ in per3.items()},
                 "attended_tflop": round(fl3 / 1e12, 3), "attended_tflops": round(tf3, 1),
                 "causal_exact_tflop": round(ex3 / 1e12, 3),
                 "causal_exact_tflops": round(ex3 / (per3["attention"] * 1e-3) / 1e12, 1),
                 "mfma_frac": round(tf3 / PEAK_BF16_TFLOPS, 4),
                 "roofline": roofline("c3", c3.D, r0.NB, tf3, args.dtype == "fp16"),
                 **kernel12_rates(r0, per3)}
        if not args.no_dense:
            sd3, _ = dense_sdpa_ms(r0.q, r0.k, r0.v, c3.scaling, torch, steps=2)
            k33, k3f = dense_kernel3_ms(r0, torch, steps=2)
            best = min(x for x in (sd3, k33) if x is not None)
            c3res.update({"dense_sdpa_ms": None if sd3 is None else round(sd3, 2),
                          "dense_kernel3_ms": round(k33, 2),
                          "dense_kernel3_tflops": round(k3f / (k33 * 1e-3) / 1e12, 1),
                          "ratio_sparse_vs_dense": round((ms_sweep / args.c3_layers) / best, 4)})
        res["c3"] = c3res
        del layers
    if not args.no_c5 and args.c3_layers > 0:
        # one layer each of configs[3] (its default policy) and configs[4]
        # (head_dim 256, QK-Norm) beside the c3 sweep
        for name in ("c4", "c5"):
            if name != args.config:
                res[name] = single_layer_block(synth.CONFIGS[name], args, torch, synth, dev)
        if args.config != "c4":
            # configs[3] runs both backbones, each with and without the router:
            # the three policies besides its default, on the same layer
            c4 = synth.CONFIGS["c4"]
            layer = synth.make_layer_fast(c4, 0, device=dev, dtype=in_dtype(args, torch))
            default = policy_key(c4, c4.sel_fields())
            res["c4_policies"] = {
                key: single_layer_block(c4, args, torch, synth, dev, policy=key, layer=layer,
                                        dense=False)
                for key in POLICIES if key != default}
            del layer
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(cfg, q, k, v, kv_for_cpu, args.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
