"""Seeded synthetic attention-layer inputs at the benchmark layer shapes.

The reference profiles real prefills of downloaded models
(``src/modal_app_profile.py:88-151``); there is no network here, so layers are
synthesised with the structure its router targets: N(0, 1) Q/K/V plus planted
"needle" KV blocks whose keys align with a Q tile's mean query (near-tied
top-k cutoffs), K-max-favouring outlier channels, and QK-Norm for the
Qwen3.6-style shape.

Draw order (one ``torch.Generator`` per (config, layer), seeded
``1000 * config_index + layer``): Q [B, Hq, S, D], K [B, Hkv, S, D],
V [B, Hkv, S, D]; then for tiles t = 2 .. Qt-1 in order and each KV head g:
``randperm(t - 1)`` picks min(n, t - 1) blocks from 1 .. t-1 and
``randn(n, 64, D)`` their noise; K of a needle block becomes
0.8 * mean(Q of the group's heads over tile t) + 0.6 * noise (later tiles
overwrite earlier ones); then the outlier channel ``randperm(D)``; then
QK-Norm; then the cast to the config dtype.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

BLOCK = 64


@dataclass(frozen=True)
class LayerConfig:
    name: str
    index: int              # position in BASELINE.json "configs"
    B: int
    Hq: int
    Hkv: int
    S: int
    D: int
    dtype: torch.dtype
    needles: int            # planted needle blocks per Q tile and KV head
    outlier_frac: float     # fraction of K channels scaled x4 (0 = none)
    qk_norm: bool
    # selector policy (SEL fields)
    mode: str
    router_score: str
    budget_blocks: int      # "top-k = N blocks" means k_base = N = 2 * budget
    router_quantile: float = 0.25
    router_mode: str = "quantile"
    router_grain: str = "row"
    layers: int = 1
    extra: dict = field(default_factory=dict)

    @property
    def scaling(self) -> float:
        return self.D ** -0.5

    def sel_fields(self) -> dict:
        return dict(mode=self.mode, budget_blocks=self.budget_blocks,
                    router_mode=self.router_mode, router_grain=self.router_grain,
                    router_quantile=self.router_quantile,
                    router_score=self.router_score)


CONFIGS = {
    # CPU plumbing run (fp32), router-on-Quest 16 -> 32
    "c1": LayerConfig("c1", 0, 1, 8, 2, 8192, 128, torch.float32, 4, 0.0, False,
                      "router", "quest", 8),
    # Qwen2.5-7B-1M layer at 32K, router-on-Quest 64 -> 128
    "c2": LayerConfig("c2", 1, 1, 28, 4, 32768, 128, torch.bfloat16, 8, 0.0, False,
                      "router", "quest", 32),
    # same shape at 128K, 28 stacked layers, 128 -> 256
    "c3": LayerConfig("c3", 2, 1, 28, 4, 131072, 128, torch.bfloat16, 8, 0.0, False,
                      "router", "quest", 64, layers=28),
    # Qwen2.5-14B at 64K, K-mean and Quest, +/- router, 96 (-> 192)
    "c4": LayerConfig("c4", 3, 1, 40, 8, 65536, 128, torch.bfloat16, 0, 0.05, False,
                      "router", "quest", 48),
    # Qwen3.6-style full-attention layer, D=256, QK-Norm, router-on-K-mean
    "c5": LayerConfig("c5", 4, 1, 16, 2, 131072, 256, torch.bfloat16, 8, 0.0, True,
                      "router", "mean", 64),
}


def rms_norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Per-head-vector RMSNorm with unit weight (QK-Norm), fp32."""
    x = x.float()
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def make_layer(cfg: LayerConfig, layer: int = 0, *, S: int | None = None,
               Hq: int | None = None, Hkv: int | None = None,
               D: int | None = None, device="cpu", dtype=None):
    """(q, k, v) for one layer of ``cfg``; shape overrides give reduced cases
    with the same structure.  Returned on ``device`` in ``dtype``
    (default: the config's dtype)."""
    S = cfg.S if S is None else S
    Hq = cfg.Hq if Hq is None else Hq
    Hkv = cfg.Hkv if Hkv is None else Hkv
    D = cfg.D if D is None else D
    dtype = cfg.dtype if dtype is None else dtype
    grp = Hq // Hkv
    g = torch.Generator(device=device).manual_seed(1000 * cfg.index + layer)
    q = torch.randn(cfg.B, Hq, S, D, generator=g, device=device)
    k = torch.randn(cfg.B, Hkv, S, D, generator=g, device=device)
    v = torch.randn(cfg.B, Hkv, S, D, generator=g, device=device)
    qt = S // BLOCK
    if cfg.needles > 0 and qt > 2:
        # mean query of each (KV group, tile): [B, Hkv, Qt, D]
        full = qt * BLOCK
        qm = q[:, :, :full].reshape(cfg.B, Hkv, grp, qt, BLOCK, D).mean(dim=(2, 4))
        for t in range(2, qt):
            n = min(cfg.needles, t - 1)
            for kh in range(Hkv):
                blocks = torch.randperm(t - 1, generator=g, device=device)[:n] + 1
                noise = torch.randn(n, BLOCK, D, generator=g, device=device)
                val = 0.8 * qm[:, kh, t][:, None, None, :] + 0.6 * noise[None]
                kb = k[:, kh, :full].view(cfg.B, qt, BLOCK, D)
                kb[:, blocks] = val
    if cfg.outlier_frac > 0:
        n_out = round(cfg.outlier_frac * D)
        ch = torch.randperm(D, generator=g, device=device)[:n_out]
        k[..., ch] *= 4.0
    if cfg.qk_norm:
        q = rms_norm(q)
        k = rms_norm(k)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def make_layer_fast(cfg: LayerConfig, layer: int = 0, *, device="cuda", dtype=None,
                    S: int | None = None):
    """Same structure as ``make_layer`` in a handful of device kernels (for
    benchmarks at full scale): each tile t still plants min(n, t-1) distinct
    needles in blocks 1 .. t-1 per KV head, the last tile to pick a block
    wins, and a planted block gets 0.8 * (its winning tile's group-mean query)
    + 0.6 * N(0, 1).  Draws differ from ``make_layer`` (a different order of
    random calls), so parity fixtures use ``make_layer``."""
    S = cfg.S if S is None else S
    dtype = cfg.dtype if dtype is None else dtype
    B, Hq, Hkv, D = cfg.B, cfg.Hq, cfg.Hkv, cfg.D
    grp = Hq // Hkv
    g = torch.Generator(device=device).manual_seed(1000 * cfg.index + layer)
    q = torch.randn(B, Hq, S, D, generator=g, device=device)
    k = torch.randn(B, Hkv, S, D, generator=g, device=device)
    v = torch.randn(B, Hkv, S, D, generator=g, device=device)
    qt = S // BLOCK
    if cfg.needles > 0 and qt > 2:
        full = qt * BLOCK
        qm = q[:, :, :full].reshape(B, Hkv, grp, qt, BLOCK, D).mean(dim=(2, 4))  # [B,Hkv,Qt,D]
        t = torch.arange(qt, device=device)
        # rank random keys among blocks 1 .. t-1 of each (tile, head); pick the n smallest
        r = torch.rand(qt, Hkv, qt, generator=g, device=device)
        blk = torch.arange(qt, device=device)
        ok = (blk[None, :] >= 1) & (blk[None, :] <= t[:, None] - 1)          # [Qt, NB]
        r = torch.where(ok[:, None, :], r, torch.full_like(r, 2.0))
        n = min(cfg.needles, qt)
        picks = r.topk(n, dim=-1, largest=False).indices                     # [Qt, Hkv, n]
        valid = torch.gather(ok[:, None, :].expand(qt, Hkv, qt), 2, picks)   # fewer than n early
        tile = t[:, None, None].expand_as(picks)
        head = torch.arange(Hkv, device=device)[None, :, None].expand_as(picks)
        win = torch.full((Hkv, qt), -1, dtype=torch.long, device=device)
        win.view(-1).scatter_reduce_(0, (head * qt + picks)[valid], tile[valid], reduce="amax")
        noise = torch.randn(B, Hkv, qt, BLOCK, D, generator=g, device=device)
        planted = win >= 0                                                    # [Hkv, NB]
        src = qm[:, torch.arange(Hkv, device=device)[:, None], win.clamp(min=0)]  # [B,Hkv,NB,D]
        val = 0.8 * src[:, :, :, None, :] + 0.6 * noise
        kb = k[:, :, :full].view(B, Hkv, qt, BLOCK, D)
        kb[:, planted] = val[:, planted]
    if cfg.outlier_frac > 0:
        n_out = round(cfg.outlier_frac * D)
        ch = torch.randperm(D, generator=g, device=device)[:n_out]
        k[..., ch] *= 4.0
    if cfg.qk_norm:
        q = rms_norm(q)
        k = rms_norm(k)
    return q.to(dtype), k.to(dtype), v.to(dtype)
