"""numpy fp32 restatement of the reference's v2 tile selector — TEST ORACLE.

Reference: ``src/sparse_attention.py:588-748`` (``_block_select_kv_idx_v2``),
with the policy knobs of ``:54-97`` (``Selector``).  Everything here runs in
IEEE fp32 on the CPU, on bf16-rounded inputs upcast to fp32; the GPU kernels
are held to these results (see the parity contract in the tests).

Deliberate definitions where the reference leaves the result unspecified:

* ``torch.topk`` does not specify the order of equal scores.  This oracle (and
  the HIP kernel) use the total order *score descending, block index
  ascending*, with NaN ranked above every number (torch's ``topk`` ordering of
  NaN).  Blocks that are invisible to a tile score ``-inf`` and therefore land
  in trailing slots in ascending block order, where the reference emits
  "arbitrary invisible ids" (``:697``); the attention skips them either way.
* ``mean(dim=1)`` for the row-grain sigma is restated as a sequential fp32 sum
  over heads followed by one IEEE division by H — ATen's CPU ``mean`` is
  ``sum(...).div_(n)``.  sigma values are integer multiples of 2**-149, so the
  sum is exact (order-independent) while it stays below 2**-125.

How each function is pinned (tests/test_oracle_selector.py):

* ``block_summaries``   brute force per block on tiny inputs; zero padding of
                        the last block counted as in ``F.pad`` (``:618-622``).
* ``tile_scores``       Quest identity sum_d max(q_d*Kmax_d, q_d*Kmin_d) and the
                        upper bound score >= max_{k in blk} q.k*scaling; tile
                        max / visibility / forcing by brute force.
* ``topk_order``        against a Python ``sorted`` with the explicit key.
* ``sigma_margin``      bit-exact against ``fractions.Fraction`` rounding on the
                        FMAX quirk (sigma = round((a-c)/FMAX) to the 2**-149
                        quantum) and the NaN rows (tile t <= k_base-1).
* ``kth_smallest``      against ``sorted`` with NaN last, with H-fold
                        replication for row grain.
* end to end            against the committed golden vectors written from the
                        reference selector itself (tests/golden/).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

BLOCK = 64                      # src/sparse_attention.py:51
FMAX = np.float32(np.finfo(np.float32).max)
SPREAD_MIN = np.float32(1e-6)   # clamp(min=1e-6), src/sparse_attention.py:706


@dataclass
class SelectorConfig:
    """The ``Selector`` fields the v2 path reads (src/sparse_attention.py:58-97)."""
    mode: str = "dense"
    budget_blocks: int = 32
    k_min: int = 8
    k_max: int = 112
    router_mode: str = "abs"
    router_grain: str = "cell"
    router_tau: float = 0.10
    router_quantile: float = 0.20
    router_score: str = "mean"

    @classmethod
    def from_selector(cls, sel) -> "SelectorConfig":
        return cls(**{f: getattr(sel, f) for f in cls.__dataclass_fields__})

    @property
    def use_quest(self) -> bool:
        # src/sparse_attention.py:627-628
        return self.mode == "quest" or (self.mode == "router"
                                        and self.router_score == "quest")


def budgets(cfg: SelectorConfig, n_blocks: int):
    """(k_base, k_slots) — src/sparse_attention.py:688-695."""
    k_row = int(max(min(cfg.k_max, cfg.budget_blocks), cfg.k_min))
    k_base = min(2 * k_row, n_blocks)
    k_slots = min(2 * k_base, n_blocks) if cfg.mode == "router" else k_base
    return k_base, k_slots


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def block_summaries(k, use_quest: bool, block_n: int = BLOCK):
    """Per-block K summaries on the zero-padded key axis.

    src/sparse_attention.py:618-622 (pad + view), :636-637 (amin/amax), :646
    (mean, pad zeros included, divided by ``block_n``).
    k: [B, Hk, N, D] -> quest: (kmin, kmax), else kmean; each [B, Hk, NB, D].
    """
    k = _f32(k)
    B, Hk, N, D = k.shape
    nb = (N + block_n - 1) // block_n
    kp = np.zeros((B, Hk, nb * block_n, D), np.float32)
    kp[:, :, :N] = k
    blocks = kp.reshape(B, Hk, nb, block_n, D)
    if use_quest:
        return blocks.min(axis=3), blocks.max(axis=3)
    return blocks.mean(axis=3, dtype=np.float32)


def tile_visibility(q_tiles: int, n_keys: int, n_blocks: int,
                    block_m: int = 64, block_n: int = BLOCK):
    """Bool [Qt, NB] and self block per tile — src/sparse_attention.py:660-666, 675-681."""
    q_tile_last = np.minimum(np.arange(q_tiles) * block_m + block_m - 1, n_keys - 1)
    blk_start = np.arange(n_blocks) * block_n
    visible = blk_start[None, :] <= q_tile_last[:, None]
    self_blk = q_tile_last // block_n
    return visible, self_blk


def tile_scores(q, k, scaling: float, use_quest: bool, block_m: int = 64,
                block_n: int = BLOCK, row_chunk: int = 8192, force: bool = True):
    """tile_score [B, H, Qt, NB] fp32 exactly as handed to ``topk``.

    Steps of src/sparse_attention.py: Q zero-pad (:623-625), per-row score
    (:638-648), tile max over rows (:655-656), -inf outside tile visibility
    (:660-666), FMAX on the sink and the tile's self block (:675-681).
    ``force=False`` stops before the forcing: the scores the score-dump
    diagnostic ranks (src/dump_block_scores.py:137-147).
    ``k`` may hold H heads (repeat_kv'd, as the reference passes) or Hk heads
    with H % Hk == 0 (query head h reads key head h // (H // Hk), the mapping
    of transformers' ``repeat_kv``).
    """
    q = _f32(q)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    assert H % Hk == 0, "query heads must be a multiple of key heads"
    grp = H // Hk
    nb = (N + block_n - 1) // block_n
    qt = (M + block_m - 1) // block_m
    mp = qt * block_m
    summ = block_summaries(k, use_quest, block_n)
    sc = np.float32(scaling)
    rc = max(block_m, (row_chunk // block_m) * block_m)
    T = np.empty((B, H, qt, nb), np.float32)
    for b in range(B):
        for h in range(H):
            kh = h // grp
            qp = np.zeros((mp, D), np.float32)
            qp[:M] = q[b, h]
            for r0 in range(0, mp, rc):
                rows = qp[r0:r0 + rc]
                if use_quest:
                    kmin, kmax = summ[0][b, kh], summ[1][b, kh]
                    s = (np.maximum(rows, np.float32(0)) @ kmax.T
                         + np.minimum(rows, np.float32(0)) @ kmin.T) * sc
                else:
                    s = (rows @ summ[b, kh].T) * sc
                T[b, h, r0 // block_m:(r0 + rows.shape[0]) // block_m] = (
                    s.reshape(-1, block_m, nb).max(axis=1))
    visible, self_blk = tile_visibility(qt, N, nb, block_m, block_n)
    T[:, :, ~visible] = -np.inf
    if force:
        T[..., 0] = FMAX
        T[:, :, np.arange(qt), self_blk] = FMAX
    return T


def tile_scores_at(q, k, scaling: float, use_quest: bool, tiles, block_m: int = 64,
                   block_n: int = BLOCK, force: bool = True):
    """tile_score rows [B, H, len(tiles), NB] of the given Q tiles only.

    The same steps as ``tile_scores`` (:623-681) restricted to a subset of
    tiles, for spot checks at sizes where the full [B, H, Qt, NB] tensor is
    too large for the CPU.
    """
    q = _f32(q)
    B, H, M, D = q.shape
    N = k.shape[2]
    nb = (N + block_n - 1) // block_n
    tiles = [int(t) for t in tiles]
    out = np.empty((B, H, len(tiles), nb), np.float32)
    summ = block_summaries(k, use_quest, block_n)
    for j, t in enumerate(tiles):
        r0 = t * block_m
        rows = np.arange(r0, min(M, r0 + block_m))
        s = row_scores(q, k, scaling, use_quest, rows, block_n, summ=summ)
        if rows.size < block_m:          # zero-padded query rows score 0 (:623-625)
            s = np.concatenate([s, np.zeros(s.shape[:2] + (block_m - rows.size, nb),
                                            np.float32)], axis=2)
        T = s.max(axis=2)
        last = min(r0 + block_m - 1, N - 1)
        T[..., np.arange(nb) * block_n > last] = -np.inf
        if force:
            T[..., 0] = FMAX
            T[..., last // block_n] = FMAX
        out[:, :, j] = T
    return out


def row_scores(q, k, scaling: float, use_quest: bool, rows, block_n: int = BLOCK,
               summ=None):
    """Per-row block scores S [B, H, len(rows), NB] fp32 of the given query rows.

    The score of src/sparse_attention.py:638-648 (no tile max, no mask), as
    the score dump reads it for its noise estimate (src/dump_block_scores.py:
    126-135, 181-187).  ``summ``: ``block_summaries(k, use_quest)`` if
    already computed.
    """
    q = _f32(q)
    B, H, M, D = q.shape
    Hk = k.shape[1]
    grp = H // Hk
    if summ is None:
        summ = block_summaries(k, use_quest, block_n)
    sc = np.float32(scaling)
    rows = np.asarray(rows, dtype=np.int64)
    nb = (summ[0] if use_quest else summ).shape[2]
    S = np.empty((B, H, rows.size, nb), np.float32)
    for b in range(B):
        for h in range(H):
            x = q[b, h, rows]
            if use_quest:
                kmin, kmax = summ[0][b, h // grp], summ[1][b, h // grp]
                S[b, h] = (np.maximum(x, np.float32(0)) @ kmax.T
                           + np.minimum(x, np.float32(0)) @ kmin.T) * sc
            else:
                S[b, h] = (x @ summ[b, h // grp].T) * sc
    return S


def sortable_key(x) -> np.ndarray:
    """uint32 key, monotone in the float value; NaN maps to the largest key."""
    x = _f32(x)
    u = x.view(np.uint32)
    key = np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000))
    return np.where(np.isnan(x), np.uint32(0xFFFFFFFF), key).astype(np.uint32)


def topk_order(T, k: int):
    """(vals, idx) of the k best blocks per row, ordered score desc, index asc.

    Stand-in for ``tile_score.topk(k, dim=-1)`` (src/sparse_attention.py:697)
    with the tie order made total.
    """
    T = _f32(T)
    nb = T.shape[-1]
    inv = (np.uint64(0xFFFFFFFF) - sortable_key(T).astype(np.uint64))
    comp = (inv << np.uint64(32)) | np.arange(nb, dtype=np.uint64)
    if k < nb:   # composite keys are unique: partition then sort the k best
        part = np.argpartition(comp, k - 1, axis=-1)[..., :k]
        sub = np.take_along_axis(comp, part, axis=-1)
        idx = np.take_along_axis(part, np.argsort(sub, axis=-1), axis=-1)
    else:
        idx = np.argsort(comp, axis=-1)[..., :k]
    vals = np.take_along_axis(T, idx, axis=-1)
    return vals, idx


def sigma_margin(vals, k_base: int):
    """Normalised cutoff margin per (b, h, t), fp32 — src/sparse_attention.py:703-707.

    s_top is the forced sink (FMAX), so sigma = fl((a - c) / FMAX), a value on
    the 2**-149 subnormal grid; NaN where c = -inf (fewer than k_base+1
    visible blocks).
    """
    vals = _f32(vals)
    s_top = vals[..., 0]
    a = vals[..., k_base - 1]
    c = vals[..., k_base]
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        spread = np.maximum(s_top - c, SPREAD_MIN)      # NaN propagates, as clamp
        return ((a - c) / spread).astype(np.float32)


def head_mean(sigma):
    """Row grain: mean over heads, broadcast back — src/sparse_attention.py:708-710."""
    sigma = _f32(sigma)
    acc = sigma[:, 0].copy()
    for h in range(1, sigma.shape[1]):
        acc = (acc + sigma[:, h]).astype(np.float32)
    with np.errstate(invalid="ignore"):
        mean = (acc / np.float32(sigma.shape[1])).astype(np.float32)
    return np.broadcast_to(mean[:, None, :], sigma.shape).copy()


def kth_smallest(flat, kq: int) -> np.float32:
    """``flat.kthvalue(kq)`` with NaN ranked above every number (:715)."""
    s = np.sort(_f32(flat).ravel())           # numpy sorts NaN last
    return np.float32(s[kq - 1])


def quantile_rank(q_frac: float, numel: int) -> int:
    """k_quant = max(1, int(q * numel)) in Python float (:714)."""
    return max(1, int(float(q_frac) * numel))


@dataclass
class Selection:
    kv_idx: np.ndarray           # int32 [B, H, Qt, k_slots]
    k_base: int
    k_slots: int
    tile_score: np.ndarray       # fp32 [B, H, Qt, NB] (topk input)
    sigma: np.ndarray | None     # fp32 [B, H, Qt] per-cell margin (router only)
    sigma_eff: np.ndarray | None  # after row-grain mean (router only)
    threshold: np.float32 | None  # quantile threshold (router quantile only)
    uncertain: np.ndarray | None  # bool [B, H, Qt] (router only)


def select_from_tile_scores(T, cfg: SelectorConfig) -> Selection:
    """Top-k, sigma, router and sentinel emission on a given fp32 tile_score.

    src/sparse_attention.py:688-725, 748.  This is the function the HIP
    selector must reproduce bit-for-bit when fed the same ``T``.
    """
    T = _f32(T)
    nb = T.shape[-1]
    k_base, k_slots = budgets(cfg, nb)
    vals, idx = topk_order(T, k_slots)
    kv = idx.astype(np.int32)
    sigma = sigma_eff = thr = unc = None
    if cfg.mode == "router" and k_base < k_slots:
        sigma = sigma_margin(vals, k_base)
        sigma_eff = head_mean(sigma) if cfg.router_grain == "row" else sigma.copy()
        with np.errstate(invalid="ignore"):
            if cfg.router_mode == "quantile":
                kq = quantile_rank(cfg.router_quantile, sigma_eff.size)
                thr = kth_smallest(sigma_eff, kq)
                unc = sigma_eff <= thr
            else:
                unc = sigma_eff < np.float32(cfg.router_tau)
        extra = kv[..., k_base:]
        extra[~unc] = nb
    return Selection(np.ascontiguousarray(kv), k_base, k_slots, T, sigma,
                     sigma_eff, thr, unc)


def select_kv_idx_v2(q, k, scaling: float, cfg: SelectorConfig,
                     block_m: int = 64) -> Selection:
    """End-to-end v2 selection (src/sparse_attention.py:588-748) in fp32."""
    T = tile_scores(q, k, scaling, cfg.use_quest, block_m)
    return select_from_tile_scores(T, cfg)


def canonical_sets(kv_idx, k_base: int, n_blocks: int, block_m: int = 64,
                   block_n: int = BLOCK, tiles=None):
    """Per (b, h, t): (base set, extra set) of visible blocks.

    The comparison sets of the parity contract: slots j < k_base and j >= k_base,
    keeping only real blocks the attention would visit (< NB and visible).
    ``tiles`` gives the tile index of each entry of the Qt axis when kv_idx
    holds a subset of tiles (default: entry t is tile t).
    Returns two lists (flattened over b, h, t) of frozensets.
    """
    kv = np.asarray(kv_idx)
    B, H, qt, _ = kv.shape
    tix = list(range(qt)) if tiles is None else [int(t) for t in tiles]
    base, extra = [], []
    for b in range(B):
        for h in range(H):
            for j in range(qt):
                t = tix[j]
                lim = (t * block_m + block_m - 1) // block_n
                row = kv[b, h, j]
                ok = (row >= 0) & (row < n_blocks) & (row <= lim)
                base.append(frozenset(row[:k_base][ok[:k_base]].tolist()))
                extra.append(frozenset(row[k_base:][ok[k_base:]].tolist()))
    return base, extra


def sigma_quantum() -> float:
    """Spacing of sigma values: the fp32 subnormal step 2**-149."""
    return math.ldexp(1.0, -149)
