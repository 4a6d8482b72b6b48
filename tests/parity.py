"""Parity helpers shared by the GPU tests.

The kv_idx contract: identical to the reference selector given the same fp32
scores — checked bit for bit with no exception wherever both sides rank the
same score array.  Where the two sides rank independently computed fp32
scores (the kernel's MFMA sums against the oracle's or the reference's numpy /
torch sums, in another order), a differing block is explained only if its
score lies within ``tol`` of the cut: ``tol`` is the contract's tie window,
1e-6, or — when both score arrays are at hand — twice the largest score
difference measured on that row (``score_gap_tol``).  If every block's score
moves by at most e, a block can only cross the cut when it sits within 2e of
it, so that is the tightest bound that still admits every rank change the
rounding can cause.  A differing trigger decision is explained by a sigma
within ``sig_tol`` of the quantile threshold.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import selector as OS


TIE_WINDOW = 1e-6   # score ties of the kv_idx contract


def score_gap_tol(T_a, T_b, floor=TIE_WINDOW):
    """Per-row tie window for two fp32 score arrays [..., NB] of the same rows:
    max(floor, 2 * max |T_a - T_b| over the row's finite entries), flattened
    to one value per row."""
    a = np.asarray(T_a, np.float64).reshape(-1, np.shape(T_a)[-1])
    b = np.asarray(T_b, np.float64).reshape(-1, np.shape(T_b)[-1])
    fin = np.isfinite(a) & np.isfinite(b)
    with np.errstate(invalid="ignore"):
        gap = np.where(fin, np.abs(a - b), 0.0).max(axis=-1)
    return np.maximum(floor, 2.0 * gap)


def bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def f32np(x: torch.Tensor) -> np.ndarray:
    return x.detach().float().cpu().numpy()


def same_float_bits(a, b) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _cut_values(T_row, k):
    vals = np.sort(T_row)[::-1]
    lo = vals[k] if k < vals.size else -np.inf
    return vals[k - 1], lo


def unexplained_differences(kv_a, kv_b, T_ref, k_base, k_slots, trig_a=None, trig_b=None,
                            sig_a=None, sig_b=None, thr_a=None, thr_b=None,
                            tol=TIE_WINDOW, sig_tol=16 * OS.sigma_quantum(), tiles=None):
    """Rows of kv_a / kv_b whose visible sets differ without a near-tie excuse.

    T_ref: fp32 tile scores [B, H, Qt, NB] used to judge ties (the oracle's).
    tol: a scalar or one value per row (``score_gap_tol``).
    trig_*: bool [B, H, Qt] trigger decisions (router) or None.
    tiles: tile index of each Qt entry when the arrays hold a subset of tiles.
    Returns (n_rows_differing, list of unexplained row indices).
    """
    nb = T_ref.shape[-1]
    base_a, extra_a = OS.canonical_sets(kv_a, k_base, nb, tiles=tiles)
    base_b, extra_b = OS.canonical_sets(kv_b, k_base, nb, tiles=tiles)
    Tf = T_ref.reshape(-1, nb)
    tols = np.broadcast_to(np.asarray(tol, np.float64), (Tf.shape[0],))
    n_diff, bad = 0, []
    ta = None if trig_a is None else np.asarray(trig_a).reshape(-1).astype(bool)
    tb = None if trig_b is None else np.asarray(trig_b).reshape(-1).astype(bool)
    sa = None if sig_a is None else np.asarray(sig_a).reshape(-1)
    sb = None if sig_b is None else np.asarray(sig_b).reshape(-1)
    for r in range(len(base_a)):
        if base_a[r] == base_b[r] and extra_a[r] == extra_b[r]:
            continue
        n_diff += 1
        ok = True
        if base_a[r] != base_b[r]:
            hi, lo = _cut_values(Tf[r], k_base)
            for blk in base_a[r] ^ base_b[r]:
                if min(abs(Tf[r, blk] - hi), abs(Tf[r, blk] - lo)) > tols[r]:
                    ok = False
        if extra_a[r] != extra_b[r]:
            trig_differs = ta is not None and ta[r] != tb[r]
            if trig_differs:
                near = (abs(float(sa[r]) - float(thr_a)) <= sig_tol
                        or abs(float(sb[r]) - float(thr_b)) <= sig_tol)
                ok = ok and near
            else:
                ua, ub = base_a[r] | extra_a[r], base_b[r] | extra_b[r]
                hi, lo = _cut_values(Tf[r], k_slots)
                hb, lb = _cut_values(Tf[r], k_base)
                for blk in ua ^ ub:
                    d = min(abs(Tf[r, blk] - x) for x in (hi, lo, hb, lb))
                    if d > tols[r]:
                        ok = False
        if not ok:
            bad.append(r)
    return n_diff, bad


def summation_bound(q, k, scaling, quest):
    """Per (b, h, tile, block): how far two fp32 evaluations of a tile score
    may differ when they add the same exact products in different orders —
    2 n 2^-24 (n = 2 D terms: two planes) times the row's sum of |terms|,
    maxed over the tile's rows — plus, for the mean planes, what the two fp16
    terms leave of the fp32 mean (2^-23 |m_d| + 2^-39 max_d |m_d| per element,
    see ``mean_plane_bound``) and 1e-5.  fp16 x fp16 products carry 22
    significant bits, bf16 x bf16 16, so with fp16 nearly every fp32 addition
    rounds; with bf16 large scores do too."""
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    grp, nb, qt = H // Hk, (N + 63) // 64, (M + 63) // 64
    n = 2 * D
    if quest:
        kmin, kmax = OS.block_summaries(k, True)
        planes = (np.abs(kmax), np.abs(kmin))
    else:
        planes = (np.abs(OS.block_summaries(k, False)),)
    bound = np.zeros((B, H, qt, nb), np.float64)
    for b in range(B):
        for h in range(H):
            qa = q[b, h].astype(np.float64)
            if quest:
                a = np.maximum(qa, 0) @ planes[0][b, h // grp].T - np.minimum(qa, 0) @ planes[1][b, h // grp].T
                rep = 0.0
            else:
                a = np.abs(qa) @ planes[0][b, h // grp].T
                mx = planes[0][b, h // grp].max(axis=-1)                      # [nb]
                rep = 2.0 ** -23 * a + 2.0 ** -39 * np.abs(qa).sum(axis=-1)[:, None] * mx[None]
            r = 2 * n * 2.0 ** -24 * a + rep                                    # per row
            r = np.concatenate([r, np.zeros((qt * 64 - M, nb))]).reshape(qt, 64, nb).max(axis=1)
            bound[b, h] = r * abs(scaling) + 1e-5
    return bound


def decode_mean_planes(planes, B, Hk, nb, D):
    """A mean summary buffer of kernel 1 (flat, any 16-bit dtype) as float64
    numpy (hi, lo, scale): hi / lo [B, Hk, NB, D] fp16 values, scale [B, Hk,
    NB] the blocks' 2^-e."""
    flat = planes.reshape(-1)
    n = B * Hk * nb * 2 * D
    hl = flat[:n].view(torch.float16).view(B, Hk, nb, 2, D).double().cpu().numpy()
    sc = flat[n:n + 2 * B * Hk * nb].view(torch.float32).view(B, Hk, nb).double().cpu().numpy()
    return hl[..., 0, :], hl[..., 1, :], sc


def check_mean_planes(planes, k):
    """Kernel 1's mean summary of k [B, Hk, N, D] (host tensor, 16-bit values)
    against the exact block means (float64, F.pad zeros included):

    * each block's scale 2^-e is a power of two with max_d |hi_d| in [2^14,
      2^15] (hi_d = fp16 of m_d 2^e; all-zero blocks: hi = lo = 0, scale 1);
    * (hi + lo) 2^-e within 2^-23 |m_d| + 2^-25 2^-e of the kernel's fp32 mean,
      which sits within the fp32 summation bound 64 2^-24 mean_r |x| of the
      exact mean;
    * lo carries the bits hi drops: hi alone misses that bound somewhere.
    Returns the reconstructed means."""
    B, Hk, N, D = k.shape
    nb = (N + 63) // 64
    hi, lo, sc = decode_mean_planes(planes, B, Hk, nb, D)
    kp = np.zeros((B, Hk, nb * 64, D))
    kp[:, :, :N] = k.double().numpy()
    blocks = kp.reshape(B, Hk, nb, 64, D)
    exact = blocks.mean(axis=3)
    mant, _ = np.frexp(sc)
    assert (mant == 0.5).all(), "block scales are powers of two"
    hmax = np.abs(hi).max(axis=-1)
    zero = np.abs(exact).max(axis=-1) == 0
    assert ((hmax >= 2.0 ** 14) & (hmax <= 2.0 ** 15) | zero).all()
    assert (sc[zero] == 1.0).all() and (hi[zero] == 0).all() and (lo[zero] == 0).all()
    rec = (hi + lo) * sc[..., None]
    bound = (64 * 2.0 ** -24 * np.abs(blocks).mean(axis=3) + 2.0 ** -23 * np.abs(exact)
             + 2.0 ** -25 * sc[..., None] + 1e-300)
    assert (np.abs(rec - exact) <= bound).all(), np.abs(rec - exact).max()
    assert not (np.abs(hi * sc[..., None] - exact) <= bound).all(), "lo term unused"
    return rec


# Attention bar of the contract (bf16 inputs, fp32 accumulation).
ATTN_MAX_ABS, ATTN_MEAN_ABS = 2e-2, 2e-3


def oracle_heads(q, k, v, kv_idx, scale, heads, workers=None, chunk=32):
    """The fp32 oracle's output rows [M, D] of each head in ``heads`` over
    every tile of ``kv_idx`` (oracle.attention.gathered_attention on the
    bf16-rounded inputs upcast to fp32).  q [B=1, H, M, D], k / v [1, Hk, N,
    D] (device or host tensors), kv_idx [1, H, Qt, S].  Tiles are split into
    chunks of ``chunk`` run on a thread pool (numpy releases the GIL in BLAS
    and ufuncs), with BLAS held to one thread per worker."""
    import os
    import time
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    from oracle import attention as OA
    if workers is None:
        workers = max(1, min(16, len(os.sched_getaffinity(0))))
    H, Hk = q.shape[1], k.shape[1]
    grp = H // Hk
    kv = kv_idx.cpu().numpy() if torch.is_tensor(kv_idx) else np.asarray(kv_idx)
    qt = kv.shape[2]
    res = {}
    with threadpool_limits(limits=1, user_api="blas"), ThreadPoolExecutor(workers) as ex:
        for h in heads:
            t0 = time.perf_counter()
            g = h // grp
            qh = f32np(q[:, h:h + 1])
            kg = f32np(k[:, g:g + 1])
            vg = f32np(v[:, g:g + 1])
            kvh = kv[:, h:h + 1]
            out = np.zeros(qh.shape, np.float32)
            jobs = [ex.submit(OA.gathered_attention, qh, kg, vg, kvh, scale,
                              tiles=range(t0_, min(qt, t0_ + chunk)), out=out)
                    for t0_ in range(0, qt, chunk)]
            for j in jobs:
                j.result()
            res[h] = out[0, 0]
            print(f"  oracle head {h}: {qt} tiles in {time.perf_counter() - t0:.1f} s", flush=True)
    return res


def check_attention_rows(got, ref, what):
    """got / ref [M, D] (one head, every row): the contract's max-abs and
    mean-abs bar; returns (max, mean) of |got - ref|."""
    err = np.abs(np.asarray(got, np.float32) - np.asarray(ref, np.float32))
    mx, mn = float(err.max()), float(err.mean())
    assert np.isfinite(got).all(), f"{what}: non-finite output rows"
    assert mx <= ATTN_MAX_ABS and mn <= ATTN_MEAN_ABS, (what, mx, mn)
    return mx, mn
