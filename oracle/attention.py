"""numpy fp32 restatement of the reference's block-sparse attention — TEST ORACLE.

Three formulations of one semantics:

* ``gathered_attention`` — the v2 kernel, ``src/triton_block_attn.py:203-264``:
  per (b, h, Q-tile) visit the kv_idx slots in order, skip ``blk >= NB`` and
  ``blk*block_n > t*block_m + block_m - 1``, causal mask ``n > i`` and ``n >= N``,
  softmax over the visited keys (a repeated slot counts twice, as the kernel's
  loop does), output ``acc / (l > 0 ? l : 1)``.  Cost: attended blocks only.
* ``masked_tile_attention`` — ``reference_attn`` (``:301-312``, SDPA with a
  materialised keep-and-causal mask) restated per 64-row tile over keys
  ``[0, 64(t+1))``: dense causal cost.  This is the CPU-baseline leg.
* ``keep_attention`` — per-row keep mask form of ``reference_attn`` for the
  v1-style tests (``src/modal_app_qwen36_kernel_test.py:100-129``).

Pinned by: agreement of the three formulations on random inputs; case A (all
blocks kept) equal to plain causal softmax attention computed independently
(tests/test_oracle_attention.py); invariance to slot order.
"""

from __future__ import annotations

import numpy as np


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _softmax_rows(s):
    m = s.max(axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, np.float32(0))
    p = np.exp(s - m)
    l = p.sum(axis=1, keepdims=True)
    return p, l


def visited_blocks(row, t: int, n_blocks: int, block_m: int = 64, block_n: int = 64):
    """Slots the kernel processes for tile t, in slot order (triton_block_attn.py:229-234)."""
    q_last = t * block_m + block_m - 1
    return [int(b) for b in row if 0 <= b < n_blocks and b * block_n <= q_last]


def gathered_attention(q, k, v, kv_idx, scale: float, block_m: int = 64,
                       block_n: int = 64, tiles=None, heads=None, out=None):
    """[B, H, M, D] fp32 output of the v2 kernel semantics.

    ``tiles`` / ``heads`` restrict the work to a subset (rows outside stay 0,
    or keep what ``out``, a caller's fp32 [B, H, M, D] array, held).
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    kv = np.asarray(kv_idx)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    grp = H // Hk
    nb = (N + block_n - 1) // block_n
    if out is None:
        out = np.zeros((B, H, M, D), np.float32)
    assert out.shape == (B, H, M, D) and out.dtype == np.float32
    sc = np.float32(scale)
    tiles = range(kv.shape[2]) if tiles is None else tiles
    heads = range(H) if heads is None else heads
    for b in range(B):
        for h in heads:
            kh = h // grp
            for t in tiles:
                r0 = t * block_m
                if r0 >= M:
                    continue
                r1 = min(M, r0 + block_m)
                blks = np.asarray(visited_blocks(kv[b, h, t], t, nb, block_m, block_n),
                                  np.int64)
                if blks.size == 0:
                    continue
                # the keys of the visited blocks in slot order, cut at N
                keys = (blks[:, None] * block_n + np.arange(block_n)).ravel()
                keys = keys[keys < N]
                s = (q[b, h, r0:r1] @ k[b, kh, keys].T) * sc
                rows = np.arange(r0, r1)
                s[keys[None, :] > rows[:, None]] = -np.inf
                p, l = _softmax_rows(s)
                l = np.where(l > 0, l, np.float32(1))
                out[b, h, r0:r1] = (p @ v[b, kh, keys]) / l
    return out


def tile_keep(kv_idx, n_blocks: int, block_m: int = 64, block_n: int = 64):
    """bool [B, H, Qt, NB]: blocks each tile visits (set semantics)."""
    kv = np.asarray(kv_idx)
    B, H, qt, _ = kv.shape
    keep = np.zeros((B, H, qt, n_blocks), bool)
    for t in range(qt):
        lim = (t * block_m + block_m - 1) // block_n
        row = kv[:, :, t]
        ok = (row >= 0) & (row < n_blocks) & (row <= lim)
        bi, hi, si = np.nonzero(ok)
        keep[bi, hi, t, row[bi, hi, si]] = True
    return keep


def masked_tile_attention(q, k, v, kv_idx, scale: float, block_m: int = 64,
                          block_n: int = 64, tiles=None, heads=None):
    """``reference_attn`` semantics per Q-tile: dense scores over keys
    [0, min(N, (t+1)*block_m)) masked by the tile's kept blocks and causality.

    ``tiles`` / ``heads`` restrict the work to a subset (the bounded CPU
    baseline sample); rows outside the subset stay zero.
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    grp = H // Hk
    nb = (N + block_n - 1) // block_n
    keep = tile_keep(kv_idx, nb, block_m, block_n)
    qt = keep.shape[2]
    out = np.zeros((B, H, M, D), np.float32)
    sc = np.float32(scale)
    tiles = range(qt) if tiles is None else tiles
    heads = range(H) if heads is None else heads
    for b in range(B):
        for h in heads:
            kh = h // grp
            for t in tiles:
                r0 = t * block_m
                if r0 >= M:
                    continue
                r1 = min(M, r0 + block_m)
                n1 = min(N, r1)
                s = (q[b, h, r0:r1] @ k[b, kh, :n1].T) * sc
                blk_ok = np.repeat(keep[b, h, t], block_n)[:n1]
                rows = np.arange(r0, r1)
                allowed = blk_ok[None, :] & (np.arange(n1)[None, :] <= rows[:, None])
                s[~allowed] = -np.inf
                p, l = _softmax_rows(s)
                l = np.where(l > 0, l, np.float32(1))
                out[b, h, r0:r1] = (p @ v[b, kh, :n1]) / l
    return out


def keep_attention(q, k, v, keep, scale: float, block_n: int = 64):
    """``reference_attn`` with a per-row keep mask [B, H, M, NB] (:301-312)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    grp = H // Hk
    out = np.zeros((B, H, M, D), np.float32)
    sc = np.float32(scale)
    causal = np.arange(N)[None, :] <= np.arange(M)[:, None]
    for b in range(B):
        for h in range(H):
            kh = h // grp
            kk = np.repeat(keep[b, h], block_n, axis=1)[:, :N]
            s = (q[b, h] @ k[b, kh].T) * sc
            s[~(kk & causal)] = -np.inf
            p, l = _softmax_rows(s)
            out[b, h] = (p @ v[b, kh]) / l
    return out


def compute_kv_idx(keep, block_m: int):
    """``_compute_kv_idx`` (src/triton_block_attn.py:125-146): OR the keep mask
    over each tile's rows, list kept blocks ascending, pad with NB, trim to the
    largest count (at least 1)."""
    keep = np.asarray(keep, bool)
    B, H, M, nb = keep.shape
    qt = (M + block_m - 1) // block_m
    pad = qt * block_m - M
    if pad:
        keep = np.concatenate([keep, np.zeros((B, H, pad, nb), bool)], axis=2)
    anyk = keep.reshape(B, H, qt, block_m, nb).any(axis=3)
    masked = np.where(anyk, np.arange(nb, dtype=np.int32), np.int32(nb))
    srt = np.sort(masked, axis=-1)
    max_kept = max(1, int((srt < nb).sum(axis=-1).max()))
    return np.ascontiguousarray(srt[..., :max_kept]), max_kept


def causal_attention(q, k, v, scale: float):
    """Plain causal softmax attention (rows i attend keys n <= i), fp64 accumulate.

    An independent statement of the dense case used to pin case A.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    grp = H // Hk
    out = np.zeros((B, H, M, D))
    for b in range(B):
        for h in range(H):
            kh = h // grp
            for i in range(M):
                n = min(N, i + 1)
                s = (k[b, kh, :n] @ q[b, h, i]) * scale
                p = np.exp(s - s.max())
                out[b, h, i] = (p @ v[b, kh, :n]) / p.sum()
    return out.astype(np.float32)
