"""Parity helpers shared by the GPU tests.

The kv_idx contract (north star): identical to the reference selector given the
same fp32 scores; across independently computed fp32 scores (kernel vs oracle),
a difference is allowed only where it is explained by a near tie — a differing
block whose score is within ``tol`` of the cutoff, or a differing trigger
decision whose sigma is within ``sig_tol`` of the quantile threshold.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import selector as OS


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
                            tol=2e-6, sig_tol=16 * OS.sigma_quantum(), tiles=None):
    """Rows of kv_a / kv_b whose visible sets differ without a near-tie excuse.

    T_ref: fp32 tile scores [B, H, Qt, NB] used to judge ties (the oracle's).
    trig_*: bool [B, H, Qt] trigger decisions (router) or None.
    tiles: tile index of each Qt entry when the arrays hold a subset of tiles.
    Returns (n_rows_differing, list of unexplained row indices).
    """
    nb = T_ref.shape[-1]
    base_a, extra_a = OS.canonical_sets(kv_a, k_base, nb, tiles=tiles)
    base_b, extra_b = OS.canonical_sets(kv_b, k_base, nb, tiles=tiles)
    Tf = T_ref.reshape(-1, nb)
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
                if min(abs(Tf[r, blk] - hi), abs(Tf[r, blk] - lo)) > tol:
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
                    if d > tol:
                        ok = False
        if not ok:
            bad.append(r)
    return n_diff, bad
