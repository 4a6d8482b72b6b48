"""Block-sparse attention launchers — the MI355X counterpart of the reference's
``src/triton_block_attn.py`` (same function names, arguments and asserts).

``block_sparse_attn_v2`` (reference ``:267-298``, per-tile ``kv_idx``) and
``block_sparse_attn`` (``:149-182``, per-row ``keep`` mask) launch the gfx950
HIP attention kernels through the C ABI; ``_compute_kv_idx`` (``:125-146``)
runs as the HIP kernel ``keep_kv_idx_kernel`` on device tensors (and in torch
for host tensors, as the reference's kernel test builds ``kv_idx``);
``reference_attn`` (``:301-312``) forms the SDPA reference in the inputs'
dtype (``reference_attn_fp32`` keeps it in fp32 for tests).  Differences from
the reference launchers, all additive:

* K/V may carry ``Hk`` heads with ``H % Hk == 0`` (GQA: query head h reads KV
  head h // (H // Hk), transformers' ``repeat_kv`` mapping), so callers need
  not materialise ``repeat_kv``; equal head counts behave as in the reference.
* Q/K/V only need unit stride on head_dim (the reference's dispatcher calls
  ``.contiguous()``); ``out`` may be any such strided view, which lets the
  dispatcher write the ``[B, S, H, D]`` layout directly.
* ``num_warps`` / ``num_stages`` are Triton tuning knobs, accepted and ignored.
* Both launchers assert query length == key length before anything else
  (the reference asserts ``q.shape == k.shape``): the causal mask takes query
  row i as key position i.
* ``block_sparse_attn``: a query row whose keep mask selects no visible key
  gets a zero output (the reference kernel returns the mean of the masked
  values there); the selector never produces such rows (sink forced).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

import _capi


def _operand(name, t, dtype=None):
    """A 16-bit device operand the kernels can read (head_dim stride 1,
    16-byte aligned rows); dtype: the format the call's other tensors have."""
    assert t.is_cuda, f"{name} must be a HIP device tensor"
    _capi.dtype_code(t.dtype)
    assert dtype is None or t.dtype == dtype, f"{name}: {dtype} required (as q), got {t.dtype}"
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def attn_workspace(B: int, Hk: int, N: int, D: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    """Workspace of ``ugbsa_attn_fwd`` (K and V in the kernel's operand
    order, 16-bit elements, then the tile schedule)."""
    n = _capi.lib().ugbsa_attn_workspace_elems(B, Hk, N, D)
    return torch.empty(n, dtype=dtype, device=device)


def block_sparse_attn_v2(q, k, v, kv_idx, scale, block_n=64, block_m=64,
                         num_warps=4, num_stages=1, out=None, workspace=None):
    """Per-tile-selection block-sparse causal attention (HIP, bf16 / fp16 MFMA).

    q : [B, H, M, D] bf16 or fp16; k, v : [B, Hk, N, D] in q's dtype (Hk == H
    or H % Hk == 0)
    kv_idx : [B, H, ceil(M / block_m), MAX_KEPT] int32, sentinel = NB skipped
    Returns out [B, H, M, D] (``out`` if given).
    """
    assert q.dim() == 4 and k.shape == v.shape and q.shape[0] == k.shape[0] \
        and q.shape[-1] == k.shape[-1], "q [B,H,M,D], k = v [B,Hk,N,D] expected"
    assert q.shape[2] == k.shape[2], "query length must equal key length (one-shot prefill)"
    assert q.is_cuda and kv_idx.dtype == torch.int32
    assert block_n == 64, "key blocks are 64 tokens"
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    assert H % Hk == 0, "query heads must be a multiple of KV heads"
    assert kv_idx.dim() == 4 and tuple(kv_idx.shape[:3]) == (B, H, (M + block_m - 1) // block_m)
    q = _operand("q", q)
    k = _operand("k", k, q.dtype)
    v = _operand("v", v, q.dtype)
    if kv_idx.stride(-1) != 1:
        kv_idx = kv_idx.contiguous()
    if out is None:
        out = torch.empty_like(q)
    assert out.shape == q.shape and out.dtype == q.dtype and out.stride(-1) == 1
    if workspace is None:
        workspace = attn_workspace(B, Hk, N, D, q.device, q.dtype)
    lib = _capi.lib()
    rc = lib.ugbsa_attn_fwd(
        q.data_ptr(), *q.stride(),
        k.data_ptr(), *k.stride(),
        v.data_ptr(), *v.stride(),
        kv_idx.data_ptr(), *kv_idx.stride(),
        B, H, Hk, M, N, D, _capi.dtype_code(q.dtype), kv_idx.shape[2], kv_idx.shape[3], block_m,
        float(scale), out.data_ptr(), *out.stride(), workspace.data_ptr(), workspace.numel(),
        _capi.stream_ptr(q.device))
    _capi.check(rc, "block_sparse_attn_v2")
    return out


def keep_kv_idx(keep, block_m=64, want_rowmask=True):
    """HIP compaction of a device keep mask [B, H, M, NB] (bool).

    Returns (kv_idx [B, H, Qt, NB] int32 ascending and NB-padded, rowmask
    [B, H, Qt, NB] int64 — bit r set where tile row r keeps the listed block —
    or None, MAX_KEPT).  Synchronises once for MAX_KEPT, as the reference.
    """
    assert keep.is_cuda and keep.dtype == torch.bool and keep.dim() == 4
    keep = keep.contiguous()
    B, H, M, NB = keep.shape
    qt = (M + block_m - 1) // block_m
    kv = torch.empty(B, H, qt, NB, dtype=torch.int32, device=keep.device)
    rm = torch.empty(B, H, qt, NB, dtype=torch.int64, device=keep.device) if want_rowmask else None
    counts = torch.empty(B, H, qt, dtype=torch.int32, device=keep.device)
    _capi.check(_capi.lib().ugbsa_keep_kv_idx(keep.data_ptr(), B, H, M, NB, block_m, kv.data_ptr(),
                                              _capi.ptr(rm), counts.data_ptr(),
                                              _capi.stream_ptr(keep.device)),
                "keep_kv_idx")
    max_kept = max(1, int(counts.max().item()))
    return kv, rm, max_kept


def block_sparse_attn(q, k, v, keep, scale, block_n=64, block_m=64,
                      num_warps=4, num_stages=1, out=None, workspace=None):
    """Per-row-selection block-sparse causal attention (HIP, bf16 / fp16 MFMA).

    q : [B, H, M, D] bf16 or fp16; k, v : [B, Hk, N, D] in q's dtype; keep : [B, H, M, NB]
    bool (True = the row attends to the block).  Same contract as
    src/triton_block_attn.py:149-182: per Q tile the union of its rows'
    blocks is visited in ascending order (``_compute_kv_idx``) and each row
    only sees the keys of its own kept blocks, causally.
    """
    assert q.dim() == 4 and k.shape == v.shape and q.shape[0] == k.shape[0] \
        and q.shape[-1] == k.shape[-1], "q [B,H,M,D], k = v [B,Hk,N,D] expected"
    assert q.shape[2] == k.shape[2], "query length must equal key length (one-shot prefill)"
    assert q.is_cuda and keep.dtype == torch.bool
    assert block_n == 64, "key blocks are 64 tokens"
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    assert H % Hk == 0, "query heads must be a multiple of KV heads"
    assert tuple(keep.shape[:3]) == (B, H, M), "keep [B, H, M, NB] expected"
    kv, rm, max_kept = keep_kv_idx(keep, block_m)
    q = _operand("q", q)
    k = _operand("k", k, q.dtype)
    v = _operand("v", v, q.dtype)
    if out is None:
        out = torch.empty_like(q)
    assert out.shape == q.shape and out.dtype == q.dtype and out.stride(-1) == 1
    if workspace is None:
        workspace = attn_workspace(B, Hk, N, D, q.device, q.dtype)
    rc = _capi.lib().ugbsa_attn_fwd_rows(
        q.data_ptr(), *q.stride(),
        k.data_ptr(), *k.stride(),
        v.data_ptr(), *v.stride(),
        kv.data_ptr(), rm.data_ptr(), *kv.stride(),
        B, H, Hk, M, N, D, _capi.dtype_code(q.dtype), kv.shape[2], max_kept, block_m,
        float(scale), out.data_ptr(), *out.stride(), workspace.data_ptr(), workspace.numel(),
        _capi.stream_ptr(q.device))
    _capi.check(rc, "block_sparse_attn")
    return out


def _compute_kv_idx(keep, block_m):
    """keep [B, H, M, NB] bool -> (kv_idx [B, H, Qt, MAX_KEPT] int32 ascending,
    NB-padded; MAX_KEPT).  Same contract as src/triton_block_attn.py:125-146:
    the HIP kernel for device tensors, torch for host tensors."""
    if keep.is_cuda:
        kv, _, max_kept = keep_kv_idx(keep, block_m, want_rowmask=False)
        return kv[..., :max_kept].contiguous(), max_kept
    B, H, M, NB = keep.shape
    q_tiles = (M + block_m - 1) // block_m
    pad = q_tiles * block_m - M
    if pad:
        keep = F.pad(keep, (0, 0, 0, pad))
    any_keep = keep.reshape(B, H, q_tiles, block_m, NB).any(dim=-2)
    blocks = torch.arange(NB, device=keep.device, dtype=torch.int32)
    masked = torch.where(any_keep, blocks.view(1, 1, 1, NB),
                         torch.full((), NB, device=keep.device, dtype=torch.int32))
    ordered, _ = masked.sort(dim=-1)
    max_kept = max(1, int((ordered < NB).sum(dim=-1).max().item()))
    return ordered[..., :max_kept].contiguous(), max_kept


def reference_attn_fp32(q, k, v, keep, scale, block_n=64):
    """``reference_attn``'s masked SDPA, computed and returned in fp32
    (inputs upcast): the tests' reference, kept apart from the drop-in."""
    B, H, M, D = q.shape
    N = k.shape[-2]
    NB = keep.shape[-1]
    if k.shape[1] != H:
        rep = H // k.shape[1]
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    kk = (keep.unsqueeze(-1).expand(B, H, M, NB, block_n)
          .reshape(B, H, M, NB * block_n)[..., :N])
    causal = (torch.arange(N, device=q.device).view(1, N)
              <= torch.arange(M, device=q.device).view(M, 1))
    return F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                          attn_mask=kk & causal, scale=scale)


def reference_attn(q, k, v, keep, scale, block_n=64):
    """SDPA with the materialised keep-and-causal mask (src/triton_block_attn.py:301-312).

    Returns the inputs' dtype, as the reference's SDPA call does.  The
    products run in fp32 (inputs upcast, result rounded once): the bf16 SDPA
    math path issues batched products on transposed views, which this ROCm
    build has faulted on, and the fp32 form is the closer reference anyway.
    """
    return reference_attn_fp32(q, k, v, keep, scale, block_n).to(q.dtype)
