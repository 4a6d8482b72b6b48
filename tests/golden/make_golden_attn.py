"""Write attention golden vectors from the reference's own ``reference_attn``.

Run in the build container only (the reference tree is absent on GPU boxes):

    python tests/golden/make_golden_attn.py [/root/reference/src]

``reference_attn`` (src/triton_block_attn.py:301-312) is the reference's
check of its attention kernels: SDPA over a materialised keep-and-causal mask.
It is plain torch and runs on the CPU, in fp32 here.  Each case draws
bf16-representable Q/K/V, a per-tile kv_idx (sink forced, no repeated block,
sentinel NB in unused slots) and expands it to the per-row keep mask the v2
kernel's semantics imply (every row of tile t keeps the tile's listed blocks;
causality inside ``reference_attn``).  Stored: inputs as bf16 bit patterns,
kv_idx, the fp32 output.  GQA cases pass repeat_kv'd K/V to the reference, as
its dispatcher does.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, B, H, Hk, S, D, blocks listed per tile, seed)
CASES = [
    ("dense_d64", 1, 4, 4, 256, 64, None, 1),      # every visible block (case A)
    ("gqa_ragged_d128", 1, 4, 2, 337, 128, 3, 2),  # ragged tail, 2 query heads per KV head
    ("multi_d256", 2, 2, 1, 200, 256, 2, 3),       # batch 2, head_dim 256, ragged
]


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def make_case(B, H, Hk, S, D, per_tile, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).float()
    k = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16).float()
    v = torch.randn(B, Hk, S, D, generator=g).to(torch.bfloat16).float()
    nb = qt = (S + 63) // 64
    slots = qt if per_tile is None else per_tile + 1
    kv = torch.full((B, H, qt, slots), nb, dtype=torch.int32)
    for b in range(B):
        for h in range(H):
            for t in range(qt):
                if per_tile is None:
                    picks = list(range(t + 1))
                else:
                    rest = torch.randperm(t, generator=g)[:per_tile] + 1 if t > 0 else torch.empty(0)
                    picks = [0] + sorted(int(x) for x in rest)   # sink + distinct blocks <= t
                kv[b, h, t, :len(picks)] = torch.tensor(picks, dtype=torch.int32)
    return q, k, v, kv


def keep_from_kv_idx(kv, S):
    B, H, qt, _ = kv.shape
    nb = (S + 63) // 64
    keep = torch.zeros(B, H, S, nb, dtype=torch.bool)
    for t in range(qt):
        rows = slice(64 * t, min(S, 64 * t + 64))
        for b in range(B):
            for h in range(H):
                blks = [int(x) for x in kv[b, h, t] if 0 <= int(x) < nb and int(x) <= t]
                keep[b, h, rows, blks] = True
    return keep


def main():
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, ref_src)
    from triton_block_attn import reference_attn  # the reference module (CPU, fp32)
    out = {}
    for name, B, H, Hk, S, D, per_tile, seed in CASES:
        q, k, v, kv = make_case(B, H, Hk, S, D, per_tile, seed)
        keep = keep_from_kv_idx(kv, S)
        kr = k.repeat_interleave(H // Hk, dim=1)
        vr = v.repeat_interleave(H // Hk, dim=1)
        o = reference_attn(q, kr, vr, keep, D ** -0.5)
        assert torch.isfinite(o).all()
        out[f"{name}/q_bf16"] = bf16_bits(q)
        out[f"{name}/k_bf16"] = bf16_bits(k)
        out[f"{name}/v_bf16"] = bf16_bits(v)
        out[f"{name}/kv_idx"] = kv.numpy()
        out[f"{name}/out"] = o.numpy().astype(np.float32)
        out[f"{name}/scale"] = np.float32(D ** -0.5)
        print(name, tuple(q.shape), tuple(kv.shape), float(o.abs().max()))
    np.savez_compressed(os.path.join(HERE, "attention_reference.npz"), **out)


if __name__ == "__main__":
    main()
