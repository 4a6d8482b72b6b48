"""Write the v2-selector golden vectors from the reference itself (CPU, fp32).

Run in the build container only (the reference tree is absent on GPU boxes):

    python tests/golden/make_golden.py [/root/reference/src]

The reference ships no fixtures and no selector test, so the end-to-end
behaviour of ``_block_select_kv_idx_v2`` (src/sparse_attention.py:588-748) —
torch ``topk`` on the fp32 tile scores, ``kthvalue`` with NaN margins, the
row-grain mean — is recorded here as data.  A spy on ``Tensor.topk`` and
``Tensor.kthvalue`` captures the exact fp32 tile scores the reference ranked
and the threshold it drew, so the oracle can be checked on the reference's
own scores (bit-exact selection) and on its own scores (near-tie tolerance).

Inputs are bf16-representable fp32 drawn by the build's seeded generator;
small cases store them as bf16 bit patterns, the c1 case stores a SHA-256 of
the regenerated inputs instead of the 33 MB tensors.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "uncertainty-gated-block-sparse-attention_amd"))
import synth  # noqa: E402


def bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


class Spy:
    """Records inputs/outputs of Tensor.topk and Tensor.kthvalue."""

    def __init__(self):
        self.topk_in = None
        self.kth_in = None
        self.kth_k = None
        self.kth_out = None

    def __enter__(self):
        self._topk, self._kth = torch.Tensor.topk, torch.Tensor.kthvalue
        spy = self

        def topk(t, *a, **kw):
            spy.topk_in = t.detach().clone()
            return spy._topk(t, *a, **kw)

        def kthvalue(t, k, *a, **kw):
            out = spy._kth(t, k, *a, **kw)
            spy.kth_in, spy.kth_k, spy.kth_out = t.detach().clone(), int(k), out.values.clone()
            return out

        torch.Tensor.topk = topk
        torch.Tensor.kthvalue = kthvalue
        return self

    def __exit__(self, *exc):
        torch.Tensor.topk, torch.Tensor.kthvalue = self._topk, self._kth


POLICIES = [
    # name, SEL fields
    ("topk", dict(mode="topk")),
    ("quest", dict(mode="quest")),
    ("router_mean_row_quantile", dict(mode="router", router_score="mean",
                                      router_grain="row", router_mode="quantile")),
    ("router_quest_row_quantile", dict(mode="router", router_score="quest",
                                       router_grain="row", router_mode="quantile")),
    ("router_mean_cell_quantile", dict(mode="router", router_score="mean",
                                       router_grain="cell", router_mode="quantile")),
    ("router_quest_cell_quantile", dict(mode="router", router_score="quest",
                                        router_grain="cell", router_mode="quantile")),
    ("router_mean_cell_abs", dict(mode="router", router_score="mean",
                                  router_grain="cell", router_mode="abs")),
    ("router_quest_row_abs", dict(mode="router", router_score="quest",
                                  router_grain="row", router_mode="abs",
                                  router_tau=1e-40)),
    # quantile beyond the finite margins: threshold is NaN, nothing triggers
    ("router_quest_row_q090", dict(mode="router", router_score="quest",
                                   router_grain="row", router_mode="quantile",
                                   router_quantile=0.90)),
]


def run_reference(sa, q, k_rep, scaling, fields):
    sa.SEL.__init__()
    sa.SEL.kernel_v2 = True
    for f, val in fields.items():
        setattr(sa.SEL, f, val)
    with Spy() as spy:
        kv = sa._block_select_kv_idx_v2(q, k_rep, scaling)
    rec = {"kv_idx": kv.numpy().astype(np.int32),
           "tile_score": spy.topk_in.numpy().astype(np.float32)}
    if spy.kth_in is not None:
        rec["kth_in"] = spy.kth_in.numpy().astype(np.float32)
        rec["kth_k"] = np.int64(spy.kth_k)
        rec["kth_out"] = np.float32(spy.kth_out.item())
    return rec


def small_case(sa, name, S, Hq, Hkv, D, needles, budget, k_min, seed_layer, quantile):
    cfg = synth.LayerConfig(name, 0, 1, Hq, Hkv, S, D, torch.float32, needles, 0.0,
                            False, "router", "quest", budget)
    q, k, _ = synth.make_layer(cfg, seed_layer)
    q = q.to(torch.bfloat16).float()
    k = k.to(torch.bfloat16).float()
    k_rep = k.repeat_interleave(Hq // Hkv, dim=1)
    out = {"q_bf16": bf16_bits(q), "k_bf16": bf16_bits(k),
           "scaling": np.float64(D ** -0.5)}
    for pname, fields in POLICIES:
        fields = dict(fields, budget_blocks=budget, k_min=k_min)
        fields.setdefault("router_quantile", quantile)
        rec = run_reference(sa, q, k_rep, D ** -0.5, fields)
        for key, val in rec.items():
            out[f"{pname}/{key}"] = val
        out[f"{pname}/fields"] = np.array(repr(sorted(fields.items())))
    path = os.path.join(HERE, f"selector_{name}.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


def c1_case(sa):
    cfg = synth.CONFIGS["c1"]
    q, k, _ = synth.make_layer(cfg, 0)
    k_rep = k.repeat_interleave(cfg.Hq // cfg.Hkv, dim=1)
    out = {"input_sha256": np.array(sha(q.numpy(), k.numpy())),
           "scaling": np.float64(cfg.scaling)}
    fields = cfg.sel_fields()
    rec = run_reference(sa, q, k_rep, cfg.scaling, fields)
    for key, val in rec.items():
        out[f"router_quest_row_quantile/{key}"] = val
    fields_mean = dict(fields, router_score="mean")
    rec = run_reference(sa, q, k_rep, cfg.scaling, fields_mean)
    for key, val in rec.items():
        out[f"router_mean_row_quantile/{key}"] = val
    path = os.path.join(HERE, "selector_c1.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


def main():
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, ref_src)
    import sparse_attention as sa  # the reference module (CPU, fp32)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    # A: c1-like structure at a fixture size; k_min lowered so the router has
    # room (NB = 16, k_base = 4, k_slots = 8).
    small_case(sa, "a", S=1024, Hq=4, Hkv=2, D=64, needles=4, budget=2, k_min=1,
               seed_layer=11, quantile=0.25)
    # B: ragged — S not a multiple of 64 (padded last block and last tile).
    small_case(sa, "b_ragged", S=1000, Hq=2, Hkv=1, D=64, needles=3, budget=2, k_min=1,
               seed_layer=12, quantile=0.25)
    # C: k_base = NB/2 so k_slots = NB exactly (NB = 8).
    small_case(sa, "c_full", S=512, Hq=4, Hkv=1, D=64, needles=2, budget=2, k_min=1,
               seed_layer=13, quantile=0.25)
    c1_case(sa)


if __name__ == "__main__":
    main()
