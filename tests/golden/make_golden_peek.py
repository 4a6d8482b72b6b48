"""Write rollout_peek golden vectors from the reference planner itself.

Run in the build container only (the reference tree is absent on GPU boxes):

    python tests/golden/make_golden_peek.py [/root/reference/src]

The reference ships no test of ``_block_select_mask_peek``
(src/sparse_attention.py:455-583): its planning-row choice, the safe / band
split, the candidate enumeration order and the first-best rule are only
written in that code.  For each case of ``tests/peek_model.py`` (a seeded
tiny Qwen2 in fp32 on the CPU and seeded planner inputs) this records the
reference's ``keep`` mask, a checksum of the block scores it ranked (a spy on
the first ``Tensor.argsort``; the tests recompute them and must match it bit
for bit), the K-mean pool it cached for the layer, the rows whose ``keep``
differs from its top-k baseline, and a checksum of the inputs so that a drift
of the generators is detected.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
TESTS = os.path.dirname(HERE)
sys.path.insert(0, TESTS)
sys.path.insert(0, HERE)
import peek_model as PM  # noqa: E402
from make_golden import sha  # noqa: E402


class ArgsortSpy:
    def __init__(self):
        self.first = None

    def __enter__(self):
        self._orig = torch.Tensor.argsort
        spy = self

        def argsort(t, *a, **kw):
            if spy.first is None:
                spy.first = t.detach().clone()
            return spy._orig(t, *a, **kw)

        torch.Tensor.argsort = argsort
        return self

    def __exit__(self, *exc):
        torch.Tensor.argsort = self._orig


def main():
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, ref_src)
    import sparse_attention as ref      # the reference module (CPU, fp32)
    torch.set_num_threads(1)
    model = PM.tiny_qwen2()
    pos = PM.position_embeddings(model)
    out = {"params_sha": np.array(sha(*[p.detach().numpy() for _, p in
                                        sorted(model.named_parameters())]))}
    grp = PM.HQ // PM.HKV
    for name, seed, layer, metric, with_pool, extra in PM.CASES:
        q, k, v, hidden, pool = PM.planner_inputs(seed, layer, with_pool)
        ref.SEL.__init__()
        for f, val in dict(PM.SEL_FIELDS, **extra).items():
            setattr(ref.SEL, f, val)
        ref.SEL.mode = "rollout_peek"
        ref.SEL.peek_metric = metric
        ref.SEL.model_ref = model
        ref.SEL.hidden_at = {layer: hidden}
        ref.SEL.k_pool_at = {} if pool is None else {layer + 1: pool}
        module = model.model.layers[layer].self_attn
        k_rep = k.repeat_interleave(grp, dim=1)
        v_rep = v.repeat_interleave(grp, dim=1)
        with torch.no_grad(), ArgsortSpy() as spy:
            keep = ref._block_select_mask_peek(module, q, k_rep, v_rep, module.scaling, pos)
        arrays = [q.numpy(), k.numpy(), v.numpy(), hidden.numpy()]
        if pool is not None:
            arrays.append(pool.numpy())
        out[f"{name}/inputs_sha"] = np.array(sha(*arrays))
        out[f"{name}/keep_bits"] = np.packbits(keep.numpy().astype(np.uint8), axis=-1)
        bs = spy.first
        out[f"{name}/block_score_sha"] = np.array(sha(bs.numpy().astype(np.float32)))
        out[f"{name}/k_pool"] = ref.SEL.k_pool_at[layer].numpy().astype(np.float32)
        # baseline: the same top-k the planner starts from (:513-519)
        base = bs.argsort(dim=-1, descending=True).argsort(dim=-1) < float(
            max(min(ref.SEL.budget_blocks, ref.SEL.k_max), ref.SEL.k_min))
        base[..., 0] = True
        base[0, :, torch.arange(PM.S), torch.arange(PM.S) // 64] = True
        changed = np.nonzero((keep != base)[0].any(dim=(0, 2)).numpy())[0]
        out[f"{name}/changed_rows"] = changed.astype(np.int64)
        print(f"{name}: rows changed from the baseline: {changed.tolist()}")
    path = os.path.join(HERE, "peek_cases.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
