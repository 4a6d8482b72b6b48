"""rollout_peek planner (src/sparse_attention.py:386-583) on the CPU.

``peek_plan`` is device-agnostic torch around the model's own modules; here
it runs in fp32 on the CPU on the inputs of ``tests/peek_model.py`` and must
reproduce the reference planner's ``keep`` mask bit for bit
(``tests/golden/peek_cases.npz``, written by ``make_golden_peek.py`` from the
reference itself).  The block scores are recomputed as the reference forms
them and checked against the reference's own by checksum; the top-k baseline
comes from the v1 oracle.  Both K/V layouts are run: repeat_kv'd (H heads,
as the reference receives them) and grouped (Hk heads, as this build's
dispatcher passes them).
"""

import os

import numpy as np
import pytest
import torch

import peek_model as PM
import sparse_attention as sa
from oracle import selector_v1 as OV1

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "peek_cases.npz")


def sha(*arrays):
    import hashlib
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.fixture(scope="module")
def model():
    torch.set_num_threads(1)
    m = PM.tiny_qwen2()
    g = np.load(GOLDEN)
    assert sha(*[p.detach().numpy() for _, p in sorted(m.named_parameters())]) == str(g["params_sha"])
    return m


@pytest.mark.parametrize("grouped", [False, True], ids=["repeat_kv", "gqa"])
@pytest.mark.parametrize("case", PM.CASES, ids=[c[0] for c in PM.CASES])
def test_peek_plan_matches_reference(model, case, grouped):
    name, seed, layer, metric, with_pool, extra = case
    g = np.load(GOLDEN)
    q, k, v, hidden, pool = PM.planner_inputs(seed, layer, with_pool)
    arrays = [q.numpy(), k.numpy(), v.numpy(), hidden.numpy()] + ([pool.numpy()] if pool is not None else [])
    assert sha(*arrays) == str(g[f"{name}/inputs_sha"]), "input generator drifted"
    grp = PM.HQ // PM.HKV
    k_rep, v_rep = k.repeat_interleave(grp, dim=1), v.repeat_interleave(grp, dim=1)
    module = model.model.layers[layer].self_attn
    nb = PM.S // 64
    # block scores formed as the reference forms them (K-mean, model dtype)
    kp = k_rep.view(1, PM.HQ, nb, 64, PM.HEAD_DIM).mean(dim=3)
    bs = torch.matmul(q, kp.transpose(2, 3)) * module.scaling
    vis = (torch.arange(nb) * 64).view(1, nb) <= torch.arange(PM.S).view(PM.S, 1)
    bs = bs.masked_fill(~vis, float("-inf"))
    assert sha(bs.numpy()) == str(g[f"{name}/block_score_sha"])
    assert np.array_equal(kp.numpy(), g[f"{name}/k_pool"])
    saved = dict(sa.SEL.__dict__)
    try:
        sa.SEL.__init__()
        for f, val in dict(PM.SEL_FIELDS, **extra).items():
            setattr(sa.SEL, f, val)
        sa.SEL.mode, sa.SEL.peek_metric, sa.SEL.model_ref = "rollout_peek", metric, model
        sa.SEL.hidden_at = {layer: hidden}
        sa.SEL.k_pool_at = {layer: kp} if pool is None else {layer: kp, layer + 1: pool}
        cfg = OV1.SelectorV1Config.from_selector(sa.SEL)
        cfg.mode = "topk"
        base = OV1.select_mask_from_scores(bs.numpy(), PM.S, cfg).keep
        trace = {}
        with torch.no_grad():
            keep = sa.peek_plan(module, q, k if grouped else k_rep, v if grouped else v_rep,
                                module.scaling, PM.position_embeddings(model), bs,
                                torch.from_numpy(base.copy()), layer, trace=trace)
    finally:
        sa.SEL.__dict__.clear()
        sa.SEL.__dict__.update(saved)
    ref = np.unpackbits(g[f"{name}/keep_bits"], axis=-1)[..., :nb].astype(bool)
    assert np.array_equal(keep.numpy(), ref), f"{name}: keep differs from the reference planner"
    changed = np.nonzero((keep.numpy() != base)[0].any(axis=(0, 2)))[0]
    assert np.array_equal(changed, g[f"{name}/changed_rows"])
    # every planned row kept its budget: safe + chosen band blocks + sink + own
    for r, tr in trace.items():
        if tr.get("chosen") is not None:
            row = keep[0, 0, r].nonzero().flatten().tolist()
            assert set(row) == set(tr["chosen"]) | {0, r // 64}
    if name == "out_of_range":
        assert not trace and changed.size == 0
    if name == "last_layer":      # no next layer: every candidate scores 0, the first wins
        assert trace and all(tr["chosen"] == tr["candidates"][0] for tr in trace.values())
