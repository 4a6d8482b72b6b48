"""rollout_peek on the GPU: HIP top-k baseline + the planner on device tensors.

The planner's logic is pinned bit for bit against the reference on the CPU
(tests/test_peek_cpu.py).  Here the same planner runs on the GPU over the HIP
selector's fp32 scores and baseline keep mask, with the tiny Qwen2 in bf16:

* rows outside the planning set keep the HIP top-k baseline exactly;
* the planning rows are those the CPU recomputes from the GPU's own scores;
* each planned row keeps its safe blocks, one candidate of its band, the sink
  and its own block, and agrees with the fp32 CPU planner run on the same
  scores except where the two candidates' fp32 scores are within 2 % (the
  candidate forward runs in bf16 here);
* end to end through transformers (``attn_implementation="block_sparse"``,
  hooks installed): finite logits and the ``SEL.log`` diagnostics.
"""

import numpy as np
import pytest
import torch

import peek_model as PM
import sparse_attention as sa

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture
def fresh_sel():
    saved = dict(sa.SEL.__dict__)
    sa.SEL.__init__()
    yield sa.SEL
    sa.SEL.__dict__.clear()
    sa.SEL.__dict__.update(saved)


@pytest.mark.parametrize("case", [c for c in PM.CASES if c[0] in ("peak", "xh", "resnorm")],
                         ids=lambda c: c[0])
def test_peek_gpu_vs_cpu_planner(hip_lib, fresh_sel, case):
    name, seed, layer, metric, with_pool, extra = case
    print(f"[case] rollout_peek gpu {name}", flush=True)
    torch.set_num_threads(1)
    m32 = PM.tiny_qwen2()
    m16 = PM.tiny_qwen2(dtype=torch.bfloat16).to(DEV)
    q, k, v, hidden, pool = PM.planner_inputs(seed, layer, with_pool)
    sel = fresh_sel
    for f, val in dict(PM.SEL_FIELDS, **extra).items():
        setattr(sel, f, val)
    sel.mode, sel.peek_metric, sel.model_ref = "rollout_peek", metric, m16
    sel.hidden_at = {layer: hidden.to(DEV, torch.bfloat16)}
    sel.k_pool_at = {} if pool is None else {layer + 1: pool.to(DEV, torch.bfloat16)}
    mod16 = m16.model.layers[layer].self_attn
    qd, kd, vd = (x.to(DEV, torch.bfloat16) for x in (q, k, v))
    # the HIP baseline and scores the planner starts from
    base_sel = sa.Selector()
    for f, val in dict(PM.SEL_FIELDS, **extra).items():
        setattr(base_sel, f, val)
    base_sel.mode = "topk"
    base = sa.select_mask_v1(qd, kd, mod16.scaling, sel=base_sel, want_scores=True)
    trace = {}
    with torch.no_grad():
        keep = sa._block_select_mask_peek(mod16, qd, kd, vd, mod16.scaling,
                                          PM.position_embeddings(m16, torch.bfloat16, DEV),
                                          trace=trace)
    torch.cuda.synchronize()
    keep = keep.cpu()
    scores = base.scores.float().cpu()
    base_keep = base.keep.cpu()
    nb = PM.S // 64
    # the planning rows from the GPU's scores, recomputed on the CPU
    vis = (torch.arange(nb) * 64).view(1, nb) <= torch.arange(PM.S).view(PM.S, 1)
    bud, w = sel.budget_blocks, sel.peek_swap_w
    tv = torch.topk(scores[0].masked_fill(~vis, float("-inf")), k=min(bud + 1, nb), dim=-1).values
    peak = (tv[..., 0] - tv[..., -1]).mean(dim=0)
    peak = torch.where(vis.sum(-1) >= bud + w, peak, torch.full_like(peak, -float("inf")))
    rows = set(peak.argsort(descending=True)[:sel.peek_rows_per_layer].tolist())
    assert set(trace) == rows          # every planning row here has a full band
    other = [r for r in range(PM.S) if r not in trace]
    assert torch.equal(keep[:, :, other], base_keep[:, :, other])
    # the fp32 CPU planner on the same scores and baseline
    sel.model_ref = m32
    sel.hidden_at = {layer: hidden}
    kp = sel.k_pool_at[layer].float().cpu()
    sel.k_pool_at = {layer: kp} if pool is None else {layer: kp, layer + 1: pool}
    trace32 = {}
    with torch.no_grad():
        keep32 = sa.peek_plan(m32.model.layers[layer].self_attn, q, k, v,
                              m32.model.layers[layer].self_attn.scaling,
                              PM.position_embeddings(m32), scores, base_keep.clone(), layer,
                              trace=trace32)
    assert set(trace32) == set(trace)
    n_same = 0
    for r, tr in trace.items():
        row = set(keep[0, 0, r].nonzero().flatten().tolist())
        assert row == set(tr["chosen"]) | {0, r // 64}
        assert all(torch.equal(keep[0, 0, r], keep[0, h, r]) for h in range(PM.HQ))
        if torch.equal(keep[0, :, r], keep32[0, :, r]):
            n_same += 1
            continue
        s32 = dict(zip(map(tuple, trace32[r]["candidates"]), trace32[r]["scores"]))
        a, b = s32[tuple(tr["chosen"])], s32[tuple(trace32[r]["chosen"])]
        assert abs(a - b) <= 0.02 * max(abs(a), abs(b), 1e-6), (r, a, b)
    print(f"  {n_same} of {len(trace)} planned rows identical to the fp32 planner", flush=True)


def test_peek_end_to_end_hf(hip_lib, fresh_sel):
    print("[case] rollout_peek end to end", flush=True)
    model = PM.tiny_qwen2(dtype=torch.bfloat16, attn="block_sparse").to(DEV)
    sel = fresh_sel
    for f, val in PM.SEL_FIELDS.items():
        setattr(sel, f, val)
    sel.mode, sel.log = "rollout_peek", True
    sa.install_rollout_hooks(model)
    ids = torch.randint(0, 64, (1, PM.S), generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.no_grad():
        logits = model(ids).logits
    torch.cuda.synchronize()
    assert torch.isfinite(logits.float()).all()
    assert sorted(sel.hidden_at) == list(range(PM.N_LAYERS))
    assert sorted(sel.kept_blocks) == list(range(PM.N_LAYERS))
    assert len(sel.budget_samples) == PM.N_LAYERS
    assert sorted(sel.k_pool_at) == list(range(PM.N_LAYERS))
