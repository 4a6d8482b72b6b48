"""The HF drop-in end to end: tiny random-weight Qwen2 and Qwen3.5-MoE models
built with ``from_config`` (no download) and run with
``attn_implementation="block_sparse"`` (src/sparse_attention.py:751-806).

Every full-attention layer's call is captured at the real transformers call
site; its ``kv_idx`` must equal the oracle's selection on the kernel's own
fp32 tile scores, and its output the oracle's attention over that ``kv_idx``
(max-abs 2e-2 / mean-abs 2e-3).  Dense mode through the same hook must match
the model's SDPA implementation; decode (Q == 1) runs through SDPA; the
``SEL.log`` diagnostics (src/sparse_attention.py:726-746) feed
``needle_hit_rate`` (src/poc_core.py:77-85).
"""

import numpy as np
import pytest
import torch

import sparse_attention as sa
from oracle import attention as OA
from oracle import selector as OS
from parity import f32np

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
MAX_ABS, MEAN_ABS = 2e-2, 2e-3
S = 4096                       # 64 blocks: k_base 16 (budget 4 clamped to k_min 8), k_slots 32


def tiny_qwen2():
    from transformers.models.qwen2 import Qwen2Config
    return Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                       num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                       max_position_embeddings=8192)


def tiny_qwen35_moe():
    """Qwen3.5-MoE text stack: three gated-delta-net layers, then one
    full-attention layer (head_dim 256, QK-norm, output gate, partial rope)."""
    from transformers.models.qwen3_5_moe import Qwen3_5MoeTextConfig
    return Qwen3_5MoeTextConfig(
        vocab_size=512, hidden_size=256, num_hidden_layers=4, num_attention_heads=4,
        num_key_value_heads=2, head_dim=256, linear_key_head_dim=32, linear_value_head_dim=32,
        linear_num_key_heads=4, linear_num_value_heads=8, moe_intermediate_size=64,
        shared_expert_intermediate_size=64, num_experts=4, num_experts_per_tok=2,
        layer_types=["linear_attention"] * 3 + ["full_attention"],
        max_position_embeddings=8192)


FAMILIES = {"qwen2": (tiny_qwen2, 2), "qwen3_5_moe": (tiny_qwen35_moe, 1)}


def build(make_cfg, impl, seed=0, dtype=torch.bfloat16):
    from transformers import AutoModelForCausalLM
    torch.manual_seed(seed)
    model = AutoModelForCausalLM.from_config(make_cfg(), attn_implementation=impl)
    return model.to(device=DEV, dtype=dtype).eval()


def input_ids(seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 512, (1, S), generator=g).to(DEV)


class Capture:
    """Records each v2 selection made by the dispatcher (the selector is
    looked up at call time, so a wrapper over the module global sees every
    layer's q / k and kv_idx)."""

    def __init__(self):
        self.calls = []
        self.orig = sa._block_select_kv_idx_v2

    def __enter__(self):
        def wrapped(query, key_states, scaling, block_m=64):
            kv = self.orig(query, key_states, scaling, block_m)
            self.calls.append((query.detach().clone(), key_states.detach().clone(), scaling, kv.clone()))
            return kv
        sa._block_select_kv_idx_v2 = wrapped
        return self

    def __exit__(self, *exc):
        sa._block_select_kv_idx_v2 = self.orig


def sel_policy(policy):
    sa.SEL.kernel_v2 = True
    sa.SEL.budget_blocks = 4
    sa.SEL.router_grain, sa.SEL.router_mode, sa.SEL.router_quantile = "row", "quantile", 0.25
    sa.SEL.mode = "router" if policy.startswith("router") else policy
    sa.SEL.router_score = "quest" if policy in ("router_quest", "quest") else "mean"


@pytest.fixture
def sel_state():
    saved = dict(vars(sa.SEL))
    yield sa.SEL
    sa.SEL.__dict__.update(saved)
    sa.SEL.reset_log()


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("policy", ["router_quest", "topk"])
def test_model_prefill_layers_match_oracle(hip_lib, sel_state, family, policy):
    check_prefill_layers(family, policy, torch.bfloat16)


@pytest.mark.parametrize("policy", ["router_quest", "topk"])
def test_qwen2_fp16_prefill_layers_match_oracle(hip_lib, sel_state, policy):
    """The same drop-in check on a model loaded in fp16: q / k / v reach the
    selector and kernel 3 as fp16 and the output comes back in fp16."""
    check_prefill_layers("qwen2", policy, torch.float16)


def check_prefill_layers(family, policy, dtype):
    print(f"[case] hf {family} {policy} {dtype}", flush=True)
    make_cfg, n_full = FAMILIES[family]
    sel_policy(policy)
    model = build(make_cfg, "block_sparse", dtype=dtype)
    # capture attention outputs too: hook the dispatcher's kernel call
    outs = []
    orig_attn = sa.block_sparse_attn_v2

    def attn_wrapped(q, k, v, kv_idx, scale, *a, **kw):
        o = orig_attn(q, k, v, kv_idx, scale, *a, **kw)
        outs.append((q.detach().clone(), k.detach().clone(), v.detach().clone(),
                     kv_idx.clone(), o.detach().clone(), scale))
        return o
    sa.block_sparse_attn_v2 = attn_wrapped
    try:
        with Capture() as cap, torch.no_grad():
            logits = model(input_ids()).logits
    finally:
        sa.block_sparse_attn_v2 = orig_attn
    torch.cuda.synchronize()
    assert torch.isfinite(logits.float()).all()
    assert len(cap.calls) == n_full and len(outs) == n_full
    cfg = OS.SelectorConfig.from_selector(sa.SEL)
    for li, ((q, k, scaling, kv), (q2, k2, v2, kv2, o, scale)) in enumerate(zip(cap.calls, outs)):
        assert torch.equal(kv, kv2)
        assert q.dtype == k.dtype == v2.dtype == o.dtype == dtype
        assert q.shape[1] == 4 and k.shape[1] == 2          # GQA reaches the kernels un-repeated
        res = sa.select_v2(q, k, scaling, want_tile_score=True)
        sel = OS.select_from_tile_scores(res.tile_score.cpu().numpy(), cfg)
        assert np.array_equal(sel.kv_idx, kv.cpu().numpy()), f"layer {li} kv_idx"
        n_blocks = S // 64
        dropped = (kv.cpu().numpy() >= n_blocks).mean()
        print(f"  layer {li}: sentinel fraction {dropped:.2f}", flush=True)
        ref = OA.gathered_attention(q2.float().cpu().numpy(), k2.float().cpu().numpy(),
                                    v2.float().cpu().numpy(), kv2.cpu().numpy(), scale)
        err = np.abs(f32np(o) - ref)
        print(f"  layer {li}: max|d|={err.max():.3e} mean|d|={err.mean():.3e}", flush=True)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_model_dense_mode_and_decode(hip_lib, sel_state, family):
    """SEL.mode = "dense" through the block_sparse hook equals the model's own
    SDPA attention; generate() decodes (Q == 1) through SDPA after a sparse
    prefill."""
    print(f"[case] hf {family} dense/decode", flush=True)
    make_cfg, _ = FAMILIES[family]
    ids = input_ids(2)[:, :512]
    sa.SEL.mode = "dense"
    with torch.no_grad():
        got = build(make_cfg, "block_sparse")(ids).logits.float()
        want = build(make_cfg, "sdpa")(ids).logits.float()
    err = (got - want).abs().max().item()
    print(f"  dense logits max|d|={err:.3e}", flush=True)
    assert err <= 2e-2
    sel_policy("router_quest")
    model = build(make_cfg, "block_sparse")
    ids = input_ids(3)
    with torch.no_grad():
        first = model(ids).logits[0, -1].argmax().item()
        gen = model.generate(ids, max_new_tokens=4, do_sample=False)
    assert gen.shape == (1, S + 4) and gen[0, S].item() == first


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_sel_log_diagnostics_and_needle_hit_rate(hip_lib, sel_state, family):
    print(f"[case] hf {family} SEL.log", flush=True)
    make_cfg, n_full = FAMILIES[family]
    sel_policy("router_quest")
    sa.SEL.log = True
    sa.SEL.reset_log()
    model = build(make_cfg, "block_sparse")
    with Capture() as cap, torch.no_grad():
        model(input_ids(4))
    n_blocks = S // 64
    assert len(sa.SEL.kept_blocks) == n_full and len(sa.SEL.router_trigger_rate) == n_full
    assert sa.SEL.budget_samples == [float(sa.budgets(n_blocks)[1])] * n_full == [32.0] * n_full
    for li, (_, _, _, kv) in enumerate(cap.calls):
        last = kv[0, :, -1, :].cpu().numpy().ravel()
        want = np.zeros(n_blocks, bool)
        want[last[last < n_blocks]] = True
        kept = sa.SEL.kept_blocks[li].numpy()
        assert kept.dtype == bool and np.array_equal(kept, want)
        assert kept[0] and kept[n_blocks - 1]          # sink and the tile's own block
    for rate in sa.SEL.router_trigger_rate:
        assert 0.0 < rate < 1.0
    kept0 = sa.SEL.kept_blocks[0].numpy()
    hit = [b for b in range(n_blocks) if kept0[b]][:3]
    miss = [b for b in range(n_blocks) if not kept0[b]][:1]
    manual = np.mean([sum(1 for b in hit + miss if kb[b]) / 4
                      for kb in (v.numpy() for v in sa.SEL.kept_blocks.values())])
    assert sa.needle_hit_rate(hit + miss) == pytest.approx(manual)
    assert sa.needle_hit_rate([]) == 1.0


@pytest.mark.parametrize("family", sorted(FAMILIES))
def test_v1_router_log_line_after_install_rollout_hooks(hip_lib, sel_state, family, capsys):
    """The reference's harnesses call install_rollout_hooks(model) after
    loading (src/modal_app.py:67); on the v1 path (kernel_v2=False) with
    SEL.log the router then prints its running means once per prefill, on the
    model's last decoder layer (src/sparse_attention.py:355-375)."""
    print(f"[case] hf {family} v1 router log line", flush=True)
    make_cfg, n_full = FAMILIES[family]
    sel_policy("router_quest")
    sa.SEL.kernel_v2 = False
    sa.SEL.log = True
    sa.SEL.reset_log()
    model = build(make_cfg, "block_sparse")
    sa.install_rollout_hooks(model)
    capsys.readouterr()
    with torch.no_grad():
        model(input_ids(5))
    torch.cuda.synchronize()
    lines = [l for l in capsys.readouterr().out.splitlines() if l.startswith("  router[")]
    assert len(sa.SEL.router_trigger_rate) == n_full
    mean = lambda xs: sum(xs) / len(xs)
    want = ("  router[quantile/row]: trigger=%.3f eff_budget=%.1f margin=%.3f q=0.25"
            % (mean(sa.SEL.router_trigger_rate), mean(sa.SEL.router_eff_budget),
               mean(sa.SEL.router_margin_mean)))
    assert lines == [want]
    assert len(sa.SEL.hidden_at) == len(model.model.layers)
