"""HF registration and dense dispatch without a GPU: a tiny random Qwen2
built with attn_implementation="block_sparse" and SEL.mode = "dense" goes
through the hook (src/sparse_attention.py:751-806) and must equal the same
weights under transformers' own SDPA attention."""

import pytest
import torch

import sparse_attention as sa


def test_block_sparse_is_registered_with_transformers():
    from transformers import AttentionInterface
    assert sa.REGISTERED
    assert AttentionInterface._global_mapping["block_sparse"] is sa.block_sparse_attention


def test_dense_mode_through_the_hook_equals_sdpa():
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config
    cfg = Qwen2Config(vocab_size=256, hidden_size=128, intermediate_size=256,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=1024)
    ids = torch.randint(0, 256, (1, 192), generator=torch.Generator().manual_seed(0))
    saved = sa.SEL.mode
    try:
        sa.SEL.mode = "dense"
        outs = []
        for impl in ("block_sparse", "sdpa"):
            torch.manual_seed(0)
            model = AutoModelForCausalLM.from_config(cfg, attn_implementation=impl).eval()
            with torch.no_grad():
                outs.append(model(ids).logits)
        assert torch.allclose(outs[0], outs[1], atol=1e-5, rtol=1e-5)
    finally:
        sa.SEL.mode = saved


def test_sparse_modes_need_the_hip_library_on_cpu():
    """No CPU fallback: a sparse policy on CPU tensors fails loudly."""
    q = torch.zeros(1, 4, 128, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)

    class M:
        num_key_value_groups, layer_idx = 2, 0
    saved = (sa.SEL.mode, sa.SEL.kernel_v2)
    try:
        sa.SEL.mode, sa.SEL.kernel_v2 = "router", True
        with pytest.raises((AssertionError, RuntimeError)):
            sa.block_sparse_attention(M(), q, k, k, None, 0.125)
    finally:
        sa.SEL.mode, sa.SEL.kernel_v2 = saved


def test_rollout_peek_is_out_of_scope():
    """rollout_peek (an abandoned research mode of the reference, off its v2
    path) raises instead of running."""
    q = torch.zeros(1, 4, 128, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)

    class M:
        num_key_value_groups, layer_idx = 2, 0
    saved = (sa.SEL.mode, sa.SEL.kernel_v2)
    try:
        sa.SEL.mode, sa.SEL.kernel_v2 = "rollout_peek", False
        with pytest.raises(NotImplementedError, match="rollout_peek"):
            sa.block_sparse_attention(M(), q, k, k, None, 0.125)
    finally:
        sa.SEL.mode, sa.SEL.kernel_v2 = saved


@pytest.mark.parametrize("kernel_v2,mode", [(True, "router"), (True, "quest"),
                                            (False, "topk"), (False, "router")])
def test_sparse_paths_reject_query_shorter_than_keys(kernel_v2, mode):
    """A query shorter than the keys (prefill continuing a cache) would need
    shifted positions in the selector and the causal mask; like the
    reference's launchers (q.shape == k.shape), the sparse paths refuse it
    before touching any device."""
    q = torch.zeros(1, 4, 64, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)

    class M:
        num_key_value_groups, layer_idx = 2, 0
    saved = (sa.SEL.mode, sa.SEL.kernel_v2)
    try:
        sa.SEL.mode, sa.SEL.kernel_v2 = mode, kernel_v2
        with pytest.raises(AssertionError, match="query length"):
            sa.block_sparse_attention(M(), q, k, k, None, 0.125)
    finally:
        sa.SEL.mode, sa.SEL.kernel_v2 = saved


def test_launchers_reject_query_shorter_than_keys():
    import block_attn
    q = torch.zeros(1, 4, 64, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="query length"):
        block_attn.block_sparse_attn_v2(q, k, k, torch.zeros(1, 4, 1, 2, dtype=torch.int32), 0.125)
    with pytest.raises(AssertionError, match="query length"):
        block_attn.block_sparse_attn(q, k, k, torch.ones(1, 4, 64, 2, dtype=torch.bool), 0.125)
    with pytest.raises(AssertionError, match="query length"):
        sa.select_v2(q, k, 0.125)


def test_v1_router_log_line_format(capsys):
    """The v1 router's per-layer diagnostics go into SEL's three lists, and the
    last prefill layer prints their running means on the line the reference's
    harness logs carry (src/sparse_attention.py:355-375)."""
    from types import SimpleNamespace

    class Model:
        model = SimpleNamespace(layers=[None, None])
    saved = dict(vars(sa.SEL))
    try:
        sa.SEL.__init__()
        sa.SEL.log, sa.SEL.model_ref = True, Model()
        sa.SEL.router_mode, sa.SEL.router_grain, sa.SEL.router_quantile = "quantile", "row", 0.4
        keep = torch.zeros(1, 2, 4, 8, dtype=torch.bool)
        keep[..., :3] = True                                   # 3 blocks per cell
        unc = torch.tensor([[[1, 0, 0, 0], [1, 1, 0, 0]]], dtype=torch.uint8)
        res = SimpleNamespace(uncertain=unc, margin=torch.full((1, 2, 4), 0.25))
        sa._log_router_layer(res, keep, 4, 0)                 # not the last layer: no line
        assert capsys.readouterr().out == ""
        keep[..., :5] = True                                   # 5 blocks per cell
        res2 = SimpleNamespace(uncertain=torch.zeros_like(unc), margin=torch.full((1, 2, 4), 0.5))
        sa._log_router_layer(res2, keep, 4, 1)
        assert sa.SEL.router_trigger_rate == [0.375, 0.0]
        assert sa.SEL.router_eff_budget == [3.0, 5.0]
        assert sa.SEL.router_margin_mean == [0.25, 0.5]
        assert capsys.readouterr().out == \
            "  router[quantile/row]: trigger=0.188 eff_budget=4.0 margin=0.375 q=0.40\n"
        sa.SEL.router_mode, sa.SEL.router_tau = "abs", 0.1
        sa._log_router_layer(res2, keep, 1, 1)                 # decode (one query row): no line
        assert capsys.readouterr().out == ""
        sa._log_router_layer(res2, keep, 4, 1)
        assert capsys.readouterr().out.endswith(" tau=0.100\n")
    finally:
        sa.SEL.__dict__.update(saved)


def test_reference_attn_returns_the_inputs_dtype():
    """reference_attn returns SDPA in the inputs' dtype, as the reference
    (src/triton_block_attn.py:301-312); reference_attn_fp32 keeps fp32."""
    from block_attn import reference_attn, reference_attn_fp32
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 2, 130, 64, generator=g).to(torch.bfloat16) for _ in range(3))
    keep = torch.ones(1, 2, 130, 3, dtype=torch.bool)
    keep[:, :, 70:, 0] = False
    o = reference_attn(q, k, v, keep, 0.125)
    o32 = reference_attn_fp32(q, k, v, keep, 0.125)
    assert o.dtype == torch.bfloat16 and o32.dtype == torch.float32
    assert torch.equal(o, o32.to(torch.bfloat16))
    # the causal mask and the keep mask: row 0 sees only key 0
    assert torch.allclose(o32[:, :, 0], v[:, :, 0].float())


def test_install_rollout_hooks_sets_model_ref_and_stashes_prefill_inputs():
    """install_rollout_hooks (src/sparse_attention.py:189-205), which the
    reference's harnesses call after loading the model: SEL.model_ref is the
    model and each decoder layer's prefill input lands in SEL.hidden_at;
    a one-token step leaves the stash alone."""
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config
    cfg = Qwen2Config(vocab_size=256, hidden_size=64, intermediate_size=128,
                      num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=512)
    saved = dict(vars(sa.SEL))
    try:
        sa.SEL.__init__()
        sa.SEL.mode = "dense"
        torch.manual_seed(0)
        model = AutoModelForCausalLM.from_config(cfg, attn_implementation="block_sparse").eval()
        sa.install_rollout_hooks(model)
        assert sa.SEL.model_ref is model and sa.SEL.hidden_at == {}
        ids = torch.randint(0, 256, (2, 70), generator=torch.Generator().manual_seed(1))
        with torch.no_grad():
            model(ids)
        assert sorted(sa.SEL.hidden_at) == [0, 1, 2]
        assert all(h.shape == (2, 70, 64) and not h.requires_grad for h in sa.SEL.hidden_at.values())
        first = sa.SEL.hidden_at[0]
        with torch.no_grad():
            model(ids[:, :1])                       # one query row: not a prefill
        assert sa.SEL.hidden_at[0] is first
    finally:
        sa.SEL.__dict__.update(saved)
