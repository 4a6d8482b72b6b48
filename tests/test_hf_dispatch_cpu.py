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


def test_install_rollout_hooks_captures_prefill_inputs():
    """src/sparse_attention.py:188-205: every decoder layer's prefill input is
    kept in SEL.hidden_at (decode steps are not), and SEL.model_ref is set."""
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config
    cfg = Qwen2Config(vocab_size=64, hidden_size=64, intermediate_size=96,
                      num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=512)
    saved = dict(sa.SEL.__dict__)
    try:
        sa.SEL.mode = "dense"
        torch.manual_seed(0)
        model = AutoModelForCausalLM.from_config(cfg, attn_implementation="block_sparse").eval()
        sa.install_rollout_hooks(model)
        assert sa.SEL.model_ref is model and sa.SEL.hidden_at == {}
        ids = torch.randint(0, 64, (1, 40), generator=torch.Generator().manual_seed(1))
        with torch.no_grad():
            model(ids)
        assert sorted(sa.SEL.hidden_at) == [0, 1, 2]
        assert all(h.shape == (1, 40, 64) for h in sa.SEL.hidden_at.values())
        first = sa.SEL.hidden_at[0].clone()
        with torch.no_grad():
            emb = model.model.embed_tokens(ids)
        assert torch.equal(first, emb)                 # layer 0's input is the embedding
        with torch.no_grad():
            model(ids[:, :1])                          # a one-token step is not kept
        assert torch.equal(sa.SEL.hidden_at[0], first)
    finally:
        sa.SEL.__dict__.clear()
        sa.SEL.__dict__.update(saved)


def test_rollout_peek_needs_the_hip_library_on_cpu():
    """rollout_peek takes its baseline from the HIP v1 selector: no CPU path."""
    q = torch.zeros(1, 4, 128, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 2, 128, 64, dtype=torch.bfloat16)

    class M:
        num_key_value_groups, layer_idx = 2, 0
    saved = (sa.SEL.mode, sa.SEL.kernel_v2)
    try:
        sa.SEL.mode, sa.SEL.kernel_v2 = "rollout_peek", False
        with pytest.raises((AssertionError, RuntimeError)):
            sa.block_sparse_attention(M(), q, k, k, None, 0.125)
    finally:
        sa.SEL.mode, sa.SEL.kernel_v2 = saved
