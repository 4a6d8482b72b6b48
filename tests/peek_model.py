"""Seeded tiny Qwen2 model and planner inputs for the rollout_peek tests.

Shared by ``tests/golden/make_golden_peek.py`` (which runs the reference's
planner on them) and the tests (which run this build's planner), so both see
the same weights and tensors.  Every value is drawn from a seeded CPU
``torch.Generator`` and rounded to bf16, so the fp32 and bf16 runs share
their inputs exactly.
"""

from __future__ import annotations

import torch

S = 768                 # 12 key blocks of 64
N_LAYERS = 3
HQ, HKV, HEAD_DIM, D_MODEL = 4, 2, 64, 256   # head_dim 64: the HIP kernels take 64 / 128 / 256


def tiny_qwen2(seed: int = 7, dtype=torch.float32, attn: str = "sdpa"):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    cfg = Qwen2Config(vocab_size=64, hidden_size=D_MODEL, intermediate_size=256,
                      num_hidden_layers=N_LAYERS, num_attention_heads=HQ,
                      num_key_value_heads=HKV, max_position_embeddings=2048,
                      attn_implementation=attn)
    model = Qwen2ForCausalLM(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for _, p in sorted(model.named_parameters()):
            p.copy_((0.08 * torch.randn(p.shape, generator=g)).to(torch.bfloat16).float())
    return model.to(dtype).eval()


def planner_inputs(seed: int, layer: int, with_next_pool: bool):
    """(query [1, HQ, S, hd], key / value [1, HKV, S, hd], hidden [1, S, d_model],
    next-layer key pool [1, HQ, S/64, hd] or None), bf16-valued fp32."""
    g = torch.Generator().manual_seed(1000 + 10 * seed + layer)

    def draw(*shape, scale=1.0):
        return (scale * torch.randn(*shape, generator=g)).to(torch.bfloat16).float()

    q = draw(1, HQ, S, HEAD_DIM)
    k = draw(1, HKV, S, HEAD_DIM)
    v = draw(1, HKV, S, HEAD_DIM)
    hidden = draw(1, S, D_MODEL, scale=0.5)
    pool = draw(1, HQ, S // 64, HEAD_DIM) if with_next_pool else None
    return q, k, v, hidden, pool


def position_embeddings(model, dtype=torch.float32, device="cpu"):
    x = torch.zeros(1, S, D_MODEL, dtype=dtype, device=device)
    pos = torch.arange(S, device=device)[None]
    return model.model.rotary_emb(x, pos)


# (name, seed, layer, metric, next pool given, extra Selector fields)
CASES = [
    ("peak", 1, 0, "peakedness", False, {}),
    ("xh", 2, 0, "cross_head_agreement", True, {}),
    ("resnorm", 3, 1, "residual_norm", True, {}),
    ("last_layer", 4, 2, "peakedness", False, {}),
    ("w1_rows6", 5, 1, "peakedness", True, {"peek_swap_w": 1, "peek_rows_per_layer": 6}),
    ("out_of_range", 6, 1, "peakedness", True, {"peek_layer_max": 0}),
]
SEL_FIELDS = dict(budget_blocks=3, k_min=1, k_max=112, peek_swap_w=2, peek_rows_per_layer=4,
                  peek_layer_min=0, peek_layer_max=999, peek_xh_threshold=0.5)
