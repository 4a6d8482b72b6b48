"""GPU parity of the score-dump diagnostic (ugbsa_score_dump) against the
oracle (oracle/score_dump.py, src/dump_block_scores.py:104-207).

Bars:
* unforced tile scores vs the oracle's independent fp32 scores — max |dT| <= 1e-5,
  and bit-identical to the selector's own scores outside the forced entries;
* g, r, sigma, g_rho bit-identical to the oracle run on the kernel's own
  unforced scores (NaN where the oracle has NaN); valid exact;
* tau_hat within rtol 1e-4 of the oracle's float64 reduction;
* through the HF hook: the model's logits are unchanged by the dump, one
  shard per full-attention layer, in the reference's format.
"""

import pickle

import numpy as np
import pytest
import torch

import dump_block_scores as dbs
import sparse_attention as sa
import synth
from parity import summation_bound
from oracle import score_dump as OD
from oracle import selector as OS

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

POLICIES = {
    "topk": dict(mode="topk"),
    "quest": dict(mode="quest"),
    "router_quest": dict(mode="router", router_score="quest"),
    "router_mean": dict(mode="router", router_score="mean"),
}


def make_sel(**fields):
    s = sa.Selector()
    s.kernel_v2 = True
    for k, v in fields.items():
        setattr(s, k, v)
    return s


def same_or_both_nan(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    return a.shape == b.shape and bool(np.all(both_nan | (a.view(np.uint32) == b.view(np.uint32))))


def check_shard(shard, q, k, scaling, sel, heads=None, scores=True, score_tol=None):
    """Kernel shard vs oracle; ``heads`` limits the from-scratch oracle to a
    slice of query heads (with their KV head) to keep big configs fast;
    ``scores=False`` skips the from-scratch tile scores (long rows)."""
    T_k = shard["tile_score"].cpu().numpy()
    cfg = OS.SelectorConfig.from_selector(sel)
    nb = T_k.shape[-1]
    k_b, rho_k = OD.dump_budgets(sel.budget_blocks, nb)
    g, r, sg, grho = OD.order_stats(T_k, k_b, rho_k)
    for name, want in (("g", g), ("r", r), ("sigma", sg), ("g_rho", grho)):
        assert same_or_both_nan(shard[name], want), name
    qt = T_k.shape[2]
    assert np.array_equal(shard["valid"], OD.tile_n_visible(qt, k.shape[2]) > rho_k)
    H, Hk = q.shape[1], k.shape[1]
    hs = slice(None) if heads is None else heads
    qh = q[:, hs].float().cpu().numpy()
    kh = k.float().cpu().numpy() if heads is None else \
        k[:, hs.start // (H // Hk):hs.start // (H // Hk) + 1].float().cpu().numpy()
    if scores:
        T_or = OS.tile_scores(qh, kh, scaling, cfg.use_quest, force=False)
        fin = np.isfinite(T_or)
        assert np.array_equal(fin, np.isfinite(T_k[:, hs]))
        tol = 1e-5 if score_tol is None else score_tol(qh, kh)[fin]
        assert (np.abs(T_or[fin] - T_k[:, hs][fin]) <= tol).all()
    tau_or = OD.tau_hat(qh, kh, scaling, cfg.use_quest)
    np.testing.assert_allclose(shard["tau_hat"][:, hs], tau_or, rtol=1e-4)
    return T_k


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("policy", sorted(POLICIES))
def test_score_dump_vs_oracle(hip_lib, D, policy):
    print(f"[case] score_dump D={D} policy={policy}", flush=True)
    cfg = synth.CONFIGS["c1"]
    S = 2000 if D != 128 else 4096                       # ragged and aligned
    q, k, _ = synth.make_layer(cfg, 5, S=S, D=D, dtype=torch.bfloat16)
    sel = make_sel(budget_blocks=4, **POLICIES[policy])  # k_b 8, rho_k 16
    qd, kd = q.to(DEV), k.to(DEV)
    shard = dbs.record(qd, kd, D ** -0.5, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    assert shard["mode_id"] == OD.mode_id(OS.SelectorConfig.from_selector(sel))
    assert shard["n_blocks"] == (S + 63) // 64 and shard["budget_blocks"] == 4
    T_k = check_shard(shard, q, k, D ** -0.5, sel)
    # the dump ranks what the selector ranks, before its sink/self forcing
    res = sa.select_v2(qd, kd, D ** -0.5, sel=sel, want_tile_score=True)
    T_sel = res.tile_score.cpu().numpy()
    qt, nb = T_k.shape[2:]
    _, self_blk = OS.tile_visibility(qt, S, nb)
    keep = np.ones(T_k.shape, bool)
    keep[..., 0] = False
    keep[:, :, np.arange(qt), self_blk] = False
    assert np.array_equal(T_k[keep].view(np.uint32), T_sel[keep].view(np.uint32))
    v = shard["valid"]
    # on valid tiles the gaps are ordered: 0 <= g <= r, so sigma <= 1; g_rho >= 0
    g, r, gr = shard["g"][..., v], shard["r"][..., v], shard["g_rho"][..., v]
    assert (g >= 0).all() and (g <= r).all() and (gr >= 0).all()


@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("policy", ["quest", "router_mean"])
def test_score_dump_fp16(hip_lib, D, policy):
    """The dump on an fp16 layer: order statistics bit-identical to the oracle
    on the kernel's own scores; scores within the fp32 summation-order bound
    of fp16 products (tests/parity.py); tau_hat within rtol 1e-4."""
    print(f"[case] score_dump fp16 D={D} policy={policy}", flush=True)
    cfg = synth.CONFIGS["c1"]
    q, k, _ = synth.make_layer(cfg, 6, S=2000, D=D, dtype=torch.float16)
    sel = make_sel(budget_blocks=4, **POLICIES[policy])
    shard = dbs.record(q.to(DEV), k.to(DEV), D ** -0.5, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    quest = OS.SelectorConfig.from_selector(sel).use_quest
    check_shard(shard, q, k, D ** -0.5, sel,
                score_tol=lambda qh, kh: summation_bound(qh, kh, D ** -0.5, quest))


def test_score_dump_c2_full_config(hip_lib):
    """BASELINE configs[1] layer: S=32768, 28/4 heads, D=128, Quest backbone,
    budget 32 -> k_b 64, rho_k 128."""
    print("[case] score_dump c2 full", flush=True)
    cfg = synth.CONFIGS["c2"]
    q, k, _ = synth.make_layer(cfg, 0)
    sel = make_sel(**cfg.sel_fields())
    shard = dbs.record(q.to(DEV), k.to(DEV), cfg.scaling, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    assert shard["g"].shape == (1, 28, 512) and shard["tau_hat"].shape == (1, 28)
    assert shard["valid"].sum() == 512 - 128
    check_shard(shard, q, k, cfg.scaling, sel, heads=slice(0, 7))


def test_score_dump_streaming_rows(hip_lib):
    """Rows past 4096 blocks (the selector's streaming form) in dump mode."""
    print("[case] score_dump streaming rows", flush=True)
    S = 4097 * 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 2, S, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 1, S, 64, generator=g).to(torch.bfloat16)
    sel = make_sel(mode="router", router_score="quest", budget_blocks=32)
    shard = dbs.record(q.to(DEV), k.to(DEV), 0.125, sel=sel, want_tile_score=True)
    torch.cuda.synchronize()
    check_shard(shard, q, k, 0.125, sel, scores=False)


def test_score_dump_no_shard_cases(hip_lib):
    print("[case] score_dump early returns", flush=True)
    q, k, _ = synth.make_layer(synth.CONFIGS["c1"], 1, S=512, D=128, dtype=torch.bfloat16)
    qd, kd = q.to(DEV), k.to(DEV)
    for budget in (4, 2):          # k_b == NB, then rho_k == NB (no valid tile)
        assert dbs.record(qd, kd, 0.1, sel=make_sel(mode="quest", budget_blocks=budget)) is None
    shard = dbs.record(qd, kd, 0.1, sel=make_sel(mode="quest", budget_blocks=1))
    assert shard["valid"].tolist() == [False] * 4 + [True] * 4


def test_dump_hook_through_hf_model(hip_lib, tmp_path):
    """install_dump_hook / flush_and_teardown around a tiny Qwen2 prefill."""
    from transformers import AutoModelForCausalLM
    from transformers.models.qwen2 import Qwen2Config
    print("[case] score_dump hf hook", flush=True)
    saved = dict(vars(sa.SEL))
    try:
        sa.SEL.kernel_v2, sa.SEL.mode, sa.SEL.router_score = True, "router", "quest"
        sa.SEL.budget_blocks = 4
        torch.manual_seed(0)
        model = AutoModelForCausalLM.from_config(
            Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512,
                        num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                        max_position_embeddings=8192),
            attn_implementation="block_sparse").to(device=DEV, dtype=torch.bfloat16).eval()
        ids = torch.randint(0, 512, (1, 4096), generator=torch.Generator().manual_seed(1)).to(DEV)
        with torch.no_grad():
            plain = model(ids).logits
        orig = sa._block_select_kv_idx_v2
        path = tmp_path / "diag.pkl"
        dbs.install_dump_hook(str(path))
        assert sa._block_select_kv_idx_v2 is not orig
        with torch.no_grad():
            hooked = model(ids).logits
        dbs.flush_and_teardown()
        assert sa._block_select_kv_idx_v2 is orig
        assert torch.equal(plain, hooked)
        with open(path, "rb") as f:          # written by this process just above
            shards = pickle.load(f)
        assert [s["call_idx"] for s in shards] == [0, 1]
        for s in shards:
            assert set(s) == {"call_idx", "n_blocks", "mode_id", "budget_blocks", "g", "r",
                              "sigma", "g_rho", "valid", "tau_hat"}
            assert s["mode_id"] == 2 and s["n_blocks"] == 64 and s["budget_blocks"] == 4
            assert s["g"].shape == (1, 4, 64) and s["g"].dtype == np.float32
            assert s["valid"].dtype == bool and s["valid"].sum() == 64 - 16
            assert s["tau_hat"].shape == (1, 4) and (s["tau_hat"] > 0).all()
            assert (s["sigma"][..., s["valid"]] <= 1).all()
    finally:
        if dbs._session is not None:
            dbs.flush_and_teardown()
        sa.SEL.__dict__.update(saved)
        sa.SEL.reset_log()
