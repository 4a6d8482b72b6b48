"""The v2 hot path under HIP graph capture: kernel 1 (block summaries),
kernel 2 (selection), the router and kernel 3 (attention, with its tile
schedule and, past 512 key blocks, its generation launches) for one layer,
captured in a torch CUDA graph on a side stream after one direct call.  Every
replay, with eager work and synchronisations between the replays, equals the
direct call bit for bit (selection and attention are deterministic: no atomics
in any accumulation).  The path allocates nothing through HIP, synchronises
nowhere and clears no memory with a memset, so a serving loop can capture it."""

import pytest
import torch

import sparse_attention as sa
import synth
from block_attn import block_sparse_attn_v2

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def layer(q, k, v, cfg, sel):
    res = sa.select_v2(q, k, cfg.scaling, sel=sel)
    out = block_sparse_attn_v2(q, k, v, res.kv_idx, cfg.scaling)
    return res, out


# (config, tokens): c1 at 2048 tokens (32 key blocks, one attention launch,
# router-on-Quest, head_dim 128); c2's heads at 34000 tokens (532 blocks: the
# attention runs in generations); c5's at 34000 (head_dim 256 with QK-Norm,
# router-on-K-mean, generations with per-XCD tile runs)
@pytest.mark.parametrize("name,S", [("c1", 2048), ("c2", 34000), ("c5", 34000)])
def test_v2_layer_replays_like_the_direct_call(hip_lib, name, S):
    print(f"[case] graph capture {name} S={S}", flush=True)
    cfg = synth.CONFIGS[name]
    q, k, v = synth.make_layer_fast(cfg, 7, device=DEV, dtype=torch.bfloat16, S=S)
    sel = sa.Selector()
    for f, val in cfg.sel_fields().items():
        setattr(sel, f, val)
    sel.kernel_v2 = True
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        res0, out0 = layer(q, k, v, cfg, sel)        # the direct call
    torch.cuda.synchronize()
    kv_ref, out_ref = res0.kv_idx.clone(), out0.clone()
    assert (kv_ref[..., 0] == 0).all()               # the sink leads every tile's list
    assert torch.isfinite(out_ref.float()).all()
    if res0.uncertain is not None:
        unc_ref = res0.uncertain.clone()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        res, out = layer(q, k, v, cfg, sel)
    for rep in range(3):
        out.fill_(float("nan"))                      # eager work between the replays
        res.kv_idx.fill_(-7)
        other = layer(q[:, :, :1024], k[:, :, :1024], v[:, :, :1024], cfg, sel)[1]
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(res.kv_idx, kv_ref), f"{name} replay {rep}: kv_idx"
        assert torch.equal(out.view(torch.int16), out_ref.view(torch.int16)), \
            f"{name} replay {rep}: attention output"
        if res0.uncertain is not None:
            assert torch.equal(res.uncertain, unc_ref), f"{name} replay {rep}: router"
        del other
