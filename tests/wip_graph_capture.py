"""ugbsa_select_mask_static under HIP graph capture: one warm-up call (its
first call on the device looks the scratch address up), then one call
captured in a torch CUDA graph on a side stream and replayed several times,
with eager work and synchronisations between the replays; every replay's keep
mask and margins must equal the direct call's bit for bit."""

import numpy as np
import pytest
import torch

import _capi
import sparse_attention as sa
import synth

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("policy", ["topk", "router"])
def test_static_scratch_under_graph_capture(hip_lib, policy):
    print(f"[case] select_mask_static graph capture {policy}", flush=True)
    lib = _capi.lib()
    q, k, _ = synth.make_layer(synth.CONFIGS["c1"], 5, S=1500, dtype=torch.bfloat16)
    q, k = q.to(DEV), k.to(DEV)
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    nb = (N + 63) // 64
    mode = _capi.MODE_QUEST
    planes = sa.block_summary(k, mode)
    keep = torch.zeros(B, H, M, nb, dtype=torch.uint8, device=DEV)
    margin = torch.zeros(B, H, M, dtype=torch.float32, device=DEV)
    k_eff = 2 if policy == "router" else 0
    side = torch.cuda.Stream(DEV)

    def call(stream):
        rc = lib.ugbsa_select_mask_static(
            q.data_ptr(), *q.stride(), planes.data_ptr(), B, H, Hk, M, N, D, _capi.DTYPE_BF16,
            mode, D ** -0.5, _capi.V1_TOPK, 3, k_eff, 1, 112, 0.9, None, keep.data_ptr(),
            margin.data_ptr() if k_eff else None, stream.cuda_stream)
        _capi.check(rc, "select_mask_static")

    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):
        call(side)                                   # warm-up: scratch address looked up
    torch.cuda.synchronize()
    keep_ref, margin_ref = keep.cpu().numpy().copy(), margin.cpu().numpy().copy()
    assert keep_ref.sum(-1).min() >= 1
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        call(side)
    for rep in range(3):
        keep.fill_(7)                                # eager work between the replays
        margin.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(keep.cpu().numpy(), keep_ref), rep
        if k_eff:
            assert np.array_equal(margin.cpu().numpy().view(np.uint32), margin_ref.view(np.uint32)), rep
