"""ugbsa_select_mask_static — the v1 per-row selector with its row-score
passes in the library's static device scratch instead of a caller workspace
(for callers that cannot allocate).  Through the C ABI, its keep mask and
margins must equal ugbsa_select_mask's with a torch workspace bit for bit, on
two calls in a row, the second with a smaller input (the scratch keeps the
first call's scores).  Under HIP graph capture (one warm-up call looks the
scratch address up, then one call is captured in a torch CUDA graph on a side
stream) every replay, with eager work and synchronisations between replays,
equals the direct call bit for bit."""

import numpy as np
import pytest
import torch

import _capi
import sparse_attention as sa
import synth

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def run_select_mask(q, k, policy, static):
    """keep [B, H, M, NB] uint8 and margin [B, H, M] (router) from one entry point."""
    lib = _capi.lib()
    B, H, M, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    nb = (N + 63) // 64
    mode = _capi.MODE_QUEST
    planes = sa.block_summary(k, mode)
    keep = torch.empty(B, H, M, nb, dtype=torch.uint8, device=DEV)
    margin = torch.empty(B, H, M, dtype=torch.float32, device=DEV)
    k_bud, k_eff = 3, (2 if policy == "router" else 0)
    belief = _capi.V1_BELIEF if policy == "belief" else _capi.V1_TOPK
    args = (q.data_ptr(), *q.stride(), planes.data_ptr(), B, H, Hk, M, N, D, _capi.DTYPE_BF16,
            mode, D ** -0.5, belief, k_bud, k_eff, 1, 112, 0.9, None)
    stream = _capi.stream_ptr(DEV)
    if static:
        rc = lib.ugbsa_select_mask_static(*args, keep.data_ptr(),
                                          margin.data_ptr() if k_eff else None, stream)
    else:
        # a workspace of two tiles' rows: several passes, as the static path
        # takes for shapes whose full row-score buffer would not fit
        ws = torch.empty(B * H * 64 * nb * 2, dtype=torch.float32, device=DEV)
        rc = lib.ugbsa_select_mask(*args, ws.data_ptr(), ws.numel(), keep.data_ptr(),
                                   margin.data_ptr() if k_eff else None, stream)
    _capi.check(rc, "select_mask" + ("_static" if static else ""))
    torch.cuda.synchronize()
    return keep.cpu().numpy(), (margin.cpu().numpy() if k_eff else None)


@pytest.mark.parametrize("policy", ["topk", "belief", "router"])
def test_static_scratch_matches_workspace_path(hip_lib, policy):
    cfg = synth.CONFIGS["c1"]
    for S, seed in ((2000, 1), (777, 2)):          # the second call is smaller
        print(f"[case] select_mask_static {policy} S={S}", flush=True)
        q, k, _ = synth.make_layer(cfg, seed, S=S, dtype=torch.bfloat16)
        q, k = q.to(DEV), k.to(DEV)
        keep_s, margin_s = run_select_mask(q, k, policy, static=True)
        keep_w, margin_w = run_select_mask(q, k, policy, static=False)
        assert np.array_equal(keep_s, keep_w)
        assert keep_s.sum(-1).min() >= 1
        if margin_w is not None:
            assert np.array_equal(margin_s.view(np.uint32), margin_w.view(np.uint32))


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
