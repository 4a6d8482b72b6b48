"""The mean-plane checker of the GPU tests (tests/parity.py::check_mean_planes)
on summaries encoded on the CPU in the documented format — [B, Hk, NB, 2, D]
fp16 hi / lo of each block's fp32 mean times 2^e (max |mean| 2^e in
[2^14, 2^15)), then [B, Hk, NB] fp32 2^-e — and on encodings with one
planted mistake each, which it must reject."""

import numpy as np
import pytest
import torch

from parity import check_mean_planes


def encode(k, e_off=0, drop_lo=False, scale_mul=1.0):
    """Mean summary of k [B, Hk, N, D] as one flat int16 tensor."""
    B, Hk, N, D = k.shape
    nb = (N + 63) // 64
    kp = np.zeros((B, Hk, nb * 64, D), np.float32)
    kp[:, :, :N] = k.float().numpy()
    mean = kp.reshape(B, Hk, nb, 64, D).sum(axis=3, dtype=np.float32) * np.float32(1 / 64)
    mx = np.abs(mean).max(axis=-1)
    ef = (mx.view(np.int32) >> 23).astype(np.int64)
    e = np.where(mx == 0, 0, 141 - ef + e_off)
    x = np.ldexp(mean, e[..., None]).astype(np.float32)
    hi = x.astype(np.float16)
    lo = (x - hi.astype(np.float32)).astype(np.float16)
    if drop_lo:
        lo[:] = 0
    sc = (np.ldexp(np.float32(1), -e) * scale_mul).astype(np.float32)
    planes = np.stack([hi, lo], axis=3).reshape(-1).view(np.int16)
    return torch.from_numpy(np.concatenate([planes, sc.reshape(-1).view(np.int16)]))


@pytest.fixture(scope="module")
def keys():
    g = torch.Generator().manual_seed(11)
    k = torch.randn(1, 2, 700, 64, generator=g)
    k *= torch.pow(2.0, torch.randint(-12, 13, (1, 2, 11, 1), generator=g).float()
                   ).repeat_interleave(64, 2)[:, :, :700]
    k[0, 1, 64:128] = 0
    return k.to(torch.bfloat16)


def test_checker_accepts_the_format(keys):
    rec = check_mean_planes(encode(keys), keys)
    assert rec.shape == (1, 2, 11, 64)


@pytest.mark.parametrize("mistake", [dict(e_off=1), dict(e_off=-1), dict(drop_lo=True),
                                     dict(scale_mul=2.0)],
                         ids=["exponent+1", "exponent-1", "lo dropped", "scale doubled"])
def test_checker_rejects_a_planted_mistake(keys, mistake):
    with pytest.raises(AssertionError):
        check_mean_planes(encode(keys, **mistake), keys)
