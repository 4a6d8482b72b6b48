"""Pins the attention oracle: three formulations agree, case A equals plain causal
attention computed independently in fp64, slot order does not matter."""

import numpy as np

from oracle import attention as A


def rand_qkv(rng, B, H, Hk, M, N, D):
    q = rng.standard_normal((B, H, M, D)).astype(np.float32)
    k = rng.standard_normal((B, Hk, N, D)).astype(np.float32)
    v = rng.standard_normal((B, Hk, N, D)).astype(np.float32)
    return q, k, v


def random_kv_idx(rng, B, H, qt, nb, slots):
    """Random per-tile block sets with sink + self forced, sentinels, invisible ids."""
    kv = np.full((B, H, qt, slots), nb, np.int32)
    for b in range(B):
        for h in range(H):
            for t in range(qt):
                self_blk = min(t, nb - 1)
                pool = [x for x in range(nb) if x not in (0, self_blk)]
                pick = rng.choice(pool, size=min(len(pool), slots - 2), replace=False)
                row = [0, self_blk] + [int(x) for x in pick]
                row = row[:slots]
                rng.shuffle(row)
                kv[b, h, t, :len(row)] = row
    return kv


def test_case_a_dense_equals_causal():
    rng = np.random.default_rng(0)
    q, k, v = rand_qkv(rng, 1, 4, 2, 256, 256, 32)
    kv = np.broadcast_to(np.arange(4, dtype=np.int32), (1, 4, 4, 4)).copy()
    ref = A.causal_attention(q, k, v, 32 ** -0.5)
    np.testing.assert_allclose(A.gathered_attention(q, k, v, kv, 32 ** -0.5), ref, atol=2e-6)
    np.testing.assert_allclose(A.masked_tile_attention(q, k, v, kv, 32 ** -0.5), ref, atol=2e-6)


def test_formulations_agree_sparse_ragged():
    rng = np.random.default_rng(1)
    M = N = 64 * 6 + 17                       # ragged last tile / block
    q, k, v = rand_qkv(rng, 1, 4, 1, M, N, 16)
    nb = qt = 7
    kv = random_kv_idx(rng, 1, 4, qt, nb, 5)
    sc = 0.25
    g = A.gathered_attention(q, k, v, kv, sc)
    m = A.masked_tile_attention(q, k, v, kv, sc)
    np.testing.assert_allclose(g, m, atol=2e-6)
    # per-row keep form of reference_attn with the tile's set on every row
    keep_t = A.tile_keep(kv, nb)
    keep = np.repeat(keep_t, 64, axis=2)[:, :, :M]
    np.testing.assert_allclose(A.keep_attention(q, k, v, keep, sc), m, atol=2e-6)


def test_slot_order_invariance_and_skips():
    rng = np.random.default_rng(2)
    q, k, v = rand_qkv(rng, 1, 2, 2, 320, 320, 16)
    kv = random_kv_idx(rng, 1, 2, 5, 5, 4)
    base = A.gathered_attention(q, k, v, kv, 0.3)
    perm = kv[..., ::-1].copy()
    np.testing.assert_allclose(A.gathered_attention(q, k, v, perm, 0.3), base, atol=2e-6)
    # invisible ids (blk > t) and sentinels are skipped like the kernel does
    noisy = np.concatenate([kv, np.full(kv.shape[:-1] + (2,), 4, np.int32),
                            np.full(kv.shape[:-1] + (1,), 5, np.int32)], axis=-1)
    noisy[..., -3] = 4   # block 4 is invisible to tiles 0..3 and already present for t=4? keep both
    g2 = A.gathered_attention(q, k, v, noisy, 0.3)
    # tiles 0..3 unchanged; tile 4 may count block 4 twice if it was already there
    np.testing.assert_allclose(g2[:, :, :256], base[:, :, :256], atol=2e-6)


def test_compute_kv_idx_bruteforce():
    rng = np.random.default_rng(3)
    keep = rng.random((1, 2, 130, 5)) < 0.3
    kv, mk = A.compute_kv_idx(keep, 64)
    assert kv.shape == (1, 2, 3, mk)
    for h in range(2):
        for t in range(3):
            rows = keep[0, h, t * 64:(t + 1) * 64]
            want = sorted(np.nonzero(rows.any(0))[0].tolist())
            got = [x for x in kv[0, h, t].tolist() if x < 5]
            assert got == want
            assert all(x == 5 for x in kv[0, h, t].tolist()[len(want):])
    kv0, mk0 = A.compute_kv_idx(np.zeros((1, 1, 64, 3), bool), 64)
    assert mk0 == 1 and kv0.tolist() == [[[[3]]]]


def load_attention_golden():
    """Cases written by tests/golden/make_golden_attn.py from the reference's
    own reference_attn (src/triton_block_attn.py:301-312, CPU fp32)."""
    import os
    from conftest import GOLDEN, bf16_bits_to_f32
    z = np.load(os.path.join(GOLDEN, "attention_reference.npz"))
    cases = {}
    for key in z.files:
        name, field = key.split("/", 1)
        cases.setdefault(name, {})[field] = z[key]
    for c in cases.values():
        for t in ("q", "k", "v"):
            c[t] = bf16_bits_to_f32(c.pop(f"{t}_bf16"))
    return cases


def test_oracle_matches_reference_attn_golden():
    """Both oracle formulations reproduce the reference's SDPA-with-mask output
    on its own fixtures (dense, GQA + ragged tail, batch 2 at head_dim 256)."""
    cases = load_attention_golden()
    assert sorted(cases) == ["dense_d64", "gqa_ragged_d128", "multi_d256"]
    for name, c in cases.items():
        sc = float(c["scale"])
        g = A.gathered_attention(c["q"], c["k"], c["v"], c["kv_idx"], sc)
        m = A.masked_tile_attention(c["q"], c["k"], c["v"], c["kv_idx"], sc)
        np.testing.assert_allclose(g, c["out"], atol=2e-6, err_msg=name)
        np.testing.assert_allclose(m, c["out"], atol=2e-6, err_msg=name)
        # a planted error would show: dropping the last listed block of one tile
        kv = c["kv_idx"].copy()
        nb = (c["k"].shape[2] + 63) // 64
        row = kv[0, 0, -1]
        row[np.flatnonzero(row < nb)[-1]] = nb                       # the sentinel: skipped
        assert np.abs(A.gathered_attention(c["q"], c["k"], c["v"], kv, sc) - c["out"]).max() > 1e-3
