"""The score-dump hook's session mechanics without a GPU
(src/dump_block_scores.py:57-101): install rebinds the selector name the
dispatcher looks up, the selection passes through untouched, a recording
failure is reported and never raised, teardown restores the selector and
writes the recorded shards as one pickled list."""

import pickle

import numpy as np
import torch

import dump_block_scores as dbs
import sparse_attention as sa


def test_hook_passes_selection_through_and_survives_record_failures(capsys):
    orig = sa._block_select_kv_idx_v2
    calls = []

    def fake_selector(q, k, scaling, block_m=64):
        calls.append(scaling)
        return "kv_idx"

    sa._block_select_kv_idx_v2 = fake_selector
    try:
        dbs.install_dump_hook("/nonexistent/never_written.pkl")
        assert sa._block_select_kv_idx_v2 is not fake_selector
        dbs.install_dump_hook("/other.pkl")                 # a second install is a no-op
        hooked = sa._block_select_kv_idx_v2
        q = torch.zeros(1, 2, 128, 64)                      # CPU tensors: record() refuses them
        assert hooked(q, q, 0.5) == "kv_idx" and hooked(q, q, 0.25) == "kv_idx"
        assert calls == [0.5, 0.25]
        out = capsys.readouterr().out
        assert "not installing another" in out and out.count("no shard") == 2
        dbs.flush_and_teardown()                            # nothing recorded: no file
        assert sa._block_select_kv_idx_v2 is fake_selector
        assert hooked(q, q, 1.0) == "kv_idx"                # a stale recorder only forwards
        assert "no shard" not in capsys.readouterr().out
        dbs.flush_and_teardown()                            # no session: no-op
    finally:
        sa._block_select_kv_idx_v2 = orig


def test_hook_writes_recorded_shards_in_call_order(tmp_path, monkeypatch):
    orig = sa._block_select_kv_idx_v2
    seen = iter([None, {"g": np.zeros((1, 2, 3), np.float32)}, {"g": np.ones((1, 2, 3), np.float32)}])
    monkeypatch.setattr(dbs, "record", lambda *a, **k: next(seen))
    sa._block_select_kv_idx_v2 = lambda q, k, s, block_m=64: "kv"
    path = tmp_path / "shards.pkl"
    try:
        dbs.install_dump_hook(str(path))
        for _ in range(3):
            assert sa._block_select_kv_idx_v2(None, None, 0.1) == "kv"
        dbs.flush_and_teardown()
    finally:
        sa._block_select_kv_idx_v2 = orig
    with open(path, "rb") as f:                             # written by this test just above
        shards = pickle.load(f)
    # the first call recorded nothing; call_idx counts every selection call
    assert [s["call_idx"] for s in shards] == [1, 2]
    assert shards[1]["g"].sum() == 6


def test_mode_ids():
    sel = sa.Selector()
    expect = {("topk", "mean"): 0, ("router", "mean"): 1, ("router", "quest"): 2,
              ("quest", "mean"): 3, ("quest", "quest"): 3, ("topk", "quest"): 0,
              ("belief", "mean"): 4, ("dense", "quest"): 4}
    for (mode, score), code in expect.items():
        sel.mode, sel.router_score = mode, score
        assert dbs._mode_id(sel) == code, (mode, score)
