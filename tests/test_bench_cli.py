"""bench.py's command-line contract on the CPU: one GPU only (the path would
shard by KV-head group; no figure at several GPUs is measured), and the c4
policy switch names the reference's four backbone / router combinations."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_policies_cover_both_backbones_with_and_without_the_router():
    sys.path.insert(0, ROOT)
    import bench
    assert set(bench.POLICIES) == {"topk_mean", "quest", "router_mean", "router_quest"}
    assert bench.POLICIES["router_mean"] == dict(mode="router", router_score="mean")
    import sparse_attention as sa
    names = set()
    for fields in bench.POLICIES.values():
        sel = sa.Selector()
        for f, v in fields.items():
            setattr(sel, f, v)
        names.add((bench.policy_name(sel), sa.use_quest(sel)))
    assert names == {("topk (K-mean)", False), ("quest", True), ("router-on-mean", False),
                     ("router-on-quest", True)}
