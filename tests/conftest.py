import ast
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "uncertainty-gated-block-sparse-attention_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> exact fp32 values."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def load_golden(name: str):
    """Golden selector vectors: (inputs dict, {policy: record dict})."""
    z = np.load(os.path.join(GOLDEN, f"selector_{name}.npz"))
    inputs, pols = {}, {}
    for key in z.files:
        if "/" in key:
            pol, field = key.split("/", 1)
            pols.setdefault(pol, {})[field] = z[key]
        else:
            inputs[key] = z[key]
    for rec in pols.values():
        if "fields" in rec:
            rec["fields"] = dict(ast.literal_eval(str(rec["fields"])))
    if "q_bf16" in inputs:
        inputs["q"] = bf16_bits_to_f32(inputs["q_bf16"])
        inputs["k"] = bf16_bits_to_f32(inputs["k_bf16"])
    return inputs, pols


@pytest.fixture(scope="session")
def hip_lib():
    """The built C-ABI library (skips CPU-only runs that have no GPU)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import _capi
    return _capi.lib()
