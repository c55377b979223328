"""Shared fixtures: toy networks from the golden fixtures, the GPU marker, library/oracle builds."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def toy(name: str) -> dict:
    z = np.load(GOLDEN / f"toy_{name}.npz", allow_pickle=False)
    return {k: z[k] for k in z.files}


def golden(name: str, hops: int, fan: int) -> dict:
    z = np.load(GOLDEN / f"idx_{name}_h{hops}_f{fan}.npz", allow_pickle=False)
    return {k: z[k] for k in z.files}


CASES = [("a", 2, 5), ("a", 3, 5), ("a", 4, 5), ("a", 3, 16), ("b", 3, 16), ("b", 2, 8), ("c", 3, 16), ("c", 4, 6)]


def lively(f, seed: int = 0):
    """Weights that make every layer fire (as the reference's test does, tests/test_fly.py:52-53)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        f.w.mul_(8.0)
        f.out.weight.normal_(0, 0.3, generator=g)
        f.theta.fill_(-2.0)
        f.gain.mul_(1 + 0.2 * torch.rand(f.gain.shape, generator=g))
        f.in_b.normal_(0, 0.1, generator=g)
        f.out.bias.normal_(0, 0.1, generator=g)
    return f


@pytest.fixture(scope="session")
def gpu_lib():
    """The HIP library on the GPU (fails loudly if it is not built)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from flyguy_amd._lib import lib
    return lib()
