"""HopHip (the HopCuda boundary, fh_spmm / fh_spmm_bwd and their binary16 forms) on random sparse products:
row and source counts from 1 to 3,000, in-degrees from a lognormal (heavy rows split over several waves, empty rows,
sources no row reads), batches of 32 to 256.  Output, source gradient and per-connection gradient against the
product in float64, relative to the largest entry <= 1e-5; the binary16 variant against the reference's half
arithmetic restated in float64 (tests/test_gpu_train.py)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import rel, say
from test_gpu_train import _half_case

pytestmark = pytest.mark.gpu


def random_product(seed: int):
    rng = np.random.default_rng(seed)
    n_rows, n_src = int(rng.integers(1, 3000)), int(rng.integers(1, 3000))
    deg = np.minimum(rng.lognormal(rng.uniform(0.5, 3.0), rng.uniform(0.5, 1.6), n_rows).astype(np.int64), n_src)
    deg[rng.random(n_rows) < 0.05] = 0                          # some rows read nothing
    crow = np.concatenate([[0], np.cumsum(deg)]).astype(np.int64)
    col = np.concatenate([np.sort(rng.choice(n_src, d, replace=False)) for d in deg]).astype(np.int32) \
        if deg.sum() else np.zeros(0, np.int32)
    E = len(col)
    r = np.repeat(np.arange(n_rows), deg)
    tperm = np.lexsort((r, col)).astype(np.int64)               # connections by source, then row
    tcrow = np.concatenate([[0], np.cumsum(np.bincount(col, minlength=n_src))]).astype(np.int64)
    tcol = r[tperm].astype(np.int32)
    w = rng.standard_normal(E)
    B = int(rng.choice([32, 64, 96, 160, 256]))
    return n_rows, n_src, B, crow, col, r, tcrow, tcol, tperm, w, rng


@pytest.mark.parametrize("seed", range(12))
def test_random_product_against_float64(gpu_lib, seed):
    from flyguy_amd.fly_hip import HopHip
    n_rows, n_src, B, crow, col, r, tcrow, tcol, tperm, w, rng = random_product(seed)
    say(f"random product {seed}: {n_rows} rows x {n_src} sources, {len(col)} connections (longest row "
        f"{int(np.diff(crow).max()) if n_rows else 0}), B {B}")
    a = torch.sparse_csr_tensor(torch.as_tensor(crow), torch.as_tensor(col.astype(np.int64)),
                                torch.as_tensor(w.astype(np.float32).astype(np.float64)), size=(n_rows, n_src))
    h = torch.as_tensor(rng.random((n_src, B)))
    gz = torch.as_tensor(rng.standard_normal((n_rows, B)))
    hf, gzf = h.float(), gz.float()
    want = (a @ hf.double()).numpy()
    want_gh = (a.t() @ gzf.double()).numpy()
    want_gw = (gzf.double()[torch.as_tensor(r)] * hf.double()[torch.as_tensor(col.astype(np.int64))]).sum(1).numpy()
    wd = torch.as_tensor(w.astype(np.float32)).cuda().requires_grad_(True)
    hd = hf.cuda().requires_grad_(True)
    out = HopHip.apply(wd, hd, torch.as_tensor(crow).cuda(), torch.as_tensor(col).cuda(), torch.as_tensor(tcrow).cuda(),
                       torch.as_tensor(tcol).cuda(), torch.as_tensor(tperm).cuda(), False)
    out.backward(gzf.cuda())
    torch.cuda.synchronize()
    for name, got, ref in (("out", out, want), ("gh", hd.grad, want_gh), ("gw", wd.grad, want_gw)):
        g = got.detach().cpu().numpy()
        assert g.shape == ref.shape and np.isfinite(g).all(), name
        if ref.size and np.abs(ref).max() > 0:
            assert rel(g, ref) <= 1e-5, (name, rel(g, ref))
        else:
            assert not np.abs(g).any(), name


@pytest.mark.parametrize("seed", range(12, 18))
def test_random_product_half(gpu_lib, seed):
    n_rows, n_src, B, crow, col, r, tcrow, tcol, tperm, w, rng = random_product(seed)
    if len(col) == 0:
        pytest.skip("a product without connections has no half-precision case")
    say(f"random product {seed} (binary16): {n_rows} rows x {n_src} sources, {len(col)} connections, B {B}")
    w32 = torch.as_tensor(w.astype(np.float32))
    a = torch.sparse_csr_tensor(torch.as_tensor(crow), torch.as_tensor(col.astype(np.int64)), w32.double(),
                                size=(n_rows, n_src))
    _half_case(a, torch.as_tensor(r), torch.as_tensor(col.astype(np.int64)), w32, n_src, n_rows, B,
               torch.as_tensor(crow), torch.as_tensor(col), torch.as_tensor(tcrow), torch.as_tensor(tcol),
               torch.as_tensor(tperm), seed)
