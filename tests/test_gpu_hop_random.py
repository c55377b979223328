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


@pytest.mark.parametrize("seed", range(18, 24))
def test_row_major_and_tiled_entry_points_agree(gpu_lib, seed):
    """fh_spmm / fh_spmm_bwd on row-major states and fh_spmm_tiled / fh_spmm_bwd_tiled on fh_to_tiled copies sum the
    same terms in the same order: identical outputs and gradients.  fh_to_tiled against torch's own reshape."""
    from flyguy_amd._lib import call
    from flyguy_amd.fly_hip import _args, _plan
    n_rows, n_src, B, crow, col, r, tcrow, tcol, tperm, w, rng = random_product(seed)
    say(f"row-major vs tiled {seed}: {n_rows} rows x {n_src} sources, {len(col)} connections, B {B}")
    dev, st = "cuda", torch.cuda.current_stream().cuda_stream
    E, T = len(col), B // 32
    wd = torch.zeros(max(E, 1), device=dev)                     # a real address also without connections
    wd[:E] = torch.as_tensor(w.astype(np.float32)).to(dev)
    h = torch.as_tensor(rng.random((n_src, B), np.float32)).to(dev)
    gz = torch.as_tensor(rng.standard_normal((n_rows, B), np.float32)).to(dev)

    def tiled(x):
        out = torch.full((x.shape[0] * B,), float("nan"), device=dev)
        call("fh_to_tiled", x.data_ptr(), x.shape[0], B, out.data_ptr(), st)
        return out

    ht, gzt = tiled(h), tiled(gz)
    assert torch.equal(ht.view(T, n_src, 32), h.view(n_src, T, 32).transpose(0, 1))
    assert torch.equal(gzt.view(T, n_rows, 32), gz.view(n_rows, T, 32).transpose(0, 1))

    d = _plan(torch.as_tensor(crow).to(dev), torch.as_tensor(col).to(dev), None, E)
    cw = torch.empty(max(d["npos"], 1), 2, dtype=torch.int32, device=dev)
    part = torch.empty(max(d["nslot"] * B, 1), device=dev)
    outs = []
    for name, src in (("fh_spmm", h), ("fh_spmm_tiled", ht)):
        out = torch.full((n_rows, B), float("nan"), device=dev)
        call(name, *_args(d), wd.data_ptr(), src.data_ptr(), out.data_ptr(), n_rows, n_src, B, cw.data_ptr(),
             part.data_ptr(), st)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])

    d = _plan(torch.as_tensor(tcrow).to(dev), torch.as_tensor(tcol).to(dev), torch.as_tensor(tperm).to(dev), E)
    cw = torch.empty(max(d["npos"], 1), 2, dtype=torch.int32, device=dev)
    part = torch.empty(max(d["nslot"] * B, 1), device=dev)
    gwpart = torch.empty(max(d["npos"] * T, 1), device=dev)
    grads = []
    for name, g in (("fh_spmm_bwd", gz), ("fh_spmm_bwd_tiled", gzt)):
        gh = torch.full((n_src, B), float("nan"), device=dev)
        gw = torch.zeros(max(E, 1), device=dev)
        call(name, *_args(d), wd.data_ptr(), g.data_ptr(), h.data_ptr(), gh.data_ptr(), gw.data_ptr(), n_rows, n_src,
             B, cw.data_ptr(), gwpart.data_ptr(), part.data_ptr(), st)
        grads.append((gh, gw))
    torch.cuda.synchronize()
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    assert not torch.isnan(outs[0]).any() and not torch.isnan(grads[0][0]).any()
