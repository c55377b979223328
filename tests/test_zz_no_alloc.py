"""fh_spmm_static, the allocation-free variant of fh_spmm (its workspace is a static device array): bit-identical
to fh_spmm on two calls in a row, the second smaller than the first; a product too large for the workspace is
refused before any device work; after one warm-up call (which looks up the workspace's address) a call leaves the
device's free memory unchanged, and the call captured in a HIP graph (PyTorch's CUDAGraph) replays bit-identically
to eager fh_spmm, with new inputs, eager work and synchronisations between the replays."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from flyguy_amd._lib import LibraryError, call
from flyguy_amd.fly_hip import _args, _plan
from flyguy_amd.synth import scaled_3hop
from gpu_helpers import say

pytestmark = pytest.mark.gpu


def _hop(div: int, k: int):
    """Hop k of the 3-hop shape at 1/div size as device tensors: (CSR row pointer int64, columns int32, weights)."""
    s, params = scaled_3hop(div)
    h = s["hop"][k]
    crow = torch.as_tensor(np.asarray(h["crow"], np.int64)).cuda()
    col = torch.as_tensor(np.asarray(h["col"], np.int32)).cuda()
    w = torch.as_tensor(params[0][np.asarray(h["widx"])]).cuda()
    return crow, col, w, s["sizes"][k], s["sizes"][k + 1]


def _both(crow, col, w, n_src, n_rows, B, seed):
    d = _plan(crow, col, None, int(col.numel()))
    h = torch.randn(n_src, B, generator=torch.Generator().manual_seed(seed)).cuda()
    st = torch.cuda.current_stream().cuda_stream
    want = torch.empty(n_rows, B, device="cuda")
    cw = torch.empty(max(d["npos"], 1), 2, dtype=torch.int32, device="cuda")
    part = torch.empty(max(d["nslot"] * B, 1), device="cuda")
    call("fh_spmm", *_args(d), w.data_ptr(), h.data_ptr(), want.data_ptr(), n_rows, n_src, B, cw.data_ptr(),
         part.data_ptr(), st)
    got = torch.full((n_rows, B), float("nan"), device="cuda")
    call("fh_spmm_static", *_args(d), w.data_ptr(), h.data_ptr(), got.data_ptr(), n_rows, n_src, B, st)
    torch.cuda.synchronize()
    return d, got, want


def test_static_workspace_matches_fh_spmm(gpu_lib):
    # first call: a hop of the 1/16 shape, whose heavy rows are split (partial sums in the workspace)
    crow, col, w, n_src, n_rows = _hop(16, 1)
    say(f"fh_spmm_static: hop 2 at 1/16 ({int(col.numel())} connections), B 256")
    d, got, want = _both(crow, col, w, n_src, n_rows, 256, 1)
    assert d["nsplit"] > 0
    assert torch.equal(got, want)
    # second call right after: a smaller product (1/64 shape, B 64) that leaves the first call's contents behind
    crow, col, w, n_src, n_rows = _hop(64, 2)
    say(f"fh_spmm_static: hop 3 at 1/64 ({int(col.numel())} connections), B 64")
    d, got, want = _both(crow, col, w, n_src, n_rows, 64, 2)
    assert torch.equal(got, want)


def test_static_workspace_refuses_a_larger_product(gpu_lib):
    crow, col, w, n_src, n_rows = _hop(16, 1)
    d = _plan(crow, col, None, int(col.numel()))
    B = 4096 * 32                       # nslot * B * 4 bytes of partial sums: more than the workspace holds
    assert d["nslot"] * B * 4 > 32 << 20
    dummy = torch.empty(1, device="cuda")
    with pytest.raises(LibraryError, match="static workspace"):
        call("fh_spmm_static", *_args(d), w.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), n_rows, n_src, B,
             torch.cuda.current_stream().cuda_stream)


def test_static_workspace_allocates_nothing_and_replays_in_a_graph(gpu_lib):
    crow, col, w, n_src, n_rows = _hop(16, 1)
    B = 128
    d = _plan(crow, col, None, int(col.numel()))
    assert d["nsplit"] > 0                                         # (split rows: partial sums in the workspace)
    h = torch.empty(n_src, B, device="cuda")
    out = torch.empty(n_rows, B, device="cuda")

    def static_call():
        call("fh_spmm_static", *_args(d), w.data_ptr(), h.data_ptr(), out.data_ptr(), n_rows, n_src, B,
             torch.cuda.current_stream().cuda_stream)

    def eager_reference():
        want = torch.empty(n_rows, B, device="cuda")
        cw = torch.empty(max(d["npos"], 1), 2, dtype=torch.int32, device="cuda")
        part = torch.empty(max(d["nslot"] * B, 1), device="cuda")
        call("fh_spmm", *_args(d), w.data_ptr(), h.data_ptr(), want.data_ptr(), n_rows, n_src, B, cw.data_ptr(),
             part.data_ptr(), torch.cuda.current_stream().cuda_stream)
        return want

    gen = torch.Generator(device="cuda").manual_seed(3)
    h.copy_(torch.randn(n_src, B, device="cuda", generator=gen))
    say("fh_spmm_static: warm-up call, then free device memory across a call")
    static_call()                                                  # (looks up the workspace's address)
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    static_call()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free_before
    assert torch.equal(out, eager_reference())
    say("fh_spmm_static: captured in a graph, three replays")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_call()
    for i in range(3):
        h.copy_(torch.randn(n_src, B, device="cuda", generator=gen))
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = eager_reference()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
