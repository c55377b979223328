"""One hop as an autograd Function on the MI355X library: the HopCuda interface of flyguy/fly_cuda.py:61-115.

z[target, b] = sum over connections (source -> target) of w * h[source, b]; states are [neurons, batch] with the
batch contiguous and a multiple of 32.  crow / col: the connections by target (CSR, int64 / int32); tcrow / tcol /
tperm: the same by source.  The backward is one pass over the transposed form that gives both the state gradient
and the per-connection gradient (fh_spmm_bwd).
"""
from __future__ import annotations

from collections import OrderedDict

import torch

from ._lib import call, lib, plan_segments

# Row plans per structure tensor.  An entry holds the tensor itself: while it is cached its memory cannot be handed
# to another tensor, so the key (address, length, version) cannot come to name different contents.
_plans: OrderedDict = OrderedDict()
_checked: OrderedDict = OrderedDict()
_CACHE = 64


def available() -> bool:
    """True when a GPU is present and the library loads (a missing library on a GPU is an error, not False)."""
    if not torch.cuda.is_available():
        return False
    lib()
    return True


def _remember(cache: OrderedDict, key, value):
    cache[key] = value
    cache.move_to_end(key)
    while len(cache) > _CACHE:
        cache.popitem(last=False)


def _plan(rowptr: torch.Tensor, n_edges: int):
    key = (rowptr.data_ptr(), rowptr.numel(), rowptr.device, rowptr._version)
    hit = _plans.get(key)
    if hit is not None and hit[0] is rowptr:
        _plans.move_to_end(key)
        return hit[1]
    rp = rowptr.detach().cpu().numpy()
    if rp[0] != 0 or rp[-1] != n_edges or (len(rp) > 1 and (rp[1:] < rp[:-1]).any()):
        raise ValueError("HopHip: row pointer does not describe the connection arrays it came with")
    seg, split, nslot = plan_segments(rp)
    dev = rowptr.device
    p = (torch.as_tensor(seg, device=dev).contiguous(), torch.as_tensor(split, device=dev).contiguous(), len(seg),
         len(split), nslot)
    _remember(_plans, key, (rowptr, p))
    return p


def _check_index(idx: torch.Tensor, bound: int, what: str) -> None:
    """Every entry of idx in [0, bound), checked once per tensor (the kernels gather through it)."""
    key = (idx.data_ptr(), idx.numel(), idx.device, idx._version, bound)
    hit = _checked.get(key)
    if hit is not None and hit is idx:
        return
    if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= bound):
        raise ValueError(f"HopHip: {what} out of range")
    _remember(_checked, key, idx)


class HopHip(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w, h, crow, col, tcrow, tcol, tperm, half: bool):
        if half:
            raise NotImplementedError("16-bit hop states are not available in this library yet")
        n_rows, B = crow.numel() - 1, h.shape[1]
        if B % 32 or not h.is_contiguous() or h.dtype != torch.float32:
            raise ValueError("HopHip: h must be contiguous float32 [n_src, B] with B a multiple of 32")
        w = w.contiguous().float()
        col = col.contiguous()
        E = col.numel()
        if w.numel() != E or col.dtype != torch.int32 or crow.dtype != torch.int64:
            raise ValueError("HopHip: w / col / crow do not match (float32 w[E], int32 col[E], int64 crow)")
        seg, split, nseg, nsplit, nslot = _plan(crow, E)
        _check_index(col, h.shape[0], "source index")
        out = torch.empty(n_rows, B, device=h.device)
        cw = torch.empty(max(E, 1), 2, dtype=torch.int32, device=h.device)
        scratch = torch.empty(max(nslot * B, 1), device=h.device)
        call("fh_spmm", crow.data_ptr(), col.data_ptr(), w.data_ptr(), h.data_ptr(), out.data_ptr(), n_rows, h.shape[0],
             B, E, seg.data_ptr(), nseg, split.data_ptr(), nsplit, nslot, cw.data_ptr(), scratch.data_ptr(),
             torch.cuda.current_stream(h.device).cuda_stream)
        ctx.save_for_backward(w, h, tcrow, tcol, tperm)
        ctx.n_rows = n_rows
        return out

    @staticmethod
    def backward(ctx, gz):
        w, h, tcrow, tcol, tperm = ctx.saved_tensors
        gz = gz.contiguous().float()
        n_src, B = h.shape
        tcol, tperm = tcol.contiguous(), tperm.contiguous()
        E = tcol.numel()
        if tperm.numel() != E or w.numel() != E or tcol.dtype != torch.int32 or tperm.dtype != torch.int64:
            raise ValueError("HopHip: tcol / tperm / w do not match")
        seg, split, nseg, nsplit, nslot = _plan(tcrow, E)
        _check_index(tcol, ctx.n_rows, "target index")
        _check_index(tperm, E, "transposed order")
        gh = torch.empty(n_src, B, device=h.device)
        gw = torch.zeros_like(w) if ctx.needs_input_grad[0] else None
        cw = torch.empty(max(E, 1), 2, dtype=torch.int32, device=h.device)
        gwpart = torch.empty(max(E * (B // 32), 1), device=h.device) if gw is not None else None
        scratch = torch.empty(max(nslot * B, 1), device=h.device)
        call("fh_spmm_bwd", tcrow.data_ptr(), tcol.data_ptr(), tperm.data_ptr(), w.data_ptr(),
             gz.data_ptr(), h.data_ptr(), gh.data_ptr(), gw.data_ptr() if gw is not None else None, ctx.n_rows, n_src, B,
             E, seg.data_ptr(), nseg, split.data_ptr(), nsplit, nslot, cw.data_ptr(),
             gwpart.data_ptr() if gwpart is not None else None, scratch.data_ptr(),
             torch.cuda.current_stream(h.device).cuda_stream)
        return gw, (gh if ctx.needs_input_grad[1] else None), None, None, None, None, None, None
