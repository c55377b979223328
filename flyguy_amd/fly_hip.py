"""One hop as an autograd Function on the MI355X library: the HopCuda interface of flyguy/fly_cuda.py:61-115.

z[target, b] = sum over connections (source -> target) of w * h[source, b]; states are [neurons, batch] with the
batch contiguous and a multiple of 32.  crow / col: the connections by target (CSR, int64 / int32); tcrow / tcol /
tperm: the same by source.  The backward is one pass over the transposed form that gives both the state gradient
and the per-connection gradient (fh_spmm_bwd).  In float32 the products gather from copies of h (forward) and of the
output gradient (backward) in the tiled layout [B/32][rows][32] (fh_to_tiled, fh_spmm_tiled, fh_spmm_bwd_tiled).

half=True reads the states as IEEE binary16 (rounded to nearest even) and the backward reads the output gradient as
binary16 after dividing it by its largest magnitude (fly_cuda.py:93, 100-114); all sums stay float32.  The
conversions and the scale are computed by the library (fh_to_half, fh_absmax).
"""
from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from ._lib import NO_ROW, call, lib, plan_rows

# Row plans per structure.  An entry holds the index tensors themselves: while they are cached their memory cannot be
# handed to other tensors, so the key (addresses, lengths, versions) cannot come to name different contents.
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


def _key(t: torch.Tensor | None):
    return None if t is None else (t.data_ptr(), t.numel(), t.device, t._version)


def _plan(rowptr: torch.Tensor, col: torch.Tensor, idx: torch.Tensor | None, n_edges: int):
    """The device plan of a product: its row plan, and per plan position the source row (col[edge]) and the weight
    index (idx[edge], or the edge itself)."""
    key = (_key(rowptr), _key(col), _key(idx))
    hit = _plans.get(key)
    if hit is not None and hit[0] is rowptr and hit[1] is col and hit[2] is idx:
        _plans.move_to_end(key)
        return hit[3]
    rp = rowptr.detach().cpu().numpy()
    if rp[0] != 0 or rp[-1] != n_edges or (len(rp) > 1 and (rp[1:] < rp[:-1]).any()):
        raise ValueError("HopHip: row pointer does not describe the connection arrays it came with")
    p = plan_rows(rp)
    pos = p["pos"].astype(np.int64)
    used = pos >= 0
    c = col.detach().cpu().numpy()
    pcol = np.full(len(pos), NO_ROW, np.int32)
    pcol[used] = c[pos[used]]
    pidx = np.full(len(pos), -1, np.int32)
    pidx[used] = (idx.detach().cpu().numpy()[pos[used]] if idx is not None else pos[used])
    dev = rowptr.device

    def put(a, width=None):
        a = a if len(a) else np.zeros((1,) + ((width,) if width else ()), np.int32)
        return torch.as_tensor(np.ascontiguousarray(a), device=dev)
    d = {"wave": put(p["wave"], 2), "seg": put(p["seg"], 4), "split": put(p["split"], 4), "pcol": put(pcol),
         "pidx": put(pidx), "nwave": len(p["wave"]), "nseg": len(p["seg"]), "nsplit": len(p["split"]),
         "nslot": p["nslot"], "npos": len(pos)}
    _remember(_plans, key, (rowptr, col, idx, d))
    return d


def _args(d):
    return (d["wave"].data_ptr(), d["nwave"], d["seg"].data_ptr(), d["nseg"], d["split"].data_ptr(), d["nsplit"],
            d["nslot"], d["pcol"].data_ptr(), d["pidx"].data_ptr(), d["npos"])


def _check_index(idx: torch.Tensor, bound: int, what: str) -> None:
    """Every entry of idx in [0, bound), checked once per tensor (the kernels gather through it)."""
    key = (idx.data_ptr(), idx.numel(), idx.device, idx._version, bound)
    hit = _checked.get(key)
    if hit is not None and hit is idx:
        return
    if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= bound):
        raise ValueError(f"HopHip: {what} out of range")
    _remember(_checked, key, idx)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class HopHip(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w, h, crow, col, tcrow, tcol, tperm, half: bool):
        n_rows, B = crow.numel() - 1, h.shape[1]
        if B % 32 or not h.is_contiguous() or h.dtype != torch.float32:
            raise ValueError("HopHip: h must be contiguous float32 [n_src, B] with B a multiple of 32")
        w = w.contiguous().float()
        col = col.contiguous()
        E, n_src = col.numel(), h.shape[0]
        if w.numel() != E or col.dtype != torch.int32 or crow.dtype != torch.int64:
            raise ValueError("HopHip: w / col / crow do not match (float32 w[E], int32 col[E], int64 crow)")
        _check_index(col, n_src, "source index")
        d = _plan(crow, col, None, E)
        out = torch.empty(n_rows, B, device=h.device)
        cw = torch.empty(max(d["npos"], 1), 2, dtype=torch.int32, device=h.device)
        if half:
            t64 = (B + 63) // 64
            hs = torch.empty(max(t64 * n_src * 64, 1), dtype=torch.float16, device=h.device)
            call("fh_to_half", h.data_ptr(), n_src, B, None, hs.data_ptr(), _stream(h))
            scratch = torch.empty(max(d["nslot"] * t64 * 64, 1), device=h.device)
            call("fh_spmm_h", *_args(d), w.data_ptr(), hs.data_ptr(), out.data_ptr(), n_rows, n_src, B, cw.data_ptr(),
                 scratch.data_ptr(), _stream(h))
            ctx.hs = hs
        else:
            # the product gathers from a tiled copy of h: half the time of gathers from the row-major h
            ht = torch.empty(max(n_src * B, 1), device=h.device)
            call("fh_to_tiled", h.data_ptr(), n_src, B, ht.data_ptr(), _stream(h))
            scratch = torch.empty(max(d["nslot"] * B, 1), device=h.device)
            call("fh_spmm_tiled", *_args(d), w.data_ptr(), ht.data_ptr(), out.data_ptr(), n_rows, n_src, B,
                 cw.data_ptr(), scratch.data_ptr(), _stream(h))
            ctx.hs = None
        ctx.save_for_backward(w, h, tcrow, tcol, tperm)
        ctx.n_rows, ctx.half = n_rows, half
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
        _check_index(tcol, ctx.n_rows, "target index")
        _check_index(tperm, E, "transposed order")
        d = _plan(tcrow, tcol, tperm, E)
        gh = torch.empty(n_src, B, device=h.device)
        gw = torch.zeros_like(w) if ctx.needs_input_grad[0] else None
        cw = torch.empty(max(d["npos"], 1), 2, dtype=torch.int32, device=h.device)
        if ctx.half:
            t64 = (B + 63) // 64
            scale = torch.empty(1, device=h.device)
            call("fh_absmax", gz.data_ptr(), gz.numel(), scale.data_ptr(), _stream(gz))
            gzs = torch.empty(max(t64 * ctx.n_rows * 64, 1), dtype=torch.float16, device=h.device)
            call("fh_to_half", gz.data_ptr(), ctx.n_rows, B, scale.data_ptr(), gzs.data_ptr(), _stream(gz))
            gwpart = torch.empty(max(d["npos"] * t64, 1), device=h.device) if gw is not None else None
            scratch = torch.empty(max(d["nslot"] * t64 * 64, 1), device=h.device)
            call("fh_spmm_bwd_h", *_args(d), w.data_ptr(), gzs.data_ptr(), ctx.hs.data_ptr(), scale.data_ptr(),
                 gh.data_ptr(), gw.data_ptr() if gw is not None else None, ctx.n_rows, n_src, B, cw.data_ptr(),
                 gwpart.data_ptr() if gwpart is not None else None, scratch.data_ptr(), _stream(gz))
        else:
            gzt = torch.empty(max(ctx.n_rows * B, 1), device=h.device)       # gathered tiled, as in the forward
            call("fh_to_tiled", gz.data_ptr(), ctx.n_rows, B, gzt.data_ptr(), _stream(gz))
            gwpart = torch.empty(max(d["npos"] * (B // 32), 1), device=h.device) if gw is not None else None
            scratch = torch.empty(max(d["nslot"] * B, 1), device=h.device)
            call("fh_spmm_bwd_tiled", *_args(d), w.data_ptr(), gzt.data_ptr(), h.data_ptr(), gh.data_ptr(),
                 gw.data_ptr() if gw is not None else None, ctx.n_rows, n_src, B, cw.data_ptr(),
                 gwpart.data_ptr() if gwpart is not None else None, scratch.data_ptr(), _stream(gz))
        return gw, (gh if ctx.needs_input_grad[1] else None), None, None, None, None, None, None


class FireHip(torch.autograd.Function):
    """h = relu(g z - t) per row of row-major [rows, B] float32 states on the library (fh_fire, fh_fire_bwd): the
    neuron activation of FlyActor's GPU path (fly.py:296-304) in one pass each way instead of PyTorch's three.  g, t:
    per row (the gain and softplus(theta) of the row's neuron).  h and the state gradient are PyTorch's bit for bit;
    the per-row gradients of g and t are the same sums in another order."""

    @staticmethod
    def forward(ctx, z, g, t):
        rows, B = z.shape
        if z.dtype != torch.float32 or not z.is_cuda or B % 4:
            raise ValueError("FireHip: z must be float32 [rows, B] on the GPU with B a multiple of 4")
        z = z.contiguous()
        g = g.detach().float().contiguous()
        t = t.detach().float().contiguous()
        if g.shape != (rows,) or t.shape != (rows,):
            raise ValueError("FireHip: g and t must hold one value per row")
        h = torch.empty_like(z)
        call("fh_fire", z.data_ptr(), g.data_ptr(), t.data_ptr(), rows, B, h.data_ptr(), _stream(z))
        ctx.save_for_backward(z, g, t)
        return h

    @staticmethod
    def backward(ctx, gh):
        z, g, t = ctx.saved_tensors
        rows, B = z.shape
        gh = gh.contiguous().float()
        gz, gg, gt = torch.empty_like(z), torch.empty_like(g), torch.empty_like(t)
        call("fh_fire_bwd", gh.data_ptr(), z.data_ptr(), g.data_ptr(), t.data_ptr(), rows, B, gz.data_ptr(),
             gg.data_ptr(), gt.data_ptr(), _stream(gh))
        return gz, gg, gt

