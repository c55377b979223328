"""ctypes binding of the MI355X library (flyguy_amd/libflyguy_core.so, include/flyguy_core.h).

Loading never falls back: if the library is missing or a call fails, an exception says why.  The library
records errors per thread (fc_last_error); every wrapper call here checks it.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libflyguy_core.so"
_lib = None

vp, ci, cll, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_float
_SIGS = {
    "fc_create": (vp, [ctypes.c_char_p, ci]),
    "fc_create_from_memory": (vp, [ctypes.c_char_p, cll, ci]),
    "fc_create_ex": (vp, [ctypes.c_char_p, cll, ci, ci]),
    "fc_free": (None, [vp]),
    "fc_set_stream": (None, [vp, vp]),
    "fc_sizes": (None, [vp, ctypes.POINTER(cll)]),
    "fc_copy": (None, [vp, ci, ci, ctypes.POINTER(vp)]),
    "fc_forward": (None, [vp, vp, ci, vp, ci]),
    "fc_zero_grad": (None, [vp]),
    "fc_backward": (None, [vp, vp, ci]),
    "fc_grad_norm": (cf, [vp]),
    "fc_step": (cf, [vp, cf, cf, cf, cf, cf]),
    "fc_adam_t": (cll, [vp, cll]),
    "fc_sync": (None, [vp]),
    "fc_last_error": (ctypes.c_char_p, []),
    "fc_clear_error": (None, []),
    "fc_kl_loss": (None, [vp, vp, vp, ci, cf, vp, vp]),
    "fc_teach_step": (cf, [vp, vp, vp, ci, cf, cf, cf, cf, cf, cf, vp]),
    "fc_export_state": (None, [vp, ci, ci, vp, ci]),
    "fc_profile": (None, [vp, ci]),
    "fc_profile_read": (ci, [vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(cll), ci, ci]),
    "fc_gather_ceiling": (ci, [ci, ci, vp, cll, ci, vp, ctypes.POINTER(ctypes.c_double)]),
    "fc_plan_rows": (ci, [vp, ci, ci, vp, cll, vp, cll, vp, cll, vp, cll, ctypes.POINTER(cll)]),
    "fc_net_plan": (ci, [ctypes.c_char_p, cll, ci, ci, vp, cll, vp, cll, vp, cll, vp, cll, ctypes.POINTER(cll)]),
    "fc_net_marks": (cll, [ctypes.c_char_p, cll, ci, ci, vp, cll]),
    "fh_spmm": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, ci, ci, ci, vp, vp, vp]),
    "fh_spmm_static": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, ci, ci, ci, vp]),
    "fh_spmm_bwd": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, vp, vp, ci, ci, ci, vp, vp, vp, vp]),
    "fh_to_half": (None, [vp, ci, ci, vp, vp, vp]),
    "fh_to_tiled": (None, [vp, ci, ci, vp, vp]),
    "fh_fire": (None, [vp, vp, vp, ci, ci, vp, vp]),
    "fh_fire_bwd": (None, [vp, vp, vp, vp, ci, ci, vp, vp, vp, vp]),
    "fh_spmm_tiled": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, ci, ci, ci, vp, vp, vp]),
    "fh_spmm_bwd_tiled": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, vp, vp, ci, ci, ci, vp, vp, vp,
                                 vp]),
    "fh_absmax": (None, [vp, cll, vp, vp]),
    "fh_spmm_h": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, ci, ci, ci, vp, vp, vp]),
    "fh_spmm_bwd_h": (None, [vp, ci, vp, ci, vp, ci, ci, vp, vp, cll, vp, vp, vp, vp, vp, vp, ci, ci, ci, vp, vp, vp,
                             vp]),
    # include/flyguy_train.h
    "ft_main": (ci, [ci, ctypes.POINTER(ctypes.c_char_p)]),
    "ft_draw": (ci, [ctypes.c_ulonglong, ctypes.POINTER(cll), ci, ci, ci, vp]),
    "ft_lr": (None, [cll, cf, cf, cf, cf, ctypes.c_double, ctypes.POINTER(cf)]),
    "ft_chunk_samples": (cll, [ctypes.c_char_p, ci, ci]),
    "ft_scan_order": (ci, [ctypes.c_char_p, ci, ctypes.c_char_p, ci]),
    "fd_gather16": (None, [vp, vp, vp, ci, vp, ci, ci, ci, vp, vp, vp]),
    "fd_unpack16": (None, [vp, ci, ci, ci, vp, vp, vp]),
    "fc_layers": (ci, [vp, ctypes.POINTER(ci), ci]),
    "fc_survey": (ci, [vp, vp, vp, ci, ci, cf, ci]),
    "fc_survey_read": (cll, [vp, vp, vp, ctypes.POINTER(ctypes.c_double)]),
    "fc_revive": (ci, [vp, vp, vp, ci, ci, cf, ctypes.c_ulonglong, cll, ctypes.c_char_p, ci]),
}


class LibraryError(RuntimeError):
    pass


def lib():
    """The loaded library (loaded once).  Raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LibraryError(f"{LIB_PATH} is not built (python -m flyguy_amd.build)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def check(what: str = "") -> None:
    """Raise the library's pending error, if any."""
    msg = lib().fc_last_error()
    if msg:
        lib().fc_clear_error()
        raise LibraryError(f"{what}: {msg.decode()}" if what else msg.decode())


def call(name: str, *args):
    out = getattr(lib(), name)(*args)
    check(name)
    return out


NO_ROW = 0x01FFFFFF      # the source index of a plan position no edge uses (gathers read zeros for it)


def seg_cap(n_edges: int) -> int:
    """The segment length cap the library uses for a product of n_edges edges: at least 4096 segments per tile
    (so that a tile's workgroups fill an XCD), between 16 and 512 edges."""
    return int(min(512, max(16, -(-int(n_edges) // 4096))))


def bwd_pairs(crow) -> bool:
    """Whether the library's backward of a layer with this CSR row pointer (gathered rows: the layer's own) takes two
    tiles per workgroup: when its 16384 most gathered rows take at least 3/4 of the gathers (core.hip:pair_tiles,
    without its FLYGUY_BWD_TILES override)."""
    import numpy as np
    deg = np.diff(np.asarray(crow, np.int64))
    E = int(deg.sum())
    if E <= 0:
        return False
    top = int(np.sort(deg)[::-1][:16384].sum())
    return 4 * top >= 3 * E


def plan_rows(rowptr, seg_max: int | None = None) -> dict:
    """Row plan of a CSR row pointer (host only, fc_plan_rows): {"wave": int32 [nwave, 2], "seg": int32 [nseg, 4],
    "split": int32 [nsplit, 4], "nslot": int, "pos": int32 [npos]} (pos: the CSR edge of each plan position, -1 none).
    seg_max defaults to seg_cap of the edge count."""
    import numpy as np
    rp = np.ascontiguousarray(rowptr, dtype=np.int32)
    rows = len(rp) - 1
    if seg_max is None:
        seg_max = seg_cap(int(rp[-1]) if rows >= 0 and len(rp) else 0)
    counts = (cll * 5)()
    lib().fc_plan_rows(rp.ctypes.data, rows, seg_max, None, 0, None, 0, None, 0, None, 0, counts)
    lib().fc_clear_error()
    nw, ns, nsp, nslot, npos = (int(counts[i]) for i in range(5))
    wave = np.zeros((max(nw, 1), 2), np.int32)
    seg = np.zeros((max(ns, 1), 4), np.int32)
    split = np.zeros((max(nsp, 1), 4), np.int32)
    pos = np.zeros(max(npos, 1), np.int32)
    rc = lib().fc_plan_rows(rp.ctypes.data, rows, seg_max, wave.ctypes.data, nw, seg.ctypes.data, ns,
                            split.ctypes.data, nsp, pos.ctypes.data, npos, counts)
    if rc != 0:
        check("fc_plan_rows")
        raise LibraryError("fc_plan_rows failed")
    return {"wave": wave[:nw], "seg": seg[:ns], "split": split[:nsp], "nslot": nslot, "pos": pos[:npos]}


def net_plan(net: bytes, product: int, backward: bool = False) -> dict:
    """The plan a handle of this network (NET.bin bytes) runs for one product (0 the plug, k hop k; backward: the
    hop's CSC rows), computed on the host by fc_net_plan; the same dict as plan_rows."""
    import numpy as np
    counts = (cll * 5)(-1, -1, -1, -1, -1)         # (written only once the network is read and planned)
    lib().fc_net_plan(net, len(net), product, int(backward), None, 0, None, 0, None, 0, None, 0, counts)
    if counts[0] < 0:
        check("fc_net_plan")
        raise LibraryError("fc_net_plan failed")
    lib().fc_clear_error()                         # (the capacity error of the sizing call)
    nw, ns, nsp, nslot, npos = (int(counts[i]) for i in range(5))
    wave = np.zeros((max(nw, 1), 2), np.int32)
    seg = np.zeros((max(ns, 1), 4), np.int32)
    split = np.zeros((max(nsp, 1), 4), np.int32)
    pos = np.zeros(max(npos, 1), np.int32)
    rc = lib().fc_net_plan(net, len(net), product, int(backward), wave.ctypes.data, nw, seg.ctypes.data, ns,
                           split.ctypes.data, nsp, pos.ctypes.data, npos, counts)
    if rc != 0:
        check("fc_net_plan")
        raise LibraryError("fc_net_plan failed")
    return {"wave": wave[:nw], "seg": seg[:ns], "split": split[:nsp], "nslot": nslot, "pos": pos[:npos]}


def net_marks(net: bytes, hop: int, which: int):
    """The backward's reduction table `which` of hop `hop` (fc_net_marks): 0 column neurons, 1 strength marks per
    backward position, 2 column marks, 3 the top layer's marks."""
    import numpy as np
    n = int(lib().fc_net_marks(net, len(net), hop, which, None, 0))
    if n < 0:
        check("fc_net_marks")
        raise LibraryError("fc_net_marks failed")
    out = np.zeros(max(n, 1), np.int32)
    if int(lib().fc_net_marks(net, len(net), hop, which, out.ctypes.data, n)) != n:
        check("fc_net_marks")
        raise LibraryError("fc_net_marks failed")
    return out[:n]


STAGES = {0: "obs transpose", 1: "pack", 2: "plug", 11: "logits", 12: "loss", 13: "readout bwd", 22: "reduce",
          23: "adam", 24: "zero"}
for _k in range(8):
    STAGES[3 + _k] = f"hop{_k + 1} fwd"
    STAGES[14 + _k] = f"hop{_k + 1} bwd"


def profile_read(core, reset: bool = True) -> dict:
    """{stage name: (total ms, timed runs)} of the stages that ran since the last reset."""
    ms = (ctypes.c_double * 25)()
    n = (cll * 25)()
    call("fc_profile_read", core, ms, n, 25, int(reset))
    return {STAGES[i]: (ms[i], int(n[i])) for i in range(25) if n[i] and i in STAGES}
