"""The C-ABI library loads on a machine without a GPU, exports every function include/*.h declares, and refuses
malformed network files before it touches the device."""
from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from conftest import ROOT, toy
from flyguy_amd._lib import LIB_PATH, lib
from flyguy_amd.export import net_bytes, structure
from flyguy_amd.fly import FlyActor


def test_cpu_decision_library_exports():
    """libfly_infer.so (no HIP) exports the functions include/fly_infer.h declares: fly_infer.cpp's six and
    fly_set_threads (an addition)."""
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "fly_infer.h").read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(fly_[a-z_]+)\s*\(", text)))
    assert names == ["fly_create", "fly_forward", "fly_free", "fly_set_hop", "fly_set_out", "fly_set_plug",
                     "fly_set_threads"]
    L = ctypes.CDLL(str(LIB_PATH.parent / "libfly_infer.so"))
    for n in names:
        assert hasattr(L, n), n


def declared() -> list[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(f[chtd]_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 30 and "fc_forward" in names and "fh_spmm_bwd" in names and "ft_main" in names
    L = ctypes.CDLL(str(LIB_PATH))
    for n in names:
        assert hasattr(L, n), n


def test_reference_entry_points_present():
    # the ten functions the reference's library exports (flyguy/native/flyguy_train.cu:569-629)
    for n in ("fc_create", "fc_sizes", "fc_copy", "fc_forward", "fc_zero_grad", "fc_backward", "fc_grad_norm",
              "fc_step", "fc_adam_t", "fc_sync"):
        assert n in declared()


def _bad(raw: bytes) -> str:
    L = lib()
    h = L.fc_create_from_memory(raw, len(raw), 64)
    assert not h
    msg = L.fc_last_error().decode()
    L.fc_clear_error()
    return msg


def test_malformed_networks_are_refused_on_the_host():
    torch = pytest.importorskip("torch")
    torch.manual_seed(0)
    f = FlyActor(toy("a"), 517, 90, hops=3, fan=5)
    s = structure(f)
    good = net_bytes(s)
    assert "FLY1" in _bad(b"NOPE" + good[4:])
    assert "short" in _bad(good[: len(good) // 2])
    # a connection whose source is outside the previous layer
    s2 = structure(f)
    s2["hop"][1]["col"] = np.array(s2["hop"][1]["col"]).copy()
    s2["hop"][1]["col"][0] = s["sizes"][1] + 5
    assert "hop 2" in _bad(net_bytes(s2))
    # a strength index used twice in one hop
    s3 = structure(f)
    w = np.array(s3["hop"][0]["widx"]).copy()
    w[1] = w[0]
    s3["hop"][0]["widx"] = w
    assert "hop 1" in _bad(net_bytes(s3))
    # a re-drive row outside the sensory layer
    s4 = structure(f)
    d = np.array(s4["hop"][0]["drow"]).copy()
    d[0] = s["n_s"] + 1
    s4["hop"][0]["drow"] = d
    assert "hop 1" in _bad(net_bytes(s4))
    # a by-source form that is not the transpose of the by-target form: two weight indices swapped (each still
    # distinct and in range), and two connections' target rows swapped
    s5 = structure(f)
    tw = np.array(s5["hop"][1]["twidx"]).copy()
    tw[[0, -1]] = tw[[-1, 0]]
    s5["hop"][1]["twidx"] = tw
    assert "not the transpose" in _bad(net_bytes(s5))
    s6 = structure(f)
    tc = np.array(s6["hop"][2]["tcol"]).copy()
    i = int(np.flatnonzero(tc != tc[0])[0])
    tc[[0, i]] = tc[[i, 0]]
    s6["hop"][2]["tcol"] = tc
    assert "not the transpose" in _bad(net_bytes(s6))


def test_hop_boundary_refuses_bad_arguments_on_the_host():
    """The HopCuda-boundary additions (tiled products, the fused activation) check their arguments before any
    device call: each refusal below names its entry point, on a machine without a GPU."""
    from flyguy_amd._lib import LibraryError, call
    x = ctypes.c_void_p(64)                                     # (never dereferenced: the checks fail first)
    with pytest.raises(LibraryError, match="fh_to_tiled"):
        call("fh_to_tiled", x, 4, 48, x, None)                  # B not a multiple of 32
    with pytest.raises(LibraryError, match="fh_fire"):
        call("fh_fire", x, x, None, 4, 32, x, None)             # no thresholds
    with pytest.raises(LibraryError, match="fh_fire"):
        call("fh_fire", x, x, x, 4, 30, x, None)                # B not a multiple of 4
    with pytest.raises(LibraryError, match="fh_fire_bwd"):
        call("fh_fire_bwd", x, x, x, x, 4, 32, x, None, x, None)   # no gain gradient
    plan = (x, 1, x, 9, None, 0, 0, x, x, 64)                   # 9 segments for 1 wave (at most 8)
    with pytest.raises(LibraryError, match="fh_spmm_tiled"):
        call("fh_spmm_tiled", *plan, x, x, x, 4, 4, 32, x, None, None)
    with pytest.raises(LibraryError, match="fh_spmm_bwd_tiled"):
        call("fh_spmm_bwd_tiled", *plan, x, x, x, x, None, 4, 4, 32, x, None, None, None)
