"""The network's structure and weights as flat binaries (the format of flyguy/native/export.py:9-15).

NET.bin (little endian, int32 unless noted): "FLY1", obs_dim, n_act, hops, n_neurons, n_w, n_s, fan, n_dn,
sizes[hops+1], E[hops]; plug: in_crow[n_s+1], in_col[E_in], in_tcrow[obs_dim+1], in_tcol[E_in], in_tperm[E_in];
n0[n_s]; per hop: nid[N_k], crow[N_k+1], col[E_k], widx[E_k], tcrow[N_{k-1}+1], tcol[E_k], twidx[E_k], drow[N_k];
dn_rows[n_dn]; wmap[n_w].  Only the n_w connections in play are library parameters ("strengths in play").
PARAMS.bin: "FLYP", step (int64), float32 W[n_w], gain, theta, in_w, in_b, out_w (row = action), out_b.

The library reads exactly this file (fc_create); structure() is computed from an actor's own buffers, so the
two cannot disagree (export.py:32-49).
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import torch

_HOP_KEYS = ("nid", "crow", "col", "widx", "tcrow", "tcol", "twidx", "drow")
_PLUG_KEYS = ("in_crow", "in_col", "in_tcrow", "in_tcol", "in_tperm", "n0")


def structure(f) -> dict:
    """The index arrays of the library from a FlyActor's buffers (export.py:32-49): the in-play connections
    `wmap` (sorted), each hop's connections as indices into them (`widx`, and `twidx` in CSC order), and the
    sensory row that keeps driving a hop row (`drow`, -1 for none)."""
    K = f.hops
    used = torch.unique(torch.cat([getattr(f, f"e{k}") for k in range(1, K + 1)])).cpu().numpy()
    compact = np.full(f.n_conn, -1, np.int64)
    compact[used] = np.arange(len(used))
    s = {"obs_dim": f.obs_dim, "n_act": f.out.out_features, "hops": K, "n_neurons": f.n_neurons, "n_w": len(used),
         "n_s": f.sizes[0], "fan": f.fan, "n_dn": len(f.dn_rows), "sizes": list(f.sizes), "wmap": used,
         "in_crow": f.in_crow.cpu().numpy(), "in_col": f.in_ci.cpu().numpy(), "in_tcrow": f.in_tcrow.cpu().numpy(),
         "in_tcol": f.in_tci.cpu().numpy(), "in_tperm": f.in_tperm.cpu().numpy(), "n0": f.n0.cpu().numpy(),
         "dn_rows": f.dn_rows.cpu().numpy(), "hop": []}
    for k in range(1, K + 1):
        buf = lambda name: getattr(f, f"{name}{k}").cpu().numpy()     # noqa: E731
        widx = compact[buf("e")]
        drow = np.full(f.sizes[k], -1, np.int64)
        drow[buf("s")] = buf("d")
        s["hop"].append({"nid": buf("n"), "crow": buf("crow"), "col": buf("ci"), "widx": widx, "tcrow": buf("tcrow"),
                         "tcol": buf("tci"), "twidx": widx[buf("tperm")], "drow": drow})
    return s


def net_bytes(s: dict) -> bytes:
    """NET.bin of a structure dict (export.py:52-65 layout)."""
    i32 = lambda a: np.ascontiguousarray(a, dtype=np.int32).tobytes()        # noqa: E731
    parts = [b"FLY1", struct.pack("<8i", s["obs_dim"], s["n_act"], s["hops"], s["n_neurons"], s["n_w"], s["n_s"],
                                   s["fan"], s["n_dn"]),
             i32(s["sizes"]), i32([len(h["col"]) for h in s["hop"]])]
    parts += [i32(s[k]) for k in _PLUG_KEYS]
    for h in s["hop"]:
        parts += [i32(h[k]) for k in _HOP_KEYS]
    parts += [i32(s["dn_rows"]), i32(s["wmap"])]
    return b"".join(parts)


def read_net(src) -> dict:
    """The structure dict of a NET.bin (a path or its bytes), the inverse of net_bytes (export.py:52-65 layout)."""
    raw = src if isinstance(src, (bytes, bytearray)) else Path(src).read_bytes()
    if raw[:4] != b"FLY1":
        raise ValueError("not a FLY1 network file")
    at = [4]

    def ints(n):
        a = np.frombuffer(raw, np.int32, n, at[0]).astype(np.int64)
        at[0] += 4 * n
        return a
    od, na, K, nn, nw, ns, fan, ndn = (int(v) for v in ints(8))
    s = {"obs_dim": od, "n_act": na, "hops": K, "n_neurons": nn, "n_w": nw, "n_s": ns, "fan": fan, "n_dn": ndn}
    s["sizes"] = [int(v) for v in ints(K + 1)]
    E = [int(v) for v in ints(K)]
    E_in = ns * fan
    s["in_crow"], s["in_col"] = ints(ns + 1), ints(E_in)
    s["in_tcrow"], s["in_tcol"], s["in_tperm"] = ints(od + 1), ints(E_in), ints(E_in)
    s["n0"] = ints(ns)
    s["hop"] = []
    for k in range(K):
        rows, src = s["sizes"][k + 1], s["sizes"][k]
        h = {"nid": ints(rows), "crow": ints(rows + 1), "col": ints(E[k]), "widx": ints(E[k]), "tcrow": ints(src + 1),
             "tcol": ints(E[k]), "twidx": ints(E[k]), "drow": ints(rows)}
        s["hop"].append(h)
    s["dn_rows"], s["wmap"] = ints(ndn), ints(nw)
    if at[0] != len(raw):
        raise ValueError("network file of unexpected length")
    return s


def write_net(f, out: Path) -> dict:
    s = structure(f)
    Path(out).write_bytes(net_bytes(s))
    return s


def params_from_torch(f, s: dict) -> list[np.ndarray]:
    """The seven weight arrays in the library's order (export.py:68-70)."""
    return [f.w.detach().cpu().numpy()[s["wmap"]], f.gain.detach().cpu().numpy(), f.theta.detach().cpu().numpy(),
            f.in_w.detach().cpu().numpy(), f.in_b.detach().cpu().numpy(), f.out.weight.detach().cpu().numpy().reshape(-1),
            f.out.bias.detach().cpu().numpy()]


def param_sizes(s: dict) -> list[int]:
    return [s["n_w"], s["n_neurons"], s["n_neurons"], s["n_s"] * s["fan"], s["n_s"], s["n_act"] * s["n_dn"], s["n_act"]]


def write_params(arrs: list[np.ndarray], out: Path, step: int = 0) -> None:
    with open(out, "wb") as fh:
        fh.write(b"FLYP")
        fh.write(struct.pack("<q", step))
        for a in arrs:
            fh.write(np.ascontiguousarray(a, dtype=np.float32).tobytes())


def read_params(path: Path, s: dict) -> tuple[int, list[np.ndarray]]:
    raw = Path(path).read_bytes()
    if raw[:4] != b"FLYP":
        raise ValueError(f"{path}: not a FLYP parameter file")
    step = struct.unpack("<q", raw[4:12])[0]
    out, at = [], 12
    for n in param_sizes(s):
        if at + 4 * n > len(raw):
            raise ValueError(f"{path}: short parameter file")
        out.append(np.frombuffer(raw, np.float32, n, at).copy())
        at += 4 * n
    return step, out


# ------------------------------------------------------------------------------------------------ command line
USAGE = """python -m flyguy_amd.export COMMAND ...  (the converter of flyguy/native/export.py:91-147)

  net GRAPH.npz NET.bin [--hops 3] [--fan 16] [--obs 517]
        the network of a graph file as NET.bin, and its initial weights as NET.init.bin (a FLYP file)
  params CKPT.pt PARAMS.bin [--graph GRAPH.npz]
        a checkpoint's actor weights as a FLYP file (step counter 0: the trainer counts its own steps)
  torch PARAMS.bin CKPT.pt OUT.pt [--graph GRAPH.npz]
        a FLYP / FLYO file's weights put back into the checkpoint CKPT.pt (the strengths in play scattered into the
        full strength array through wmap), written as OUT.pt
  batch CKPT.pt BATCH.bin [--n 64] [--graph GRAPH.npz]
        a fixed FLYB batch (n observations ~ 0.7 N(0,1), teacher logits ~ 2 N(0,1), torch seed 0) and the PyTorch
        path's answer on it, printed as `flyguy_train --check NET PARAMS BATCH` prints the library's

A checkpoint is read with torch.load(weights_only=True): its "model" holds the actor.* weights, and its
config.model.fly_graph / fly_hops / fly_fan name the graph, hop count and plug fan unless --graph / --hops / --fan
are given."""

ARRAY_NAMES = ("W", "gain", "theta", "in_w", "in_b", "out_w", "out_b")


def _graph_path(p) -> str:
    """A graph path as given on the command line: relative to the working directory when the file is there, else as
    FlyActor resolves it (relative to the repository)."""
    q = Path(p)
    return str(q.resolve()) if q.exists() else str(p)


def actor_of(ck: dict, graph: str | None = None, hops: int | None = None, fan: int | None = None,
             obs_dim: int = 517, cls=None, **kw):
    """The actor of a checkpoint dict: built on its graph with its hop count and plug fan (config.model.fly_graph,
    fly_hops, fly_fan, unless given), with its actor.* weights loaded.  `cls` is FlyActor or a subclass of it
    (NativeFlyActor, with its own keyword arguments in kw)."""
    from .fly import FlyActor
    cfg = (ck.get("config") or {}).get("model") or {}
    g = graph or cfg.get("fly_graph")
    if not g:
        raise SystemExit("the checkpoint names no graph (config.model.fly_graph): give --graph")
    weights = {k[len("actor."):]: v for k, v in ck["model"].items() if k.startswith("actor.")}
    if "in_w" not in weights:
        raise SystemExit("the checkpoint holds no fly actor (no actor.in_w)")
    n_act = int(weights["out.bias"].numel()) if "out.bias" in weights else 90
    f = (cls or FlyActor)(_graph_path(g), obs_dim, n_act, hops=int(hops or cfg.get("fly_hops", 3)),
                          fan=int(fan or cfg.get("fly_fan", 16)), **kw)
    f.load_state_dict(weights, strict=False)
    return f


def _load(path) -> dict:
    return torch.load(path, map_location="cpu", weights_only=True)


def _cmd_net(a) -> str:
    from .fly import FlyActor
    f = FlyActor(_graph_path(a.args[0]), a.obs, 90, hops=a.hops or 3, fan=a.fan or 16)
    out = Path(a.args[1])
    s = write_net(f, out)
    write_params(params_from_torch(f, s), out.with_suffix(".init.bin"))
    steps = sum(len(h["col"]) for h in s["hop"])
    return (f"{out}: {s['n_w']:,} strengths in play, neurons per hop {s['sizes']}, {steps:,} connection steps; "
            f"initial weights in {out.with_suffix('.init.bin')}")


def _cmd_params(a) -> str:
    ck = _load(a.args[0])
    f = actor_of(ck, a.graph, a.hops, a.fan, a.obs)
    write_params(params_from_torch(f, structure(f)), Path(a.args[1]), 0)
    return f"{a.args[1]}: the weights of {a.args[0]} (trained {int(ck.get('steps', 0)):,} steps); step counter 0"


def _cmd_torch(a) -> str:
    params_path, ck_path, out = a.args[0], a.args[1], a.args[2]
    ck = _load(ck_path)
    f = actor_of(ck, a.graph, a.hops, a.fan, a.obs)
    s = structure(f)
    step, arrs = read_params(Path(params_path), s)
    model = dict(ck["model"])
    w = model["actor.w"].detach().clone()
    w[torch.as_tensor(np.asarray(s["wmap"], np.int64))] = torch.as_tensor(arrs[0])
    named = dict(zip(("w", "gain", "theta", "in_w", "in_b", "out.weight", "out.bias"), [w] + arrs[1:]))
    named["out.weight"] = torch.as_tensor(named["out.weight"]).reshape(s["n_act"], s["n_dn"])
    for k, v in named.items():
        model["actor." + k] = torch.as_tensor(v).clone()
    torch.save({"model": model, "steps": step, "config": ck.get("config"), "note": f"native weights of {params_path}"},
               out)
    return f"{out}: the weights of {params_path} (step {step:,}) in the checkpoint {ck_path}"


def _cmd_batch(a) -> str:
    f = actor_of(_load(a.args[0]), a.graph, a.hops, a.fan, a.obs)
    n = a.n
    torch.manual_seed(0)
    x = 0.7 * torch.randn(n, f.obs_dim)
    t = 2.0 * torch.randn(n, f.out.out_features)
    f.zero_grad()
    logits = f(x)
    lt = torch.log_softmax(t, -1)
    loss = (lt.exp() * (lt - torch.log_softmax(logits, -1))).sum(-1).mean()
    loss.backward()
    s = structure(f)
    with open(a.args[1], "wb") as fh:
        fh.write(b"FLYB" + struct.pack("<i", n) + x.numpy().astype(np.float32).tobytes() +
                 t.numpy().astype(np.float32).tobytes())
    grads = [f.w.grad.numpy()[np.asarray(s["wmap"], np.int64)], f.gain.grad.numpy(), f.theta.grad.numpy(),
             f.in_w.grad.numpy(), f.in_b.grad.numpy(), f.out.weight.grad.numpy().reshape(-1), f.out.bias.grad.numpy()]
    agree = float((logits.argmax(-1) == t.argmax(-1)).float().mean())
    lines = [f"{a.args[1]}: {n} samples", f"torch: loss {float(loss.detach()):.6f} agree {agree:.4f}",
             "   logits[0][:5] " + " ".join(f"{v:.6f}" for v in logits[0, :5].tolist())]
    for name, g in zip(ARRAY_NAMES, grads):
        g64 = g.astype(np.float64)
        lines.append(f"   grad {name:6s} norm {float(np.sqrt((g64 * g64).sum())):.6e} sum {float(g64.sum()):+.6e}")
    return "\n".join(lines)


_COMMANDS = {"net": (_cmd_net, 2), "params": (_cmd_params, 2), "torch": (_cmd_torch, 3), "batch": (_cmd_batch, 2)}


def main(argv=None) -> int:
    import argparse
    ap = argparse.ArgumentParser(prog="python -m flyguy_amd.export", description=USAGE,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("command", choices=sorted(_COMMANDS))
    ap.add_argument("args", nargs="+")
    ap.add_argument("--graph", default=None)
    ap.add_argument("--hops", type=int, default=None)
    ap.add_argument("--fan", type=int, default=None, help="plug fan (default: the checkpoint's fly_fan, else 16)")
    ap.add_argument("--obs", type=int, default=517)
    ap.add_argument("--n", type=int, default=64)
    a = ap.parse_args(argv)
    fn, nargs = _COMMANDS[a.command]
    if len(a.args) != nargs:
        ap.error(f"{a.command} takes {nargs} paths")
    print(fn(a), flush=True)
    return 0


if __name__ == "__main__":
    import sys
    sys.exit(main())
