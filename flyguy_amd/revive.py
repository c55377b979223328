"""Bring silent neurons back without changing what the network does, on the CPU (the tool of
flyguy/native/revive.py; the trainer's own surgery is fc_revive in the library):

    python -m flyguy_amd.revive NET.bin PARAMS_IN.bin CHUNK.bin PARAMS_OUT.bin [--samples 512] [--seed 0]
                                [--passes 3] [--target 0.4]

A neuron outside the sensory layer that fires for none of the first --samples moments of CHUNK.bin (a FLYD file with
the teacher's answers) in any hop it takes part in is silent: it passes no gradient, so nothing would ever wake it.
The surgery (revive.py:96-128):
  - its incoming strengths keep their sizes and get random signs (numpy default_rng(--seed), one draw per strength
    in weight-index order), so its input is positive about half the time;
  - its gain and threshold return to their starting values 1 and -4;
  - its outgoing strengths onto live neurons, and for a descending neuron its action weights, become 0: it sent
    nothing before and sends nothing now, so the network's answers do not change (a connection between two silent
    neurons keeps its new sign: its target is silent too);
  - then, --passes times, its incoming strengths are scaled so that its input's rms over the samples comes to
    --target (the factor clipped to 0.02..200).
After every pass the KL to the teacher is checked to be unchanged.  NET.bin takes the place of the reference's
TEMPLATE.pt and graph file: the sending and receiving neuron of every strength in play come from the hop index
arrays.  Float32, PyTorch CPU tensors; the GPU beside it belongs to the trainer.
"""
from __future__ import annotations

import argparse
import struct
import sys
from pathlib import Path
from typing import NamedTuple

import numpy as np
import torch

from .export import read_net, read_params, write_params

CHUNK = 64                                       # samples per pass of the survey


def _chunk(path: Path, samples: int, obs_dim: int, n_act: int):
    """The first `samples` moments of a FLYD file: observations and teacher logits as float32 tensors."""
    raw = Path(path).read_bytes()
    if raw[:4] != b"FLYD":
        raise SystemExit(f"{path}: not a FLYD file")
    n, od, na = struct.unpack_from("<qii", raw, 4)
    if od != obs_dim or na != n_act:
        raise SystemExit(f"{path}: moments of {od} numbers and {na} answers, the network reads {obs_dim} and scores {n_act}")
    k = min(samples, n)
    obs = np.frombuffer(raw, np.float16, k * od, 20).reshape(k, od)
    answers = np.frombuffer(raw, np.float16, k * na, 20 + 2 * n * od).reshape(k, na)
    return torch.from_numpy(obs.astype(np.float32)), torch.from_numpy(answers.astype(np.float32))


class Survey(NamedTuple):
    fired: np.ndarray        # per neuron: (layer, sample) pairs in which it fires, over the hops it takes part in
    seen: np.ndarray         # per neuron: whether it takes part in a hop
    rms: np.ndarray          # per neuron: the largest rms of its input over the hops it takes part in
    share: list[float]       # per layer (sensory first): the share of (row, sample) pairs that fire
    kl: float                # mean KL(teacher || network) over the samples


class Net:
    """The network of a NET.bin, evaluated with one set of weights on PyTorch CPU tensors (gather / index_add
    products), and the sending (`pre`) and receiving (`post`) neuron of every strength in play."""

    def __init__(self, s: dict):
        self.s = s
        t = torch.as_tensor
        counts = np.diff(np.asarray(s["in_crow"]))
        self.plug = (t(np.repeat(np.arange(s["n_s"]), counts)), t(np.asarray(s["in_col"])))
        self.n0 = t(np.asarray(s["n0"]))
        self.layers = []
        self.pre = np.full(s["n_w"], -1, np.int64)
        self.post = np.full(s["n_w"], -1, np.int64)
        below = np.asarray(s["n0"])
        for h in s["hop"]:
            nid, col, widx = np.asarray(h["nid"]), np.asarray(h["col"]), np.asarray(h["widx"])
            target = np.repeat(np.arange(len(nid)), np.diff(np.asarray(h["crow"])))
            drow = np.asarray(h["drow"])
            redriven = np.flatnonzero(drow >= 0)
            self.layers.append({"row": t(target), "col": t(col), "widx": t(widx), "nid": t(nid),
                                "redriven": t(redriven), "drive_rows": t(drow[redriven])})
            self.pre[widx] = below[col]
            self.post[widx] = nid[target]
            below = nid
        self.dn = t(np.asarray(s["dn_rows"]))

    def _states(self, P, x: torch.Tensor):
        """Per layer of a batch: (neurons, pre-activation, firing), sensory layer first; then the logits."""
        s = self.s
        W, gain, theta, in_w, in_b, ow, ob = (torch.as_tensor(p) for p in P)
        thr = torch.nn.functional.softplus(theta)
        rows, cols = self.plug
        drive = torch.zeros(len(x), s["n_s"]).index_add_(1, rows, x[:, cols] * in_w) + in_b
        h = torch.relu(gain[self.n0] * drive - thr[self.n0])
        yield self.n0, drive, h
        for L in self.layers:
            z = torch.zeros(len(x), len(L["nid"])).index_add_(1, L["row"], h[:, L["col"]] * W[L["widx"]])
            if len(L["redriven"]):
                z = z.index_add(1, L["redriven"], drive[:, L["drive_rows"]])
            h = torch.relu(gain[L["nid"]] * z - thr[L["nid"]])
            yield L["nid"], z, h
        yield None, None, h[:, self.dn] @ ow.view(s["n_act"], s["n_dn"]).t() + ob

    @torch.no_grad()
    def survey(self, P, obs: torch.Tensor, teacher: torch.Tensor) -> Survey:
        """The Survey of the moments, in passes of CHUNK samples (revive.py:61-95)."""
        N, layers = self.s["n_neurons"], len(self.layers) + 1
        fired = torch.zeros(N)
        seen = torch.zeros(N, dtype=torch.bool)
        sq = [None] * layers
        firing = [0.0] * layers
        kl = 0.0
        n = len(obs)
        for i in range(0, n, CHUNK):
            x = obs[i:i + CHUNK]
            for k, (nid, z, h) in enumerate(self._states(P, x)):
                if nid is None:                                   # the logits
                    lt = torch.log_softmax(teacher[i:i + CHUNK], -1)
                    kl += float((lt.exp() * (lt - torch.log_softmax(h, -1))).sum())
                    continue
                on = h > 0
                firing[k] += float(on.float().mean()) * len(x)
                if k == 0:
                    continue                                      # (the sensory layer is never revived)
                fired[nid] += on.float().sum(0)
                seen[nid] = True
                sq[k] = z.pow(2).sum(0) if sq[k] is None else sq[k] + z.pow(2).sum(0)
        rms = torch.zeros(N)
        for k, L in enumerate(self.layers, start=1):
            rms[L["nid"]] = torch.maximum(rms[L["nid"]], (sq[k] / n).sqrt())
        return Survey(fired.numpy(), seen.numpy(), rms.numpy(), [v / n for v in firing], kl / n)


class Revival:
    """The surgery on one set of weights (the seven arrays, in the library's order)."""

    def __init__(self, net: Net, P: list[np.ndarray], dead: np.ndarray, seed: int):
        s = net.s
        self.net, self.dead = net, dead
        self.incoming = dead[net.post]                            # strengths into a silent neuron
        outgoing = dead[net.pre] & ~self.incoming                 # strengths from a silent neuron onto a live one
        w = P[0].copy()
        signs = np.random.default_rng(seed).choice([-1.0, 1.0], int(self.incoming.sum())).astype(np.float32)
        w[self.incoming] = np.abs(w[self.incoming]) * signs
        w[outgoing] = 0.0
        gain, theta = P[1].copy(), P[2].copy()
        gain[dead], theta[dead] = 1.0, -4.0
        actions = P[5].copy().reshape(s["n_act"], s["n_dn"])
        descending = np.asarray(s["hop"][-1]["nid"])[np.asarray(s["dn_rows"])]
        actions[:, dead[descending]] = 0.0
        self.P = [w, gain, theta, P[3], P[4], actions.reshape(-1), P[6]]
        self.counts = (int(self.incoming.sum()), int(outgoing.sum()), int(dead[descending].sum()))

    def rescale(self, rms: np.ndarray, target: float) -> None:
        """Bring every revived neuron's input rms to `target` (factors clipped to 0.02..200)."""
        factor = np.ones(len(rms), np.float32)
        m = self.dead & (rms > 0)
        factor[m] = np.clip(target / rms[m], 0.02, 200.0)
        w = self.P[0]
        w[self.incoming] *= factor[self.net.post[self.incoming]]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("net")
    ap.add_argument("params")
    ap.add_argument("chunk")
    ap.add_argument("out")
    ap.add_argument("--samples", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--passes", type=int, default=3,
                    help="survey-and-rescale rounds applied to the inputs of the neurons brought back")
    ap.add_argument("--target", type=float, default=0.4,
                    help="root-mean-square pre-activation each neuron brought back is scaled towards")
    args = ap.parse_args(argv)
    s = read_net(Path(args.net))
    step, P = read_params(Path(args.params), s)
    net = Net(s)
    obs, teacher = _chunk(Path(args.chunk), args.samples, s["obs_dim"], s["n_act"])
    fired, seen, _, share, kl0 = net.survey(P, obs, teacher)
    outside = np.ones(s["n_neurons"], bool)
    outside[np.asarray(s["n0"])] = False                          # neurons outside the sensory layer
    dead = seen & (fired == 0) & outside
    n = len(obs)
    print(f"weights of step {step:,} surveyed on {n} samples | share of (neuron, sample) firing per layer "
          f"{[round(v, 3) for v in share]} | KL {kl0:.4f}")
    print(f"silent neurons: {int(dead.sum()):,} of the {int((seen & outside).sum()):,} hop neurons outside the sensory "
          f"layer fire for none of the samples")
    rev = Revival(net, P, dead, args.seed)
    print("surgery: {:,} strengths into silent neurons given a new sign, {:,} from them into live neurons set to 0, "
          "read-out weights of {} silent descending neurons set to 0".format(*rev.counts))
    for k in range(args.passes + 1):
        fired2, _, rms, share2, kl = net.survey(rev.P, obs, teacher)
        still = seen & (fired2 == 0) & outside
        woke = float((fired2[dead] / n).mean()) if dead.any() else 0.0
        print(f"   round {k} | firing shares {[round(v, 3) for v in share2]} | silent {int(still.sum()):,} | "
              f"those brought back fire on {woke:.3f} of the samples | KL {kl:.4f}")
        if abs(kl - kl0) >= 1e-4 * max(1.0, abs(kl0)):
            raise SystemExit("the surgery changed the network's output")
        if k < args.passes:
            rev.rescale(rms, args.target)
    write_params(rev.P, Path(args.out), step)
    print(f"{args.out}: written (step {step:,})")
    return 0


if __name__ == "__main__":
    sys.exit(main())
