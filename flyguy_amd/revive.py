"""Bring silent neurons back without changing what the network does, on the CPU (the tool of
flyguy/native/revive.py; the trainer's own surgery is fc_revive in the library):

    python -m flyguy_amd.revive NET.bin PARAMS_IN.bin CHUNK.bin PARAMS_OUT.bin [--samples 512] [--seed 0]
                                [--passes 3] [--target 0.4]

NET.bin takes the place of the reference's TEMPLATE.pt and graph file: the sending and receiving neuron of every
strength in play comes from the hop index arrays.  The first --samples moments of CHUNK.bin (a FLYD file with the
teacher's answers) are surveyed: a neuron outside the sensory layer that fires for none of them in any hop is
silent.  Its incoming strengths keep their sizes and get a random sign (numpy default_rng(--seed)), its gain and
threshold return to 1 and -4, its strengths onto live neurons and its action weights become 0 (it sent nothing and
still sends nothing, so the network's answers do not change), and then, --passes times, its incoming strengths are
scaled so that its input's rms is --target (clipped to 0.02..200 times).  The KL to the teacher is checked to be
unchanged after every pass.  Everything runs in float32 with PyTorch CPU tensors (revive.py:56-128); the GPU beside it
belongs to the trainer.
"""
from __future__ import annotations

import argparse
import struct
import sys
from pathlib import Path

import numpy as np
import torch

from .export import read_net, read_params, write_params


def _chunk(path: Path, samples: int, obs_dim: int, n_act: int):
    """The first `samples` moments of a FLYD file: observations and teacher logits, float32 (revive.py:51-56)."""
    with open(path, "rb") as fh:
        if fh.read(4) != b"FLYD":
            raise SystemExit(f"{path}: not a FLYD file")
        n, od, na = struct.unpack("<qii", fh.read(16))
        if od != obs_dim or na != n_act:
            raise SystemExit(f"{path}: moments of {od} numbers and {na} answers, the network reads {obs_dim} and scores {n_act}")
        k = min(samples, n)
        obs = np.frombuffer(fh.read(k * od * 2), np.float16).reshape(k, od).astype(np.float32)
        fh.seek(20 + n * od * 2)
        tl = np.frombuffer(fh.read(k * na * 2), np.float16).reshape(k, na).astype(np.float32)
    return torch.from_numpy(obs), torch.from_numpy(tl)


class Net:
    """The network of a NET.bin with one set of weights, as PyTorch CPU tensors (index_add form, as revive.py's)."""

    def __init__(self, s: dict):
        self.s = s
        L = torch.as_tensor
        self.in_r = L(np.repeat(np.arange(s["n_s"]), np.diff(s["in_crow"])))
        self.in_c = L(s["in_col"])
        self.n0 = L(s["n0"])
        self.hop = []
        for h in s["hop"]:
            rows = len(h["nid"])
            drow = np.asarray(h["drow"])
            keep = np.flatnonzero(drow >= 0)
            self.hop.append({"r": L(np.repeat(np.arange(rows), np.diff(h["crow"]))), "c": L(h["col"]), "widx": L(h["widx"]),
                             "nid": L(h["nid"]), "s": L(keep), "d": L(drow[keep]), "rows": rows})
        self.dn = L(s["dn_rows"])
        # the sending / receiving neuron of every strength in play
        self.pre = np.full(s["n_w"], -1, np.int64)
        self.post = np.full(s["n_w"], -1, np.int64)
        below = np.asarray(s["n0"])
        for h in s["hop"]:
            nid = np.asarray(h["nid"])
            tgt = np.repeat(np.arange(len(nid)), np.diff(h["crow"]))
            self.pre[np.asarray(h["widx"])] = below[np.asarray(h["col"])]
            self.post[np.asarray(h["widx"])] = nid[tgt]
            below = nid

    @torch.no_grad()
    def survey(self, P, obs: torch.Tensor, tl: torch.Tensor):
        """Firing counts per neuron over every hop it takes part in, neurons seen in a hop, the largest input rms over
        those hops, the firing share per layer and the KL to the teacher (revive.py:61-95)."""
        s = self.s
        W, gain, theta, in_w, in_b, ow, ob = (torch.as_tensor(p) for p in P)
        ow = ow.view(s["n_act"], s["n_dn"])
        N, K = s["n_neurons"], s["hops"]
        fired = torch.zeros(N)
        seen = torch.zeros(N, dtype=torch.bool)
        sq = [torch.zeros(h["rows"]) for h in self.hop]
        share = [0.0] * (K + 1)
        kl = 0.0
        thr = torch.nn.functional.softplus(theta)
        n = obs.shape[0]
        for i in range(0, n, 64):
            x = obs[i:i + 64]
            drive = torch.zeros(len(x), s["n_s"]).index_add_(1, self.in_r, x[:, self.in_c] * in_w) + in_b
            h = torch.relu(gain[self.n0] * drive - thr[self.n0])
            share[0] += float((h > 0).float().mean()) * len(x)
            for k, hp in enumerate(self.hop):
                z = torch.zeros(len(x), hp["rows"]).index_add_(1, hp["r"], h[:, hp["c"]] * W[hp["widx"]])
                if len(hp["s"]):
                    z = z.index_add(1, hp["s"], drive[:, hp["d"]])
                sq[k] += z.pow(2).sum(0)
                h = torch.relu(gain[hp["nid"]] * z - thr[hp["nid"]])
                fired[hp["nid"]] += (h > 0).float().sum(0)
                seen[hp["nid"]] = True
                share[k + 1] += float((h > 0).float().mean()) * len(x)
            lp = torch.log_softmax(h[:, self.dn] @ ow.t() + ob, -1)
            tp = torch.log_softmax(tl[i:i + 64], -1)
            kl += float((tp.exp() * (tp - lp)).sum())
        rms = torch.zeros(N)
        for k, hp in enumerate(self.hop):
            rms[hp["nid"]] = torch.maximum(rms[hp["nid"]], (sq[k] / n).sqrt())
        return fired.numpy(), seen.numpy(), rms.numpy(), [v / n for v in share], kl / n


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("net")
    ap.add_argument("params")
    ap.add_argument("chunk")
    ap.add_argument("out")
    ap.add_argument("--samples", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--passes", type=int, default=3, help="rounds of bringing the revived neurons' inputs to --target")
    ap.add_argument("--target", type=float, default=0.4, help="input size (rms) given to a revived neuron")
    args = ap.parse_args(argv)
    s = read_net(Path(args.net))
    step, P = read_params(Path(args.params), s)
    net = Net(s)
    obs, tl = _chunk(Path(args.chunk), args.samples, s["obs_dim"], s["n_act"])
    fired, seen, _, share, kl0 = net.survey(P, obs, tl)
    is_sens = np.zeros(s["n_neurons"], bool)
    is_sens[np.asarray(s["n0"])] = True
    dead = seen & (fired == 0) & ~is_sens
    print(f"native step {step:,}, {len(obs)} samples: firing share per hop {[round(v, 3) for v in share]}; KL {kl0:.4f}")
    print(f"silent neurons (never fire in any hop): {int(dead.sum()):,} of {int((seen & ~is_sens).sum()):,} in play "
          f"outside the sensory layer")
    rng = np.random.default_rng(args.seed)
    w = P[0].copy()
    inc, outg = dead[net.post], dead[net.pre]
    w[inc] = np.abs(w[inc]) * rng.choice([-1.0, 1.0], int(inc.sum())).astype(np.float32)
    w[outg & ~inc] = 0.0                       # silent -> live only: a connection between two silent neurons stays
    gain, theta = P[1].copy(), P[2].copy()
    gain[dead], theta[dead] = 1.0, -4.0
    out_w = P[5].copy().reshape(s["n_act"], -1)
    dn_ids = np.asarray(s["hop"][-1]["nid"])[np.asarray(s["dn_rows"])]
    out_w[:, dead[dn_ids]] = 0.0               # a silent descending neuron sent nothing to the actions either
    P2 = [w, gain, theta, P[3], P[4], out_w.reshape(P[5].shape), P[6]]
    print(f"re-signed {int(inc.sum()):,} incoming strengths, zeroed {int((outg & ~inc).sum()):,} outgoing ones and the "
          f"action weights of {int(dead[dn_ids].sum())} descending neurons")
    for it in range(args.passes + 1):          # hop after hop: bring every revived neuron's input to the target size
        fired2, _, rms, share2, kl1 = net.survey(P2, obs, tl)
        dead2 = seen & (fired2 == 0) & ~is_sens
        rate = (fired2[dead] / len(obs)).mean() if dead.any() else 0.0
        print(f"   pass {it}: firing share per hop {[round(v, 3) for v in share2]}; still silent {int(dead2.sum()):,}; "
              f"the revived fire {rate:.3f} of the time; KL {kl1:.4f}")
        if abs(kl1 - kl0) >= 1e-4 * max(1.0, abs(kl0)):
            raise SystemExit("the surgery changed the network's output")
        if it == args.passes:
            break
        scale = np.ones(s["n_neurons"], np.float32)
        m = dead & (rms > 0)
        scale[m] = np.clip(args.target / rms[m], 0.02, 200.0)
        w[inc] *= scale[net.post[inc]]
    write_params(P2, Path(args.out), step)
    print("wrote", args.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
