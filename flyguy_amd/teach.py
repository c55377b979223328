"""Teach a fly network to choose what a teacher chooses: the small, all-PyTorch teaching loop (flyguy/teach.py).

    python -m flyguy_amd.teach --data MOMENTS.bin [MORE.bin ...] --graph GRAPH.npz [--teacher TEACHER.pt]
        [--start fresh | CKPT.pt] [--hops 3] [--steps 3000] [--batch 128] [--lr 4e-4] [--temp 0.5] [--average 0.999]
        [--holdout 0.05] [--eval-every 250] [--out runs/teach/student.pt] [--device cuda] [--kernel torch|hip] [--seed 0]

What is learned: a teacher scores the 90 actions of a game moment, and the student - a FlyActor on --graph - is
moved toward the same answer: the loss is KL(teacher || student) with the teacher's logits sharpened by --temp.
Teachers: a fly-actor checkpoint (--teacher; its "model" holds actor.* weights of a network on --teacher-graph, by
default --graph), or, without --teacher, the answers stored in the FLYD files.  (The reference can build any network
its model factory knows as the teacher; the factory and those networks are outside this package.)

DATA: FLYD files (observations as binary16, and the teacher's answers when the file has them) and FLYR recordings
of the bot, in any mix (teach.py:53-66).  The last --holdout share of every file is never learned from; the log's
"unseen" figures are measured on (at most about 4,096 of) those held-out moments.

Training (teach.py:96-165): Adam over three groups - the strengths and the plugs at --lr, the neurons' gains and
thresholds at 0.3 of it - with every rate decaying geometrically to a tenth at the last step; batches are drawn
uniformly with replacement (numpy default_rng(--seed)) and sorted.  A running average of the weights (decay
--average, but never slower than step / (step + 9), so that a young average follows closely) is what is scored and
saved.  --kernel hip runs the student's products on the MI355X library (HopHip).
"""
from __future__ import annotations

import argparse
import struct
import sys
import time
from pathlib import Path

import numpy as np
import torch

from .fly import FlyActor


# ------------------------------------------------------------------------------------------------ data
def moments(path: Path):
    """(observations [n, obs size] float16, teacher answers [n, n_act] float16 or None) of a FLYD file or a FLYR
    recording of the bot (teach.py:53-66)."""
    with open(path, "rb") as fh:
        tag = fh.read(4)
        head = fh.read(16)
    if tag == b"FLYD":
        n, obs_dim, n_ans = struct.unpack("<qii", head)
        obs = np.memmap(path, np.float16, "r", 20, (n, obs_dim))
        ans = np.memmap(path, np.float16, "r", 20 + 2 * n * obs_dim, (n, n_ans)) if n_ans > 0 else None
        return obs, ans
    if tag == b"FLYR":
        obs_dim, extra = struct.unpack("<ii", head[:8])
        record = 8 + extra + 2 * obs_dim                 # each decision: 8 bytes, `extra` bytes, the observation
        n = (Path(path).stat().st_size - 12) // record
        rows = np.memmap(path, np.uint8, "r", 12, (n, record))
        return np.ascontiguousarray(rows[:, record - 2 * obs_dim:]).view(np.float16), None
    raise SystemExit(f"{path}: neither a FLYD file nor a recording of the bot")


class Moments:
    """The moments of all data files, cut into the part learned from and the held-out part (the last `holdout` share
    of every file), the held-out part thinned to about 4,096 moments."""

    def __init__(self, paths: list[Path], holdout: float, need_answers: bool):
        learn, held, learn_t, held_t = [], [], [], []
        for p in paths:
            obs, ans = moments(p)
            if need_answers and ans is None:
                raise SystemExit(f"{p}: no teacher's answers in the file and no --teacher")
            keep = len(obs) - max(1, int(len(obs) * holdout))
            learn.append(obs[:keep])
            held.append(obs[keep:])
            if ans is not None:
                learn_t.append(ans[:keep])
                held_t.append(ans[keep:])
            print(f"{p.name}: {len(obs):,} moments read, {len(obs) - keep:,} at its end kept for scoring", flush=True)
        stride = max(1, sum(len(h) for h in held) // 4096)
        self.obs_dim = learn[0].shape[1]
        self.learn = torch.from_numpy(np.concatenate(learn))
        self.held = torch.from_numpy(np.concatenate(held)[::stride].copy())
        self.learn_answers = self.held_answers = None
        if need_answers:
            self.learn_answers = torch.from_numpy(np.concatenate(learn_t))
            self.held_answers = torch.from_numpy(np.concatenate(held_t)[::stride].copy())


# ------------------------------------------------------------------------------------------------ teacher
def _actor_weights(ck: dict) -> dict:
    return {k[len("actor."):]: v for k, v in ck["model"].items() if k.startswith("actor.")}


class Teacher:
    """The teacher's logits for a batch of moments: a fly actor's, or the answers stored with the moments."""

    def __init__(self, data: Moments, checkpoint: Path | None, graph: str, fallback_graph: str, hops: int, device):
        """graph: --teacher-graph (may be empty: then the checkpoint's own config.model.fly_graph, then
        fallback_graph, the student's)."""
        self.data, self.device = data, device
        self.net = None
        self.name = "the answers in the data"
        if checkpoint is not None:
            ck = torch.load(checkpoint, map_location="cpu", weights_only=True)
            cfg = (ck.get("config") or {}).get("model", {})
            net = FlyActor(graph or cfg.get("fly_graph") or fallback_graph, data.obs_dim, 90,
                           hops=int(cfg.get("fly_hops", hops)), fan=int(cfg.get("fly_fan", 16)))
            net.load_state_dict(_actor_weights(ck), strict=False)
            self.net = net.to(device).eval()
            self.name = checkpoint.name

    @property
    def n_act(self) -> int:
        return 90 if self.net is not None else self.data.learn_answers.shape[1]

    def logits(self, x: torch.Tensor, rows, held: bool) -> torch.Tensor:
        if self.net is not None:
            return self.net(x).float()
        stored = self.data.held_answers if held else self.data.learn_answers
        return stored[rows].to(self.device).float()


# ------------------------------------------------------------------------------------------------ student
def kl_to(target: torch.Tensor, logits: torch.Tensor) -> torch.Tensor:
    """Per moment: KL(target || softmax(logits)), target a probability vector (teach.py:139-141)."""
    return (target * (torch.log(target.clamp_min(1e-12)) - torch.log_softmax(logits, -1))).sum(-1)


class Student:
    """The network being taught, its optimiser and learning-rate schedule, and the running average of its weights."""

    NEURON_SHARE = 0.3                   # the gains' and thresholds' rate, as a share of --lr

    def __init__(self, net: FlyActor, shown: FlyActor, lr: float, steps: int, average: float):
        self.net, self.shown = net, shown
        self.steps, self.average = steps, average
        neuron = [net.gain, net.theta]
        others = [p for name, p in net.named_parameters() if name not in ("w", "gain", "theta")]
        self.opt = torch.optim.Adam([{"params": [net.w], "lr": lr},
                                     {"params": neuron, "lr": self.NEURON_SHARE * lr},
                                     {"params": others, "lr": lr}])
        self.base = [g["lr"] for g in self.opt.param_groups]

    def learn(self, step: int, x: torch.Tensor, target: torch.Tensor) -> float:
        decay = 0.1 ** (step / self.steps)               # a tenth of the rate at the last step
        for g, b in zip(self.opt.param_groups, self.base):
            g["lr"] = b * decay
        loss = kl_to(target, self.net(x).float()).mean()
        self.opt.zero_grad(set_to_none=True)
        loss.backward()
        self.opt.step()
        follow = 1.0 - min(self.average, step / (step + 9.0))
        with torch.no_grad():
            for a, b in zip(self.shown.parameters(), self.net.parameters()):
                a.lerp_(b, follow)
        return float(loss.detach())


@torch.no_grad()
def score(shown: FlyActor, teacher: Teacher, data: Moments, temp: float, device) -> tuple[float, float]:
    """On the held-out moments: the share where the student's first choice is the teacher's, and the mean KL."""
    agree = total = 0.0
    for i in range(0, len(data.held), 512):
        x = data.held[i:i + 512].to(device).float()
        t = teacher.logits(x, slice(i, i + 512), held=True)
        s = shown(x).float()
        agree += float((t.argmax(-1) == s.argmax(-1)).sum())
        total += float(kl_to(torch.softmax(t / temp, -1), s).sum())
    return agree / len(data.held), total / len(data.held)


def _make_student(args, obs_dim: int, n_act: int) -> tuple[FlyActor, int]:
    if args.start == "fresh":
        return FlyActor(args.graph, obs_dim, n_act, hops=args.hops, fan=args.fan or 16), 0
    ck = torch.load(args.start, map_location="cpu", weights_only=True)
    cfg = (ck.get("config") or {}).get("model", {})
    net = FlyActor(args.graph, obs_dim, n_act, hops=int(cfg.get("fly_hops", args.hops)),
                   fan=int(args.fan or cfg.get("fly_fan", 16)))
    net.load_state_dict(_actor_weights(ck), strict=False)
    return net, int(ck.get("taught_steps", 0))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--data", nargs="+", type=Path, required=True)
    ap.add_argument("--graph", required=True)
    ap.add_argument("--teacher", type=Path, default=None)
    ap.add_argument("--teacher-graph", default="")
    ap.add_argument("--start", default="fresh")
    ap.add_argument("--hops", type=int, default=3)
    ap.add_argument("--fan", type=int, default=None, help="plug fan (default: the --start checkpoint's fly_fan, else 16)")
    ap.add_argument("--steps", type=int, default=3000)
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--lr", type=float, default=4e-4,
                    help="Adam rate of the strengths and the plug / read-out weights (gains and thresholds: 0.3 x this)")
    ap.add_argument("--temp", type=float, default=0.5)
    ap.add_argument("--average", type=float, default=0.999,
                    help="decay of the weights' running average, the network that is scored and written out")
    ap.add_argument("--holdout", type=float, default=0.05)
    ap.add_argument("--eval-every", type=int, default=250)
    ap.add_argument("--out", type=Path, default=Path("runs") / "teach" / "student.pt")
    ap.add_argument("--device", default="cuda" if torch.cuda.is_available() else "cpu")
    ap.add_argument("--kernel", default="torch", choices=["torch", "hip", "cuda"])
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args(argv)
    device = torch.device(args.device)
    torch.manual_seed(args.seed)
    draw = np.random.default_rng(args.seed)

    data = Moments(args.data, args.holdout, need_answers=args.teacher is None)
    teacher = Teacher(data, args.teacher, args.teacher_graph, args.graph, args.hops, device)
    net, step0 = _make_student(args, data.obs_dim, teacher.n_act)
    net.kernel = "torch" if args.kernel == "torch" else "hip"
    net = net.to(device)
    shown = FlyActor(args.graph, data.obs_dim, teacher.n_act, hops=net.hops, fan=net.fan).to(device).eval()
    shown.load_state_dict(net.state_dict())
    print(net.describe(), flush=True)
    student = Student(net, shown, args.lr, args.steps, args.average)
    saved_cfg = {"fly_graph": str(args.graph), "fly_hops": net.hops, "fly_fan": net.fan, "fly_kernel": "torch"}

    first, first_kl = score(shown, teacher, data, args.temp, device)
    agree = first
    print(f"before learning | held-out moments: argmax agreement {first:.3f}, KL {first_kl:.3f} | "
          f"{len(data.learn):,} moments to learn from over {args.steps * args.batch / len(data.learn):.1f} passes",
          flush=True)
    began, smooth = time.time(), 0.0
    for step in range(1, args.steps + 1):
        rows = torch.as_tensor(np.sort(draw.integers(0, len(data.learn), args.batch)))
        x = data.learn[rows].to(device).float()
        with torch.no_grad():
            target = torch.softmax(teacher.logits(x, rows, held=False) / args.temp, -1)
        loss = student.learn(step, x, target)
        smooth = loss if step == 1 else 0.98 * smooth + 0.02 * loss
        if step % args.eval_every and step != args.steps:
            continue
        agree, dist = score(shown, teacher, data, args.temp, device)
        rate = step * args.batch / (time.time() - began)
        print(f"step {step:,} | KL (running) {smooth:.3f} | held-out moments: argmax agreement {agree:.3f}, KL "
              f"{dist:.3f} | {rate:,.0f} moments/s", flush=True)
        args.out.parent.mkdir(parents=True, exist_ok=True)
        torch.save({"model": {"actor." + k: v.detach().cpu() for k, v in shown.state_dict().items()},
                    "steps": step0 + step, "taught_steps": step0 + step, "config": {"model": saved_cfg},
                    "taught_by": teacher.name, "unseen_same_first_choice": agree}, args.out)
    print(f"{args.out}: running average written; argmax agreement with the teacher on held-out moments "
          f"{first:.3f} -> {agree:.3f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
