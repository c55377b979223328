"""Teach a fly network to choose what a teacher chooses: the small, all-PyTorch loop of flyguy/teach.py.

    python -m flyguy_amd.teach --data MOMENTS.bin [MORE.bin ...] --graph GRAPH.npz [--teacher TEACHER.pt]
        [--start fresh | CKPT.pt] [--hops 3] [--steps 3000] [--batch 128] [--lr 4e-4] [--temp 0.5] [--average 0.999]
        [--holdout 0.05] [--eval-every 250] [--out runs/teach/student.pt] [--device cuda] [--kernel torch|hip] [--seed 0]

DATA: game moments, any mix of FLYD files (observations as 16-bit floats, and the teacher's answers when the file
holds them) and FLYR recordings of the bot (teach.py:53-66).  The last --holdout share of every file is never
learned from; "unseen" in the log is the share of those moments on which the student's first choice is the
teacher's.  The teacher scores the 90 actions of a moment: a fly actor checkpoint (--teacher; its "model" holds the
actor.* weights of a network on --teacher-graph, by default --graph), or, without --teacher, the answers stored in
the FLYD files.  The reference builds any model its factory knows as the teacher; the factory and the other network
kinds are outside this package.

The student: a FlyActor on --graph, fresh (--start fresh: strengths from the synapse counts and transmitter signs) or
from a checkpoint.  Adam with the neurons' gains and thresholds at 0.3 of the rate, the rate falling to a tenth by
the end, the loss the distance from the teacher's answer sharpened by --temp, and a running average of the weights
that is scored and saved (teach.py:96-165).  --kernel hip runs the hops on the MI355X library (HopHip).
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


def moments(path: Path):
    """(observations [n, obs size] float16, teacher answers [n, n_act] float16 or None) of a FLYD file or a FLYR
    recording (teach.py:53-66)."""
    with open(path, "rb") as fh:
        kind = fh.read(4)
        if kind == b"FLYD":
            n, od, na = struct.unpack("<qii", fh.read(16))
            obs = np.memmap(path, np.float16, "r", 20, (n, od))
            ans = np.memmap(path, np.float16, "r", 20 + 2 * n * od, (n, na)) if na > 0 else None
            return obs, ans
        if kind == b"FLYR":
            od, extra = struct.unpack("<ii", fh.read(8))
            rec = 8 + extra + 2 * od
            n = (path.stat().st_size - 12) // rec
            raw = np.memmap(path, np.uint8, "r", 12, (n, rec))
            return np.ascontiguousarray(raw[:, 8 + extra:]).view(np.float16), None
    raise SystemExit(f"{path}: neither a FLYD file nor a recording of the bot")


def _actor_state(ck: dict) -> dict:
    return {k[len("actor."):]: v for k, v in ck["model"].items() if k.startswith("actor.")}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--data", nargs="+", type=Path, required=True)
    ap.add_argument("--graph", required=True)
    ap.add_argument("--teacher", type=Path, default=None)
    ap.add_argument("--teacher-graph", default="")
    ap.add_argument("--start", default="fresh")
    ap.add_argument("--hops", type=int, default=3)
    ap.add_argument("--fan", type=int, default=16)
    ap.add_argument("--steps", type=int, default=3000)
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--lr", type=float, default=4e-4,
                    help="for the connection strengths and the plugs; the neurons' gains and thresholds get 0.3 of it")
    ap.add_argument("--temp", type=float, default=0.5)
    ap.add_argument("--average", type=float, default=0.999, help="the running average of the weights that is saved and scored")
    ap.add_argument("--holdout", type=float, default=0.05)
    ap.add_argument("--eval-every", type=int, default=250)
    ap.add_argument("--out", type=Path, default=Path("runs") / "teach" / "student.pt")
    ap.add_argument("--device", default="cuda" if torch.cuda.is_available() else "cpu")
    ap.add_argument("--kernel", default="torch", choices=["torch", "hip", "cuda"])
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args(argv)
    dev = torch.device(args.device)
    torch.manual_seed(args.seed)
    rng = np.random.default_rng(args.seed)

    # ---- the game moments (and the teacher's answers where the files hold them)
    seen, unseen, seen_t, unseen_t = [], [], [], []
    for p in args.data:
        m, ans = moments(p)
        if args.teacher is None and ans is None:
            raise SystemExit(f"{p}: no teacher's answers in the file and no --teacher")
        cut = len(m) - max(1, int(len(m) * args.holdout))
        seen.append(m[:cut]); unseen.append(m[cut:])
        if ans is not None:
            seen_t.append(ans[:cut]); unseen_t.append(ans[cut:])
        print(f"{p.name}: {len(m):,} moments, the last {len(m) - cut:,} held out", flush=True)
    od = seen[0].shape[1]
    every = max(1, sum(len(u) for u in unseen) // 4096)                    # (4,096 of them are enough)
    seen = torch.from_numpy(np.concatenate(seen))
    unseen = torch.from_numpy(np.concatenate(unseen)[::every].copy())
    stored = args.teacher is None
    if stored:
        seen_t = torch.from_numpy(np.concatenate(seen_t))
        unseen_t = torch.from_numpy(np.concatenate(unseen_t)[::every].copy())

    # ---- the teacher, and the student
    teacher = None
    n_act = seen_t.shape[1] if stored else 90
    if not stored:
        tck = torch.load(args.teacher, map_location="cpu", weights_only=True)
        tcfg = (tck.get("config") or {}).get("model", {})
        teacher = FlyActor(args.teacher_graph or tcfg.get("fly_graph") or args.graph, od, 90,
                           hops=int(tcfg.get("fly_hops", args.hops)))
        teacher.load_state_dict(_actor_state(tck), strict=False)
        teacher = teacher.to(dev).eval()
    if args.start == "fresh":
        student, step0 = FlyActor(args.graph, od, n_act, hops=args.hops, fan=args.fan), 0
    else:
        sck = torch.load(args.start, map_location="cpu", weights_only=True)
        scfg = (sck.get("config") or {}).get("model", {})
        student = FlyActor(args.graph, od, n_act, hops=int(scfg.get("fly_hops", args.hops)), fan=args.fan)
        student.load_state_dict(_actor_state(sck), strict=False)
        step0 = int(sck.get("taught_steps", 0))
    student.kernel = "hip" if args.kernel in ("hip", "cuda") else "torch"
    student = student.to(dev)
    shown = FlyActor(args.graph, od, n_act, hops=student.hops, fan=args.fan).to(dev).eval()   # the running average
    shown.load_state_dict(student.state_dict())
    print(student.describe(), flush=True)
    cfg = {"fly_graph": str(args.graph), "fly_hops": student.hops, "fly_kernel": "torch"}

    def answers(x, idx, held):
        if stored:
            return (unseen_t if held else seen_t)[idx].to(dev).float()
        return teacher(x).float()

    @torch.no_grad()
    def score() -> tuple[float, float]:
        same = kl = 0.0
        for i in range(0, len(unseen), 512):
            x = unseen[i:i + 512].to(dev).float()
            t = answers(x, slice(i, i + 512), True)
            s = shown(x).float()
            same += float((t.argmax(-1) == s.argmax(-1)).sum())
            target = torch.softmax(t / args.temp, -1)
            kl += float((target * (torch.log(target.clamp_min(1e-12)) - torch.log_softmax(s, -1))).sum())
        return same / len(unseen), kl / len(unseen)

    plugs = [p for k, p in student.named_parameters() if k not in ("w", "gain", "theta")]
    opt = torch.optim.Adam([{"params": [student.w], "lr": args.lr},
                            {"params": [student.gain, student.theta], "lr": 0.3 * args.lr},
                            {"params": plugs, "lr": args.lr}])
    base = [g["lr"] for g in opt.param_groups]
    a0, k0 = score()
    a = a0
    print(f"start | unseen: same first choice {a0:.3f}, distance {k0:.3f} | {len(seen):,} moments to learn from, "
          f"{args.steps * args.batch / len(seen):.1f} passes over them", flush=True)
    t0, run = time.time(), 0.0
    for step in range(1, args.steps + 1):
        for g, b in zip(opt.param_groups, base):                   # the rate falls to a tenth by the end
            g["lr"] = b * 0.1 ** (step / args.steps)
        idx = torch.as_tensor(np.sort(rng.integers(0, len(seen), args.batch)))
        x = seen[idx].to(dev).float()
        with torch.no_grad():
            target = torch.softmax(answers(x, idx, False) / args.temp, -1)
        loss = (target * (torch.log(target.clamp_min(1e-12)) - torch.log_softmax(student(x).float(), -1))).sum(-1).mean()
        opt.zero_grad(set_to_none=True)
        loss.backward()
        opt.step()
        keep = min(args.average, step / (step + 9.0))               # (a young average follows closely)
        with torch.no_grad():
            for sa, sb in zip(shown.parameters(), student.parameters()):
                sa.lerp_(sb, 1.0 - keep)
        run = loss.item() if step == 1 else 0.98 * run + 0.02 * loss.item()
        if step % args.eval_every == 0 or step == args.steps:
            a, k = score()
            print(f"step {step:,} | distance {run:.3f} | unseen: same first choice {a:.3f}, distance {k:.3f} | "
                  f"{step * args.batch / (time.time() - t0):,.0f} moments a second", flush=True)
            args.out.parent.mkdir(parents=True, exist_ok=True)
            torch.save({"model": {"actor." + k_: v.detach().cpu() for k_, v in shown.state_dict().items()},
                        "steps": step0 + step, "taught_steps": step0 + step, "config": {"model": cfg},
                        "taught_by": args.teacher.name if args.teacher else "the answers in the data",
                        "unseen_same_first_choice": a}, args.out)
    print(f"saved {args.out} (the running average; the teacher's first choice on {a:.3f} of unseen moments, {a0:.3f} at "
          f"the start)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
