"""The all-PyTorch teaching loop (python -m flyguy_amd.teach, flyguy/teach.py): a student fly network learns a teacher
fly network's choices on a toy graph, from a teacher checkpoint and from the answers stored in FLYD files; the
saved running average loads into a FlyActor."""
from __future__ import annotations

import re

import numpy as np
import torch

from conftest import GOLDEN, lively, toy
from flyguy_amd.fly import FlyActor
from flyguy_amd.teach import main
from oracle import trainer as ot


def _data(tmp_path, teacher=None, n=640):
    rng = np.random.default_rng(3)
    obs = rng.standard_normal((n, 517)).astype(np.float16)
    if teacher is None:
        ans = np.zeros((n, 0), np.float16)
    else:
        with torch.no_grad():
            ans = teacher(torch.from_numpy(obs.astype(np.float32))).numpy().astype(np.float16)
    p = tmp_path / ("answers.bin" if teacher is not None else "moments.bin")
    ot.write_chunk(p, obs, ans)
    return p


def _teacher(tmp_path):
    graph = str(GOLDEN / "toy_a.npz")
    torch.manual_seed(5)
    t = lively(FlyActor(toy("a"), 517, 90, hops=3), 5)
    with torch.no_grad():
        t.out.weight.mul_(10.0)                       # decided answers, so that first choices can be learned
    ck = tmp_path / "teacher.pt"
    torch.save({"model": {"actor." + k: v for k, v in t.state_dict().items()},
                "config": {"model": {"fly_graph": graph, "fly_hops": 3}}}, ck)
    return graph, t, ck


def _distances(out):
    start = float(re.search(r"before learning \| held-out moments: argmax agreement [0-9.]+, KL ([0-9.]+)", out).group(1))
    last = [float(v) for v in re.findall(r"\| held-out moments: argmax agreement [0-9.]+, KL ([0-9.]+) \|", out)][-1]
    return start, last


def test_teach_from_a_teacher_network(tmp_path, capsys):
    graph, t, ck = _teacher(tmp_path)
    data = _data(tmp_path)
    out_ck = tmp_path / "student.pt"
    assert main(["--data", str(data), "--graph", graph, "--teacher", str(ck), "--steps", "60", "--batch", "32",
                 "--lr", "3e-3", "--temp", "1.0", "--eval-every", "30", "--out", str(out_ck), "--device", "cpu"]) == 0
    out = capsys.readouterr().out
    start, last = _distances(out)
    assert last < start
    ck2 = torch.load(out_ck, weights_only=True)
    assert ck2["taught_steps"] == 60 and ck2["config"]["model"]["fly_hops"] == 3
    s = FlyActor(graph, 517, 90, hops=3)
    s.load_state_dict({k[6:]: v for k, v in ck2["model"].items()})


def test_teach_from_stored_answers(tmp_path, capsys):
    graph, t, _ = _teacher(tmp_path)
    data = _data(tmp_path, teacher=t)
    assert main(["--data", str(data), "--graph", graph, "--steps", "60", "--batch", "32", "--lr", "3e-3", "--temp", "1.0",
                 "--eval-every", "60", "--out", str(tmp_path / "s.pt"), "--device", "cpu"]) == 0
    start, last = _distances(capsys.readouterr().out)
    assert last < start


@__import__("pytest").mark.gpu
def test_teach_on_the_gpu_kernels(tmp_path, capsys, gpu_lib):
    """--kernel hip: the student's hops run as the library's products (HopHip) on the GPU."""
    graph, t, ck = _teacher(tmp_path)
    data = _data(tmp_path)
    import flyguy_amd.fly_hip as fh
    calls = []
    orig = fh.HopHip.forward

    def counted(ctx, *a):
        calls.append(1)
        return orig(ctx, *a)
    fh.HopHip.forward = staticmethod(counted)
    try:
        assert main(["--data", str(data), "--graph", graph, "--teacher", str(ck), "--steps", "40", "--batch", "64",
                     "--lr", "3e-3", "--temp", "1.0", "--eval-every", "20", "--out", str(tmp_path / "g.pt"), "--device",
                     "cuda", "--kernel", "hip"]) == 0
    finally:
        fh.HopHip.forward = staticmethod(orig)
    start, last = _distances(capsys.readouterr().out)
    assert calls and last < start
