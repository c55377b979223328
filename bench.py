#!/usr/bin/env python3
"""Benchmark of the fly actor's batched inference and teaching step on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--batch 4096] [--cpu-sample 8192] [--cpu-train-batch 4096]
                    [--no-cpu] [--no-floor] [--latency-calls 200] [--trainer-steps 60] [--bf16-steps 10]
                    [--connectome-steps 10] [--hophip-steps 5] [--shipped-steps 20]

Workload: the synthetic 3-hop network of the benchmark shape (16,894 -> 46,393 -> 37,748 -> 1,332 rows; 1.2M /
1.5M / 292,734 connections = 2,992,734 strengths; lognormal(1.5) in-degree; re-drive rows 12,698 / 5,278 / 12),
fp32, B = 4096, observations ~N(0,1) and teacher logits ~N(0,2) already in device memory.
  value  : decisions / s of the batched forward (fc_forward: plug, 3 hops, read-out), K timed batches;
  train  : samples / s of the full teaching step (fc_teach_step: forward, KL loss, backward, Adam + running
           average), K timed steps;
  roofline: the dominant kernel's algorithmic bytes per launch / its mean duration (HIP events around that kernel
           alone, on the library's stream over the timed region), against 8 TB/s; the dominant kernel and the
           per-stage times (stages_ms) come from a few calls profiled stage by stage before the timed region;
  cpu_baseline: the reference's own CPU forward (fly_infer.cpp, compiled into oracle/_ref) on a bounded sample of
           the same network, one core (and, under "all_cores", one handle per thread on up to 16 host cores), and
           under "torch_cpu" the reference's PyTorch CPU path (FlyActor's sparse products) at batch 1 and 4096;
           train: one teaching step of that PyTorch path on the CPU at B = 4096.
  silent_floor (in each roofline): the dominant hop launch re-timed with its source layer silenced, so that every
           gather is skipped: the kernel's floor without memory traffic, measured in the same run.
  gather_ceiling (in each roofline): the time the dominant hop's line gathers take at the device's gather rate
           (fc_gather_ceiling: random 128-byte lines from a slab of the same size, 8 lines per wave instruction,
           every CU issuing nothing else), measured in the same run, and the share of it the kernel reaches.
  decision_latency_gpu: one fc_forward of a 32-sample tile (a batch-1 decision padded), synchronised per call;
  bf16_b16384: the bfloat16-state core at B = 16384 (forward and teaching step) on the same network and on its
           Erdos-Renyi control;
  shipped_b4096: the reference's shipped network (its 3-hop graph and trained model.pt, copied into oracle/_ref/shipped
           as data) at B = 4096: forward and teaching step, the dominant hop's roofline, per layer the share of silent
           (row, tile) lines, and the reference's CPU forward on it (cpu_baseline, one core);
  whole_connectome_b1024: forward and teaching step at B = 1024 on a graph of the whole connectome's size (166,700
           neurons, 15.3M connections) indexed by FlyActor, with roofline fractions on the pruned hops' bytes;
  hophip_b4096: the HopCuda-style path at B = 4096: FlyActor's forward and a teaching step through PyTorch autograd
           and torch.optim.Adam, its hop products on the fh_* kernels (float32 and binary16 states);
  trainer: samples / s of the teaching trainer's own loop (flyguy_amd/flyguy_train, run as a child process on
           synthetic binary16 FLYD chunks of the same network: draw, gather, step, as its log reports them) at
           B = 4096, at the reference trainer's default B = 512, and with --bf16 1 at B = 16384.
One JSON line on stdout.  Only one GPU: --gpus N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes / s
METRIC = "decisions/sec (B=4096 fwd) + train samples/sec; % of MI355X HBM peak"


def algorithmic_bytes(s: dict, B: int, sz: int = 4) -> dict:
    """Compulsory traffic of the reference dataflow: every tensor written once and read once per consuming stage,
    sources read once per hop, structure once per batch (no widx: synthetic connections belong to one hop).
    Per hop launch and per whole batch, inference and train."""
    N = list(s["sizes"])
    E = [len(h["col"]) for h in s["hop"]]
    D = [int((h["drow"] >= 0).sum()) for h in s["hop"]]
    A, OD, K = s["n_act"], s["obs_dim"], s["hops"]
    hop_fwd = [N[k] * B * sz + D[k] * B * sz + N[k + 1] * B * sz + E[k] * 8 + (N[k + 1] + 1) * 4 for k in range(K)]
    infer = OD * B * 4 + 2 * N[0] * B * sz + s["fan"] * N[0] * 8 + N[0] * 4 + sum(hop_fwd) \
        + N[K] * B * sz + A * B * 4 + A * N[K] * 4
    if s["n_w"] < sum(E):        # strengths shared by several hops (the whole connectome): (col, widx) per connection
        infer += 4 * s["n_w"]    # (counted above as its 8 bytes) and each strength read once
    n_neurons_in_play = len(set(s["n0"].tolist()).union(*[set(h["nid"].tolist()) for h in s["hop"]]))
    n_params = s["n_w"] + 2 * n_neurons_in_play + s["n_s"] * s["fan"] + s["n_s"] + A * N[K] + A
    hop_bwd = []
    train = infer + sum(N[k] * B * sz for k in range(1, K + 1)) + 3 * A * B * 4 + A * B * 4 + 2 * N[K] * B * sz
    for k in range(K, 0, -1):
        b = 4 * N[k] * B * sz + (N[k] + N[k - 1]) * B * sz + (N[k] + N[k - 1]) * B * sz + 8 * E[k - 1] + 2 * D[k - 1] * B * sz
        hop_bwd.insert(0, b)
        train += b
    train += 3 * N[0] * B * sz + 2 * N[0] * B * 4 + OD * B * 4 + 36 * n_params
    return {"hop_fwd": hop_fwd, "hop_bwd": hop_bwd, "infer": infer, "train": train, "n_params": n_params}


def gather_ceiling(ms: float, row_of, B: int, rows: int, tiles: int) -> dict:
    """A hop launch against the device's gather ceiling, measured in this run (fc_gather_ceiling): the time the same
    number of 128-byte line gathers takes when every CU does nothing but gather, 8 lines per wave instruction and 8
    row indices loaded per step as the hop kernels do, from a slab of `rows` lines (per tile; `tiles` of them for a
    backward that takes two tiles per workgroup), each row drawn as a random connection's (row_of: the gathered row
    of every connection, so that rows come as often as the kernel gathers them).  The kernel gathers one line per
    connection and tile; frac is the ceiling's time over the kernel's, the share of the gather rate it reaches."""
    import numpy as np
    import torch
    from flyguy_amd._lib import call
    idx = torch.as_tensor(np.ascontiguousarray(row_of, dtype=np.int32)).cuda()
    ns = ctypes.c_double(0.0)
    call("fc_gather_ceiling", rows, tiles, idx.data_ptr(), idx.numel(), 5,
         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ctypes.byref(ns))
    lines = idx.numel() * (B // 32)
    at = lines * ns.value * 1e-6
    return {"slab_rows": rows, "tiles": tiles, "ns_per_line": round(ns.value, 6), "lines_per_launch": lines,
            "ms_at_ceiling": round(at, 4), "frac": round(at / ms, 4),
            "note": "fc_gather_ceiling: 128-byte lines of a tile's slab, rows drawn as the kernel's connections draw "
                    "them, 16 bytes a lane, 8 lines per wave instruction, every CU gathering and nothing else; the "
                    "bound the hop kernels meet before HBM bandwidth"}


def silent_floor(ms: float, floor_ms: float, E: int, B: int) -> dict:
    """A hop launch against the same launch with every source row silent, measured in this run: each gather then reads
    NO_ROW (zeros, no memory access), so that launch takes only the kernel's instruction issue and data return for
    the same lines (one 128-byte line per connection and 32-sample tile)."""
    lines = E * (B // 32)
    return {"ms": round(floor_ms, 4), "frac": round(floor_ms / ms, 4), "lines_per_launch": lines,
            "gathered_GB_per_s_at_floor": round(lines * 128 / (floor_ms * 1e-3) / 1e9, 1),
            "note": "the same kernel with the source layer's gains set to 0 (every gather skipped); 1 - frac is the "
                    "share of the launch spent waiting on the memory system"}


def kernel_sources_sha() -> str:
    """SHA-256 over the library's kernel sources without their comments and with runs of white space made one
    space: a counter run recorded for other code is stale, one recorded before a change of comments only is not."""
    import hashlib
    import re
    h = hashlib.sha256()
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flyguy_amd", "csrc")
    for n in sorted(os.listdir(d)):
        if n.endswith((".hip", ".h")):
            with open(os.path.join(d, n), encoding="utf-8") as fh:
                code = re.sub(r"/\*.*?\*/|//[^\n]*", " ", fh.read(), flags=re.S)
            h.update(n.encode() + b"\0" + " ".join(code.split()).encode())
    return h.hexdigest()


def host_info() -> dict:
    """The host the CPU baselines ran on: CPU model, logical CPUs, the CPUs this process may use, torch's threads."""
    model = ""
    try:
        with open("/proc/cpuinfo") as fh:
            model = next((l.split(":", 1)[1].strip() for l in fh if l.startswith("model name")), "")
    except OSError:
        pass
    import torch
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "torch_threads": torch.get_num_threads(), "pinning": "none (threads scheduled by the OS)"}


def cpu_baselines(s, params, sample: int, train_batch: int) -> tuple[dict | None, dict | None]:
    import numpy as np
    from oracle import refinfer
    rng = np.random.default_rng(1)
    fwd = None
    if refinfer.available() and sample > 0:
        ref = refinfer.RefInfer(s, params)
        obs = rng.standard_normal((sample, s["obs_dim"])).astype(np.float32)
        ref.forward(obs[:8])
        t0 = time.perf_counter()
        ref.forward(obs)
        dt = time.perf_counter() - t0
        fwd = {"value": sample / dt, "unit": "decisions/s", "cores": 1, "kind": "reference",
               "sample": f"{sample} batch-1 decisions of the same network through fly_infer.cpp (compiled from the "
                         f"reference), {dt:.1f} s"}
        # batch-1 decisions one call at a time, median latency over 300 (as the bot times them), of
        # the reference's compiled CPU forward and of this package's CPU decision library (include/fly_infer.h),
        # alternating decision by decision so that both meet the same clock and cache conditions
        from flyguy_amd.cpu_decisions import CpuDecisions
        ours = CpuDecisions(s, params)
        one = rng.standard_normal((300, s["obs_dim"])).astype(np.float32)
        fs = (("reference", ref), ("ours", ours))
        lat = {who: [] for who, _ in fs}
        for _, f in fs:
            f.forward(one[:5])
        for i in range(300):
            for who, f in (fs if i % 2 == 0 else fs[::-1]):
                t0 = time.perf_counter()
                f.forward(one[i:i + 1])
                lat[who].append(time.perf_counter() - t0)
        c1 = {who: {"median_ms": round(1e3 * float(np.median(v)), 4), "p90_ms": round(1e3 * float(np.percentile(v, 90)), 4)}
              for who, v in lat.items()}
        c1["decisions"] = 300
        c1["workload"] = "batch-1 fp32 decision (plug, 3 hops pushing only firing neurons, read-out), one call each, 1 core"
        # one decision on several host cores (fly_set_threads: bit-identical answers), up to every core this process
        # may use (at most 16, a GPU's share of the host)
        n_max = max(1, min(16, len(os.sched_getaffinity(0))))
        c1["ours_threads"] = {}
        for n_thr in sorted({n for n in (2, 4, 8, 16) if n <= n_max} | {n_max}):
            if n_thr < 2:
                continue
            f = CpuDecisions(s, params, threads=n_thr)
            f.forward(one[:20])
            lat = []
            for i in range(300):
                t0 = time.perf_counter()
                f.forward(one[i:i + 1])
                lat.append(time.perf_counter() - t0)
            c1["ours_threads"][str(n_thr)] = {"median_ms": round(1e3 * float(np.median(lat)), 4),
                                              "p90_ms": round(1e3 * float(np.percentile(lat, 90)), 4)}
            del f
        fwd["batch1"] = c1
        del ours
        # the same on every host core this process may use (at most 16, a GPU's share of the host): one handle per
        # thread (a handle is not thread-safe; ctypes releases the GIL during the call), sample / 4 decisions each
        n_thr = max(1, min(16, len(os.sched_getaffinity(0))))
        if n_thr > 1:
            import threading
            refs = [refinfer.RefInfer(s, params) for _ in range(n_thr)]
            per = max(1, sample // 4)
            xs = [rng.standard_normal((per, s["obs_dim"])).astype(np.float32) for _ in range(n_thr)]
            for r, x in zip(refs, xs):
                r.forward(x[:2])
            th = [threading.Thread(target=r.forward, args=(x,)) for r, x in zip(refs, xs)]
            t0 = time.perf_counter()
            for t in th:
                t.start()
            for t in th:
                t.join()
            dt = time.perf_counter() - t0
            fwd["all_cores"] = {"value": n_thr * per / dt, "unit": "decisions/s", "cores": n_thr,
                                "sample": f"{n_thr} threads x {per} batch-1 decisions, {dt:.1f} s"}
            del refs
        fwd["host"] = host_info()
    train = None
    if train_batch > 0:
        torch_fwd, train = torch_cpu_baselines(s, params, train_batch)
        if fwd is not None:
            fwd["torch_cpu"] = torch_fwd
    return fwd, train


def torch_cpu_baselines(s, params, batch: int) -> tuple[dict, dict]:
    """The reference's PyTorch CPU path (fly.py:252-305, this package's FlyActor over the same network): batch-1
    decisions (median of 30) and a batch forward through sparse CSR products of the current weights (the CPU
    decision library switched off, as FLYGUY_NATIVE=0 does), and one teaching step (forward, KL, backward through
    the sparse products' own backward, Adam over three rate groups) on `batch` samples, on torch's CPU threads."""
    import numpy as np
    import torch
    from flyguy_amd.fly import FlyActor
    rng = np.random.default_rng(2)
    f = FlyActor.from_structure(s, params)
    threads = torch.get_num_threads()
    old = os.environ.get("FLYGUY_NATIVE")
    os.environ["FLYGUY_NATIVE"] = "0"
    try:
        x = torch.as_tensor(rng.standard_normal((batch, s["obs_dim"])).astype(np.float32))
        with torch.no_grad():
            f(x[:1])
            lat = []
            for i in range(30):
                t0 = time.perf_counter()
                f(x[i:i + 1])
                lat.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            f(x)
            dt_f = time.perf_counter() - t0
    finally:
        if old is None:
            os.environ.pop("FLYGUY_NATIVE")
        else:
            os.environ["FLYGUY_NATIVE"] = old
    fwd = {"batch1_median_ms": round(1e3 * float(np.median(lat)), 3), "value": round(batch / dt_f, 1),
           "unit": "decisions/s", "cores": threads, "kind": "port",
           "sample": f"30 batch-1 decisions and one batch of {batch} through FlyActor's sparse CSR products "
                     f"(fly.py:252-284), {dt_f:.1f} s for the batch"}
    tl = torch.as_tensor((rng.standard_normal((batch, s["n_act"])) * 2).astype(np.float32))
    others = [p for n, p in f.named_parameters() if n not in ("w", "gain", "theta")]
    opt = torch.optim.Adam([{"params": [f.w], "lr": 1e-4}, {"params": [f.gain, f.theta], "lr": 3e-5},
                            {"params": others, "lr": 1e-4}])
    t0 = time.perf_counter()
    lt = torch.log_softmax(tl, -1)
    loss = (lt.exp() * (lt - torch.log_softmax(f(x), -1))).sum(-1).mean()
    opt.zero_grad()
    loss.backward()
    opt.step()
    dt = time.perf_counter() - t0
    train = {"value": round(batch / dt, 1), "unit": "samples/s", "cores": threads, "kind": "port",
             "sample": f"one teaching step (forward, KL, backward, Adam) on {batch} samples through FlyActor's "
                       f"PyTorch path on the CPU (sparse products with their own backward, fly.py:51-72), {dt:.1f} s"}
    return fwd, train


def trainer_leg(s, params, batches, steps: int) -> dict:
    """samples/s of flyguy_train's loop on synthetic chunks (3 chunks of 32,768 samples), from its last log line."""
    import re
    import struct
    import subprocess
    import tempfile
    from pathlib import Path

    import numpy as np
    from flyguy_amd.export import net_bytes, write_params

    exe = Path(__file__).resolve().parent / "flyguy_amd" / "flyguy_train"
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        tmp = Path(tmp)
        (tmp / "net.bin").write_bytes(net_bytes(s))
        write_params(params, tmp / "init.bin", 0)
        data = tmp / "data"
        data.mkdir()
        rng = np.random.default_rng(0)
        for i in range(3):
            n = 32768
            with open(data / f"chunk_{i:04d}.bin", "wb") as fh:
                fh.write(b"FLYD" + struct.pack("<qii", n, s["obs_dim"], s["n_act"]))
                fh.write(rng.standard_normal((n, s["obs_dim"]), dtype=np.float32).astype(np.float16).tobytes())
                fh.write((2 * rng.standard_normal((n, s["n_act"]), dtype=np.float32)).astype(np.float16).tobytes())
        for B, bf16 in batches:
            n_steps = steps * max(1, 4096 // B)
            key = f"B={B}" + (" bf16" if bf16 else "")
            cmd = [str(exe), str(tmp / "net.bin"), str(tmp / "init.bin"), str(data), str(tmp / f"out{B}{bf16}"),
                   "--batch", str(B), "--steps", str(n_steps), "--log", str(n_steps // 2), "--eval-batches", "0",
                   "--save-sec", "1e9", "--ring", "3", "--bf16", str(int(bf16))]
            print(f"# trainer {key}: {n_steps} steps", file=sys.stderr, flush=True)
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
            rates = [float(m.group(1)) for m in re.finditer(r"^step \d+ \| ([0-9.]+) samples/s", r.stdout, re.M)]
            if r.returncode != 0 or not rates:
                raise RuntimeError(f"flyguy_train failed ({r.returncode}): {r.stderr[-2000:]}")
            out[key] = {"value": rates[-1], "unit": "samples/s", "steps_timed": n_steps - n_steps // 2}
    return out


def bf16_leg(steps: int, warmup: int, B: int = 16384) -> dict:
    """The bfloat16-state core (fc_create_ex, FC_STATES_BF16) at B = 16384 on the synthetic network and on its
    Erdos-Renyi control (uniform in-degrees, same counts): forward decisions/s and teaching-step samples/s."""
    import numpy as np
    import torch
    from flyguy_amd._lib import call, lib, profile_read
    from flyguy_amd.export import net_bytes
    from flyguy_amd.synth import synth_3hop

    out = {}
    dev = torch.device("cuda:0")
    for kind in ("lognormal", "er"):
        s, params = synth_3hop(kind=kind)
        raw = net_bytes(s)
        core = lib().fc_create_ex(raw, len(raw), B, 1)
        if not core:
            call("fc_create_ex")
        tens = [torch.as_tensor(p).to(dev).contiguous() for p in params]
        ptrs = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in tens])
        call("fc_copy", core, 0, 1, ptrs)
        call("fc_copy", core, 1, 1, ptrs)
        g = torch.Generator(device=dev).manual_seed(0)
        obs = torch.randn(B, s["obs_dim"], device=dev, generator=g)
        teacher = torch.randn(B, s["n_act"], device=dev, generator=g) * 2.0
        logits = torch.empty(B, s["n_act"], device=dev)
        stats = torch.zeros(2, device=dev)
        ab = algorithmic_bytes(s, B, 2)
        res = {}
        for what, fn in (("forward", lambda: call("fc_forward", core, obs.data_ptr(), B, logits.data_ptr(), 0)),
                         ("train", lambda: call("fc_teach_step", core, obs.data_ptr(), teacher.data_ptr(), B, 1.0, 1e-4,
                                                3e-5, 1e-4, 0.0, 0.999, stats.data_ptr()))):
            for _ in range(warmup):
                fn()
            call("fc_profile", core, 1)             # per-stage times from a few calls outside the timed region
            profile_read(core, reset=True)
            for _ in range(min(steps, 3)):
                fn()
            torch.cuda.synchronize()
            prof = profile_read(core, reset=True)
            call("fc_profile", core, 0)
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            t = (time.perf_counter() - t0) / steps
            byts = ab["infer" if what == "forward" else "train"]
            res[what] = {"value": round(B / t, 1), "unit": "decisions/s" if what == "forward" else "samples/s",
                         "ms_per_step": round(1e3 * t, 4), "whole_batch_frac": round(byts / t / PEAK_HBM, 4),
                         "algorithmic_bytes": byts,
                         "stages_ms": {k: round(v[0] / v[1], 4) for k, v in prof.items()}}
        assert torch.isfinite(logits).all() and np.isfinite(float(stats[0]))
        out[kind] = res
        print(f"# bf16 B={B} {kind}: forward {res['forward']['ms_per_step']:.3f} ms ({res['forward']['value']:,.0f}/s), "
              f"train {res['train']['ms_per_step']:.3f} ms ({res['train']['value']:,.0f}/s)", file=sys.stderr, flush=True)
        lib().fc_free(core)
        del tens, obs, teacher, logits
        torch.cuda.empty_cache()
    return out


def connectome_leg(steps: int, warmup: int, B: int = 1024) -> dict:
    """The whole-connectome case (synthetic graph of 166,700 neurons and 15,283,167 connections, indexed by FlyActor)
    at B = 1024, float32: forward decisions/s and teaching-step samples/s."""
    import torch
    from flyguy_amd._lib import call, lib
    from flyguy_amd.export import net_bytes, params_from_torch, structure
    from flyguy_amd.fly import FlyActor
    from flyguy_amd.synth import whole_connectome

    torch.manual_seed(0)
    f = FlyActor(whole_connectome(), 517, 90, hops=3, fan=16)
    s = structure(f)
    params = params_from_torch(f, s)
    raw = net_bytes(s)
    core = lib().fc_create_from_memory(raw, len(raw), B)
    if not core:
        call("fc_create_from_memory")
    dev = torch.device("cuda:0")
    tens = [torch.as_tensor(p).to(dev).contiguous() for p in params]
    ptrs = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in tens])
    call("fc_copy", core, 0, 1, ptrs)
    call("fc_copy", core, 1, 1, ptrs)
    g = torch.Generator(device=dev).manual_seed(0)
    obs = torch.randn(B, s["obs_dim"], device=dev, generator=g)
    teacher = torch.randn(B, s["n_act"], device=dev, generator=g) * 2.0
    logits = torch.empty(B, s["n_act"], device=dev)
    stats = torch.zeros(2, device=dev)
    res = {"hop_connections": [len(h["col"]) for h in s["hop"]], "strengths": s["n_w"], "batch": B}
    ab = algorithmic_bytes(s, B)                # (of the pruned hops the library runs: the masked-out work is not done)
    for what, fn in (("forward", lambda: call("fc_forward", core, obs.data_ptr(), B, logits.data_ptr(), 0)),
                     ("train", lambda: call("fc_teach_step", core, obs.data_ptr(), teacher.data_ptr(), B, 1.0, 1e-4,
                                            3e-5, 1e-4, 0.0, 0.999, stats.data_ptr()))):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        t = (time.perf_counter() - t0) / steps
        byts = ab["infer" if what == "forward" else "train"]
        res[what] = {"value": round(B / t, 1), "unit": "decisions/s" if what == "forward" else "samples/s",
                     "ms_per_step": round(1e3 * t, 4), "algorithmic_bytes": byts,
                     "whole_batch_frac": round(byts / t / PEAK_HBM, 4)}
    print(f"# whole connectome B={B}: forward {res['forward']['ms_per_step']:.3f} ms, train "
          f"{res['train']['ms_per_step']:.3f} ms", file=sys.stderr, flush=True)
    lib().fc_free(core)
    return res


SHIPPED_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle", "_ref", "shipped")


def stage_timing(core, fn, stage: str, steps: int) -> tuple[float, float]:
    """`steps` calls of fn bracketed by synchronisations, with only `stage` bracketed by HIP events on the library's
    stream (fc_profile 2 + stage): (seconds for all calls, that stage's mean ms per launch)."""
    import torch
    from flyguy_amd._lib import STAGES, call, profile_read
    stage_of = {name: i for i, name in STAGES.items()}
    call("fc_profile", core, 2 + stage_of[stage])
    profile_read(core, reset=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    t = time.perf_counter() - t0
    prof = profile_read(core, reset=True)
    call("fc_profile", core, 0)
    tot, n = prof.get(stage, (0.0, 0))
    return t, (tot / n if n else float("nan"))


def stages_profiled(core, fn, n: int = 5) -> dict:
    """n calls with every stage bracketed by HIP events (fc_profile 1), outside any timed region: {stage: mean ms}."""
    import torch
    from flyguy_amd._lib import call, profile_read
    call("fc_profile", core, 1)
    profile_read(core, reset=True)
    for _ in range(n):
        fn()
    torch.cuda.synchronize()
    prof = profile_read(core, reset=True)
    call("fc_profile", core, 0)
    return {k: v[0] / v[1] for k, v in prof.items()}


def shipped_leg(steps: int, warmup: int, B: int = 4096, cpu_sample: int = 0) -> dict:
    """The shipped network: the reference's 3-hop graph (male_cns_min2_3hop.npz) with its trained actor (model.pt),
    indexed by FlyActor; forward and teaching step at B = 4096, observations ~N(0,1), teacher logits ~N(0,2).  The
    roofline of the dominant hop launch on the same compulsory-traffic model as the synthetic network (here with
    strengths shared between hops, so (col, widx) per connection and each strength read once), and per layer the share
    of (row, 32-sample tile) lines that are silent (h = 0 on the whole tile: gathers the library skips), plain and
    weighted by how often the next hop gathers each row.  cpu_sample > 0: the reference's CPU forward (fly_infer.cpp,
    oracle/_ref) on that many batch-1 decisions of the same network, one core, and the median of 300 one-call
    decisions, as its cpu_baseline."""
    import numpy as np
    import torch
    from flyguy_amd._lib import bwd_pairs, call, lib
    from flyguy_amd.export import actor_of, net_bytes, params_from_torch, structure

    graph, model = os.path.join(SHIPPED_DIR, "male_cns_min2_3hop.npz"), os.path.join(SHIPPED_DIR, "model.pt")
    if not (os.path.exists(graph) and os.path.exists(model)):
        return {"skipped": "the shipped graph and model.pt are not in oracle/_ref/shipped (make -C oracle shipped)"}
    f = actor_of(torch.load(model, map_location="cpu", weights_only=True), graph=graph)
    s = structure(f)
    params = params_from_torch(f, s)
    raw = net_bytes(s)
    core = lib().fc_create_from_memory(raw, len(raw), B)
    if not core:
        call("fc_create_from_memory")
    dev = torch.device("cuda:0")
    tens = [torch.as_tensor(p).to(dev).contiguous() for p in params]
    ptrs = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in tens])
    call("fc_copy", core, 0, 1, ptrs)
    call("fc_copy", core, 1, 1, ptrs)
    g = torch.Generator(device=dev).manual_seed(0)
    obs = torch.randn(B, s["obs_dim"], device=dev, generator=g)
    teacher = torch.randn(B, s["n_act"], device=dev, generator=g) * 2.0
    logits = torch.empty(B, s["n_act"], device=dev)
    stats = torch.zeros(2, device=dev)
    ab = algorithmic_bytes(s, B)
    res = {"batch": B, "rows": s["sizes"], "connections": [len(h["col"]) for h in s["hop"]], "strengths": s["n_w"],
           "redrive_rows": [int((h["drow"] >= 0).sum()) for h in s["hop"]], "weights": "bot/model.pt (trained)",
           "algorithmic_kB_per_decision": round(ab["infer"] / B / 1e3, 1),
           "algorithmic_kB_per_sample": round(ab["train"] / B / 1e3, 1)}

    def fwd():
        call("fc_forward", core, obs.data_ptr(), B, logits.data_ptr(), 0)

    def teach():
        call("fc_teach_step", core, obs.data_ptr(), teacher.data_ptr(), B, 1.0, 1e-4, 3e-5, 1e-4, 0.0, 0.999,
             stats.data_ptr())

    for _ in range(warmup):
        fwd()
    # silent lines per layer, of the forward the timed passes run (the weights do not change during the forwards)
    silent = []
    for layer in range(s["hops"] + 1):
        rows = s["sizes"][layer]
        h = torch.empty(rows, B, device=dev)
        call("fc_export_state", core, layer, 0, h.data_ptr(), B)
        quiet = (h.view(rows, B // 32, 32) <= 0).all(-1).float()
        entry = {"layer": layer, "silent_lines": round(float(quiet.mean()), 4)}
        if layer < s["hops"]:
            deg = torch.as_tensor(np.bincount(s["hop"][layer]["col"], minlength=rows).astype(np.float32), device=dev)
            entry["silent_gathers_next_hop"] = round(float((quiet * deg[:, None]).sum() / (deg.sum() * (B // 32))), 4)
        silent.append(entry)
        del h, quiet
    res["silent"] = silent
    for what, fn, kind in (("forward", fwd, "fwd"), ("train", teach, "bwd")):
        for _ in range(warmup):
            fn()
        prof = stages_profiled(core, fn)
        hops = {f"hop{k + 1} {kind}": prof.get(f"hop{k + 1} {kind}", 0.0) for k in range(s["hops"])}
        dom = max(hops, key=hops.get)
        t, dom_ms = stage_timing(core, fn, dom, steps)
        t /= steps
        k = int(dom[3]) - 1
        per_launch = ab["hop_fwd" if kind == "fwd" else "hop_bwd"][k]
        byts = ab["infer" if what == "forward" else "train"]
        kern = "k_fwd " if kind == "fwd" else ("k_bwd2 " if bwd_pairs(s["hop"][k]["crow"]) else "k_bwd ")
        res[what] = {"value": round(B / t, 1), "unit": "decisions/s" if what == "forward" else "samples/s",
                     "ms_per_step": round(1e3 * t, 4), "algorithmic_bytes": byts,
                     "whole_batch_frac": round(byts / t / PEAK_HBM, 4),
                     "roofline": {"bound": "hbm", "kernel": kern + dom, "mean_launch_ms": round(dom_ms, 4),
                                  "algorithmic_bytes_per_launch": per_launch,
                                  "achieved": round(per_launch / (dom_ms * 1e-3) / 1e9, 1), "peak": 8000.0,
                                  "unit": "GB/s", "frac": round(per_launch / (dom_ms * 1e-3) / PEAK_HBM, 4)},
                     "stages_ms": {k_: round(v, 4) for k_, v in prof.items()}}
    assert torch.isfinite(logits).all() and np.isfinite(float(stats[0]))
    print(f"# shipped network B={B}: forward {res['forward']['ms_per_step']:.3f} ms "
          f"({res['forward']['value']:,.0f}/s), train {res['train']['ms_per_step']:.3f} ms "
          f"({res['train']['value']:,.0f}/s); silent lines {[e['silent_lines'] for e in silent]}",
          file=sys.stderr, flush=True)
    lib().fc_free(core)
    del tens, obs, teacher, logits
    torch.cuda.empty_cache()
    if cpu_sample > 0:
        res["cpu_baseline"] = shipped_cpu_baseline(s, params, cpu_sample)
    return res


def shipped_cpu_baseline(s, params, sample: int) -> dict | None:
    """The reference's compiled CPU forward on the shipped network: `sample` batch-1 decisions in one call (one
    core), and one decision per call, median over 300."""
    import numpy as np
    from oracle import refinfer
    if not refinfer.available():
        return None
    ref = refinfer.RefInfer(s, params)
    rng = np.random.default_rng(3)
    obs = rng.standard_normal((sample, s["obs_dim"])).astype(np.float32)
    ref.forward(obs[:8])
    t0 = time.perf_counter()
    ref.forward(obs)
    dt = time.perf_counter() - t0
    lat = []
    for i in range(300):
        t1 = time.perf_counter()
        ref.forward(obs[i:i + 1])
        lat.append(time.perf_counter() - t1)
    return {"value": round(sample / dt, 1), "unit": "decisions/s", "cores": 1, "kind": "reference",
            "batch1_median_ms": round(1e3 * float(np.median(lat)), 4),
            "sample": f"{sample} batch-1 decisions of the shipped network (model.pt weights) through fly_infer.cpp "
                      f"(compiled from the reference), {dt:.1f} s; then 300 one-call decisions"}


def hophip_leg(s, params, steps: int, warmup: int, B: int = 4096) -> dict:
    """The HopCuda-style path (fly_cuda.py's, fly.py:170-185): FlyActor's own forward with its hop products on the
    fh_* kernels (HopHip, states [rows][B], PyTorch autograd between the hops), KL against teacher logits, backward
    and PyTorch's Adam, on the benchmark network at B = 4096; binary16 states too (kernel "cuda16")."""
    import torch
    from flyguy_amd.fly import FlyActor

    dev = torch.device("cuda:0")
    f = FlyActor.from_structure(s, params).to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    obs = torch.randn(B, s["obs_dim"], device=dev, generator=g)
    teacher = torch.randn(B, s["n_act"], device=dev, generator=g) * 2.0
    pt = torch.softmax(teacher, 1)
    opt = torch.optim.Adam(f.parameters(), lr=1e-4)

    def teach():
        lp = torch.log_softmax(f(obs), 1)
        loss = (pt * (torch.log(pt) - lp)).sum(1).mean()
        opt.zero_grad(set_to_none=False)
        loss.backward()
        opt.step()

    def decide():
        with torch.no_grad():
            f(obs)

    res = {"batch": B, "workload": "FlyActor forward / teaching step (KL, autograd backward, torch.optim.Adam) with "
                                   "its hop products on HopHip (float32: fh_to_tiled copies into fh_spmm_tiled / fh_spmm_bwd_tiled; "
                                   "binary16 states: fh_spmm_h / fh_spmm_bwd_h) and float32 activations on FireHip "
                                   "(fh_fire / fh_fire_bwd), states [rows][B]"}
    for kernel in ("hip", "cuda16"):
        f.kernel = kernel
        out = {}
        for what, fn in (("forward", decide), ("train", teach)):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            t = (time.perf_counter() - t0) / steps
            out[what] = {"value": round(B / t, 1), "unit": "decisions/s" if what == "forward" else "samples/s",
                         "ms_per_step": round(1e3 * t, 4)}
        res["fp32" if kernel == "hip" else "binary16_states"] = out
        print(f"# HopHip path B={B} kernel {kernel}: forward {out['forward']['ms_per_step']:.3f} ms, train "
              f"{out['train']['ms_per_step']:.3f} ms", file=sys.stderr, flush=True)
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=4096)
    ap.add_argument("--cpu-sample", type=int, default=8192)
    ap.add_argument("--cpu-train-batch", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--trainer-steps", type=int, default=60, help="teaching-trainer loop steps at B=4096 (0: skip)")
    ap.add_argument("--bf16-steps", type=int, default=10, help="timed bfloat16 B=16384 batches and steps (0: skip)")
    ap.add_argument("--latency-calls", type=int, default=200,
                    help="synchronised one-tile forwards timed for a single decision's latency (the first 20 untimed; 0: skip)")
    ap.add_argument("--hophip-steps", type=int, default=5,
                    help="timed steps of the HopCuda-style path (FlyActor over HopHip) at B=4096 (0: skip)")
    ap.add_argument("--connectome-steps", type=int, default=10,
                    help="timed whole-connectome B=1024 batches and steps (0: skip; its index build takes ~20 s)")
    ap.add_argument("--shipped-steps", type=int, default=20,
                    help="timed B=4096 batches and steps on the shipped network (graph + model.pt; 0: skip)")
    ap.add_argument("--no-floor", action="store_true",
                    help="skip the silent-source re-timing of the dominant hops (a counter run then sees only the "
                         "benchmark's own launches)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run 3 copies of 1 GiB (read 1 GiB, write 1 GiB each) so a counter run can scale "
                         "FETCH_SIZE / WRITE_SIZE by what they read for a copy of known size")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py runs on one GPU only (asked for {max(args.gpus, world)}): it measures one GPU's share of "
              f"the data-parallel path (a batch of samples); the gradient exchange between GPUs is not measured here",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch
    from flyguy_amd._lib import STAGES, bwd_pairs, call, lib, profile_read
    from flyguy_amd.export import net_bytes
    from flyguy_amd.synth import synth_3hop

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    B, K, W = args.batch, args.steps, args.warmup
    t_setup = time.perf_counter()
    s, params = synth_3hop()
    raw = net_bytes(s)
    L = lib()
    core = L.fc_create_from_memory(raw, len(raw), B)
    if not core:
        call("fc_create_from_memory")
    dev = torch.device("cuda:0")
    tens = [torch.as_tensor(p).to(dev).contiguous() for p in params]
    ptrs = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in tens])
    call("fc_copy", core, 0, 1, ptrs)
    call("fc_copy", core, 1, 1, ptrs)
    g = torch.Generator(device=dev).manual_seed(0)
    obs = torch.randn(B, s["obs_dim"], device=dev, generator=g)
    teacher = torch.randn(B, s["n_act"], device=dev, generator=g) * 2.0
    logits = torch.empty(B, s["n_act"], device=dev)
    stats = torch.zeros(2, device=dev)
    torch.cuda.synchronize()
    print(f"# set-up {time.perf_counter() - t_setup:.1f} s", file=sys.stderr, flush=True)
    ab = algorithmic_bytes(s, B)

    stage_of = {name: i for i, name in STAGES.items()}

    def stage_ms(prof, name):
        tot, n = prof.get(name, (0.0, 0))
        return tot / n if n else float("nan")

    def profiled(fn, n=5):
        """n calls with every stage bracketed by HIP events (fc_profile 1): the per-stage times, which pick the
        dominant kernel; outside the timed region, since ~30 events per call lengthen it by about 3%"""
        call("fc_profile", core, 1)
        profile_read(core, reset=True)
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        prof = profile_read(core, reset=True)
        call("fc_profile", core, 0)
        return prof

    def timed(fn, stage):
        """K calls bracketed by synchronisations; only `stage` is bracketed by HIP events on the library's stream
        (fc_profile 2 + stage), so its mean launch duration comes from the timed region itself"""
        call("fc_profile", core, 2 + stage_of[stage])
        profile_read(core, reset=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(K):
            fn()
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        prof = profile_read(core, reset=True)
        call("fc_profile", core, 0)
        return t, stage_ms(prof, stage)

    def dominant(prof, kind):
        hops = {f"hop{k + 1} {kind}": stage_ms(prof, f"hop{k + 1} {kind}") for k in range(s["hops"])}
        return max(hops, key=hops.get)

    # ---- batched forward
    def fwd():
        call("fc_forward", core, obs.data_ptr(), B, logits.data_ptr(), 0)
    for _ in range(W):
        fwd()
    torch.cuda.synchronize()
    prof_fwd = profiled(fwd)
    dom_f = dominant(prof_fwd, "fwd")
    t_fwd, dom_f_ms = timed(fwd, dom_f)
    assert torch.isfinite(logits).all()
    ms_fwd = 1e3 * t_fwd / K
    dps = B * K / t_fwd
    print(f"# forward: {ms_fwd:.3f} ms / batch of {B}, {dps:,.0f} decisions/s", file=sys.stderr, flush=True)

    # ---- one decision on the GPU: batch 1 padded to one 32-sample tile (NativeFlyActor's rule), each call
    # synchronised, as a bot deciding one car at a time would run it
    lat = []
    for _ in range(args.latency_calls):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        call("fc_forward", core, obs.data_ptr(), 32, logits.data_ptr(), 0)
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t0)
    lat_b32 = None
    if len(lat) > 20:
        lat_b32 = {"median_ms": round(1e3 * float(np.median(lat[20:])), 4),
                   "p90_ms": round(1e3 * float(np.percentile(lat[20:], 90)), 4), "calls": len(lat) - 20,
                   "workload": "fc_forward of one 32-sample tile (a batch-1 decision padded), synchronised per call"}
        print(f"# one decision (B=32 tile) on the GPU: {lat_b32['median_ms']:.3f} ms median", file=sys.stderr, flush=True)

    # ---- teaching step
    def teach():
        call("fc_teach_step", core, obs.data_ptr(), teacher.data_ptr(), B, 1.0, 1e-4, 3e-5, 1e-4, 0.0, 0.999, stats.data_ptr())
    for _ in range(W):
        teach()
    torch.cuda.synchronize()
    prof_train = profiled(teach)
    dom_b = dominant(prof_train, "bwd")
    t_train, dom_b_ms = timed(teach, dom_b)
    assert np.isfinite(float(stats[0]))
    kl = float(stats[0]) / B
    ms_train = 1e3 * t_train / K
    sps = B * K / t_train
    print(f"# train: {ms_train:.3f} ms / step of {B}, {sps:,.0f} samples/s, kl {kl:.4f}",
          file=sys.stderr, flush=True)

    # dominant kernels: the largest hop of the forward, the largest hop backward of the step, timed in the timed region
    kf = int(dom_f[3]) - 1
    ach_f = ab["hop_fwd"][kf] / (dom_f_ms * 1e-3)
    kb = int(dom_b[3]) - 1
    ach_b = ab["hop_bwd"][kb] / (dom_b_ms * 1e-3)
    traffic, traffic_b, traffic_note = None, None, "no counter run recorded"
    tfile = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic_synth3hop_b4096.json")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            tj = json.load(fh)
        if tj.get("sources_sha256") == kernel_sources_sha():
            traffic, traffic_note = tj.get("k_fwd " + dom_f), tj.get("command", "")
            traffic_b = tj.get(("k_bwd2 " if bwd_pairs(s["hop"][kb]["crow"]) else "k_bwd ") + dom_b)
        else:
            traffic_note = "the counter run predates the current kernel sources (profiles/traffic_synth3hop_b4096.json)"

    # the dominant hops' floors: the same launches with their source layer silenced (gains 0, so every gather is
    # skipped), forward and teaching step (rate 0: the weights stay as they are), then the weights restored
    def layer_neurons(layer):
        return np.asarray(s["n0"] if layer == 0 else s["hop"][layer - 1]["nid"], np.int64)
    floor_f = floor_b = ceil_f = ceil_b = None
    if not args.no_floor:
        quiet = params[1].copy()
        for layer in {kf, kb}:
            quiet[layer_neurons(layer)] = 0.0
        gq = torch.as_tensor(quiet).to(dev)
        call("fc_copy", core, 0, 1, (ctypes.c_void_p * 7)(None, gq.data_ptr(), None, None, None, None, None))
        for _ in range(W):
            fwd()
        _, quiet_f_ms = timed(fwd, dom_f)

        def teach_still():
            call("fc_teach_step", core, obs.data_ptr(), teacher.data_ptr(), B, 1.0, 0.0, 0.0, 0.0, 0.0, 0.999,
                 stats.data_ptr())
        for _ in range(W):
            teach_still()
        _, quiet_b_ms = timed(teach_still, dom_b)
        call("fc_copy", core, 0, 1, ptrs)
        floor_f = silent_floor(dom_f_ms, quiet_f_ms, len(s["hop"][kf]["col"]), B)
        floor_b = silent_floor(dom_b_ms, quiet_b_ms, len(s["hop"][kb]["col"]), B)
        # the gather ceilings: the forward gathers the source layer's slab, the backward the hop's own layer (gz), two
        # tiles' slabs at once when it takes two tiles per workgroup
        ceil_f = gather_ceiling(dom_f_ms, s["hop"][kf]["col"], B, s["sizes"][kf], 1)
        crow_b = np.asarray(s["hop"][kb]["crow"])
        ceil_b = gather_ceiling(dom_b_ms, np.repeat(np.arange(len(crow_b) - 1), np.diff(crow_b)), B,
                                s["sizes"][kb + 1], 2 if bwd_pairs(s["hop"][kb]["crow"]) else 1)
        print(f"# floors: {dom_f} {floor_f['ms']:.3f} of {dom_f_ms:.3f} ms, {dom_b} {floor_b['ms']:.3f} of "
              f"{dom_b_ms:.3f} ms", file=sys.stderr, flush=True)

    cpu_f = cpu_t = None
    if not args.no_cpu:
        cpu_f, cpu_t = cpu_baselines(s, params, args.cpu_sample, args.cpu_train_batch)
    L.fc_free(core)
    core = None
    bf16 = None
    if args.bf16_steps > 0:
        bf16 = bf16_leg(args.bf16_steps, W)
        bf16["workload"] = ("bfloat16 states (x, drive, every layer's h, gathered gz), float32 sums, gradients and "
                               "Adam; B=16384; the synthetic network (lognormal in-degree) and its Erdos-Renyi control")
    shipped = None
    if args.shipped_steps > 0:
        shipped = shipped_leg(args.shipped_steps, W, B, 0 if args.no_cpu else min(args.cpu_sample, 2048))
    connectome = connectome_leg(args.connectome_steps, W) if args.connectome_steps > 0 else None
    hophip = hophip_leg(s, params, args.hophip_steps, W) if args.hophip_steps > 0 else None
    trainer = None
    if args.trainer_steps > 0:
        trainer = trainer_leg(s, params, ((4096, False), (512, False), (16384, True)), args.trainer_steps)
        trainer["workload"] = ("flyguy_train loop on synthetic binary16 FLYD chunks (3 x 32,768 samples, ring of 3) of "
                               "the same network: draw, gather, teaching step, samples/s from its own log; float32 "
                               "at B=4096 and 512, and --bf16 1 (bfloat16 states and edge weights) at B=16384")
        trainer["reference_published"] = {"value": 10300, "unit": "samples/s", "batch": 512,
                                          "hardware": "RTX 4070 laptop"}
        print(f"# trainer: {trainer['B=4096']['value']:,.0f} samples/s at B=4096, "
              f"{trainer['B=512']['value']:,.0f} at B=512, {trainer['B=16384 bf16']['value']:,.0f} at B=16384 bf16",
              file=sys.stderr, flush=True)

    line = {
        "metric": METRIC, "value": round(dps, 1), "unit": "decisions/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_fwd, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic: random 3-hop network of the benchmark shape, obs ~N(0,1), teacher ~N(0,2)",
        "config": {"workload": "batched fp32 inference (plug, 3 sparse hops, read-out) on the synthetic 3-hop network "
                               "16894/46393/37748/1332 rows, 1.2M/1.5M/292,734 connections, B=4096",
                   "batch": B, "rows": s["sizes"], "connections": [len(h["col"]) for h in s["hop"]],
                   "redrive_rows": [int((h["drow"] >= 0).sum()) for h in s["hop"]]},
        "roofline": {"bound": "hbm", "kernel": "k_fwd " + dom_f, "achieved": round(ach_f / 1e9, 1), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(ach_f / PEAK_HBM, 4), "traffic": traffic,
                     "traffic_source": traffic_note,
                     "algorithmic_bytes_per_launch": ab["hop_fwd"][kf], "mean_launch_ms": round(dom_f_ms, 4),
                     "whole_batch_frac": round(ab["infer"] / (t_fwd / K) / PEAK_HBM, 4),
                     "whole_batch_algorithmic_bytes": ab["infer"],
                     "silent_floor": floor_f, "gather_ceiling": ceil_f},
        "decision_latency_gpu": lat_b32,
        "cpu_baseline": cpu_f,
        "train": {"value": round(sps, 1), "unit": "samples/s", "ms_per_step": round(ms_train, 4),
                  "workload": "fp32 teaching step: forward, KL(teacher||student) over 90 actions, fused backward, "
                              "Adam (lr 1e-4, betas 0.9/0.999) + running average over 2,992,734 strengths, gains, "
                              "thresholds and plugs, B=4096",
                  "roofline": {"bound": "hbm", "kernel": ("k_bwd2 " if bwd_pairs(s["hop"][kb]["crow"]) else "k_bwd ")
                                                         + dom_b, "achieved": round(ach_b / 1e9, 1),
                               "peak": 8000.0, "unit": "GB/s", "frac": round(ach_b / PEAK_HBM, 4),
                               "traffic": traffic_b, "traffic_source": traffic_note,
                               "algorithmic_bytes_per_launch": ab["hop_bwd"][kb],
                               "mean_launch_ms": round(dom_b_ms, 4),
                               "whole_step_frac": round(ab["train"] / (t_train / K) / PEAK_HBM, 4),
                               "whole_step_algorithmic_bytes": ab["train"],
                               "silent_floor": floor_b, "gather_ceiling": ceil_b},
                  "cpu_baseline": cpu_t},
        "trainer": trainer,
        "bf16_b16384": bf16,
        "shipped_b4096": shipped,
        "whole_connectome_b1024": connectome,
        "hophip_b4096": hophip,
        "stages_ms": {"forward": {k: round(v[0] / v[1], 4) for k, v in prof_fwd.items()},
                      "train": {k: round(v[0] / v[1], 4) for k, v in prof_train.items()}},
    }
    print(json.dumps(line), flush=True)
    if args.calibrate:
        a = torch.ones(1 << 28, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
