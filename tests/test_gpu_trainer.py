"""The teaching trainer on the GPU: its data path, survey and revive surgery against the oracle, and whole runs of
the trainer against a replay of the same steps through the library's teaching step.

Bars: the batch gather is bit-exact (binary16 -> float32 is exact); survey counts are exact against the states the
library exports, and the sums of squares and loss sums within 1e-5 of the float64 oracle; the revive surgery marks,
signs and resets exactly what the oracle's restatement does, and scales within 1e-4 (its scale factors come from
float32 surveys); the network's output is bit-identical before and after a revive.  A trainer run leaves weights,
running average and Adam state bit-identical to the replay (the same kernels on the same batches).  On a
bfloat16-state handle: survey counts exact against its own stored states, sums of squares and the loss sum within
1e-3 of the bfloat16 oracle (oracle/core16.py); a --bf16 trainer run bit-identical to its replay."""
from __future__ import annotations

import ctypes
import os
import re
import struct
import subprocess

import numpy as np
import pytest
import torch

from conftest import lively, toy
from flyguy_amd._lib import call, lib
from flyguy_amd.export import net_bytes, param_sizes, params_from_torch, structure, write_params
from flyguy_amd.fly import FlyActor
from gpu_helpers import Core, rel, say
from oracle import trainer as ot
from oracle.core16 import Core16, bf16
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu
OD, NA = 517, 90


def toy_net(name="a", hops=3, fan=5, seed=0):
    torch.manual_seed(seed)
    f = lively(FlyActor(toy(name), OD, NA, hops=hops, fan=fan), seed)
    s = structure(f)
    return s, params_from_torch(f, s)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def test_gather16_and_unpack16(gpu_lib):
    rng = np.random.default_rng(0)
    sizes = [37, 5, 64]
    obs = [rng.standard_normal((n, OD)).astype(np.float16) for n in sizes]
    lg = [(2 * rng.standard_normal((n, NA))).astype(np.float16) for n in sizes]
    obs[0][0, :5] = [np.inf, -np.inf, 6e-8, -0.0, 65504]          # infinities, a subnormal, -0, the largest finite
    d_obs = [torch.as_tensor(a).cuda() for a in obs]
    d_lg = [torch.as_tensor(a).cuda() for a in lg]
    tab_o = torch.tensor([t.data_ptr() for t in d_obs], dtype=torch.int64, device="cuda")
    tab_l = torch.tensor([t.data_ptr() for t in d_lg], dtype=torch.int64, device="cuda")
    n_tab = torch.tensor(sizes, dtype=torch.int64, device="cuda")
    B = 64
    sel = ot.draws(7, sizes, B, 1).astype(np.int32)
    sel[0] = (0, 0)
    bad = {5: (3, 0), 9: (1, 5), 11: (2, -1)}                      # chunk past the table, sample past a chunk's end
    for i, v in bad.items():
        sel[i] = v
    d_sel = torch.as_tensor(sel).cuda()
    x = torch.empty(B, OD, device="cuda")
    t = torch.empty(B, NA, device="cuda")
    say("fd_gather16", B, sizes)
    call("fd_gather16", tab_o.data_ptr(), tab_l.data_ptr(), n_tab.data_ptr(), len(sizes), d_sel.data_ptr(), B, OD, NA,
         x.data_ptr(), t.data_ptr(), _stream())
    gx, gt = x.cpu().numpy(), t.cpu().numpy()
    for i in range(B):
        if i in bad:
            assert np.isnan(gx[i]).all() and np.isnan(gt[i]).all()
            continue
        c, s = sel[i]
        assert np.array_equal(gx[i].view(np.uint32), obs[c][s].astype(np.float32).view(np.uint32))
        assert np.array_equal(gt[i].view(np.uint32), lg[c][s].astype(np.float32).view(np.uint32))
    # the staged form [B][obs_dim + n_act]
    good = [i for i in range(B) if i not in bad]
    st = np.stack([np.concatenate([obs[sel[i][0]][sel[i][1]], lg[sel[i][0]][sel[i][1]]]) for i in good])
    d_st = torch.as_tensor(st).cuda()
    x2 = torch.empty(len(good), OD, device="cuda")
    t2 = torch.empty(len(good), NA, device="cuda")
    call("fd_unpack16", d_st.data_ptr(), len(good), OD, NA, x2.data_ptr(), t2.data_ptr(), _stream())
    assert np.array_equal(x2.cpu().numpy().view(np.uint32), gx[good].view(np.uint32))
    assert np.array_equal(t2.cpu().numpy().view(np.uint32), gt[good].view(np.uint32))


def _layers(h):
    sizes = (ctypes.c_int * 16)()
    n = call("fc_layers", h, sizes, 16)
    return list(sizes[:n])


def _survey_read(h, rows):
    cnt = np.zeros(rows, np.int32)
    sq = np.zeros(rows, np.float32)
    stats = (ctypes.c_double * 3)()
    assert call("fc_survey_read", h, cnt.ctypes.data, sq.ctypes.data, stats) == rows
    return cnt, sq, list(stats)


def _oracle_survey(s, params, batches):
    """cnt, sq, samples, kl sum, agree sum, max |h| near zero per row over `batches` [(obs, teacher)] in float64."""
    o = Oracle(net_bytes(s), params, "f64")
    cnt = sq = None
    kl = agree = 0.0
    near = np.zeros(sum(s["sizes"]), bool)
    for obs, tl in batches:
        logits = o.forward(obs)
        _, k, a = o.loss(logits, tl, 1.0)
        kl += k
        agree += a
        states = [(o.state(0, 0, s["sizes"][0]), None)]
        states += [(o.state(k2, 0, s["sizes"][k2]), o.state(k2, 1, s["sizes"][k2])) for k2 in range(1, s["hops"] + 1)]
        c, q = ot.survey_sums(states)
        cnt = c if cnt is None else cnt + c
        sq = q if sq is None else sq + q
        near |= np.concatenate([((h > 0) & (h < 1e-4)).any(1) for h, _ in states])
    return cnt, sq, len(batches) * batches[0][0].shape[0], kl, agree, near


def test_survey_matches_oracle(gpu_lib):
    s, params = toy_net("a", 3, 5)
    B = 64
    core = Core(s, params, max_batch=B)
    ema = [p * np.float32(0.7) for p in params]
    core.set(1, ema)
    rows = _layers(core.h)
    assert rows == list(s["sizes"])
    R = sum(rows)
    rng = np.random.default_rng(3)
    batches = [(rng.standard_normal((B, OD)).astype(np.float32), (2 * rng.standard_normal((B, NA))).astype(np.float32))
               for _ in range(2)]
    for use_ema, P in ((0, params), (1, ema)):
        mine = np.zeros(R, np.int64)
        for i, (obs, tl) in enumerate(batches):
            x, t = torch.as_tensor(obs).cuda(), torch.as_tensor(tl).cuda()
            say("fc_survey", use_ema, i)
            call("fc_survey", core.h, x.data_ptr(), t.data_ptr(), B, use_ema, 1.0, int(i == 0))
            hs = [core.state(k, 0, rows[k], B) for k in range(len(rows))]
            mine += np.concatenate([(h > 0).sum(1) for h in hs])
        cnt, sq, (kl, agree, samples) = _survey_read(core.h, R)
        assert samples == 2 * B
        assert np.array_equal(cnt, mine)                               # the counts of the library's own states
        ocnt, osq, _, okl, oagree, near = _oracle_survey(s, P, batches)
        assert np.array_equal(cnt[~near], ocnt[~near]), int((cnt != ocnt).sum())
        assert (sq[:rows[0]] == 0).all()
        assert rel(sq, osq) <= 1e-5, rel(sq, osq)
        assert abs(kl - okl) <= 1e-5 * max(abs(okl), 1.0), (kl, okl)
        assert abs(agree - oagree) <= 2, (agree, oagree)


def test_bf16_survey_matches_oracle(gpu_lib):
    """Surveys of a bfloat16-state handle count and square its stored bfloat16 states (oracle/core16.py)."""
    s, params = toy_net("b", 3, 8, seed=3)
    B = 128
    core = Core(s, params, max_batch=B, flags=1)
    rows = _layers(core.h)
    R = sum(rows)
    rng = np.random.default_rng(5)
    batches = [(rng.standard_normal((B, OD)).astype(np.float32), (2 * rng.standard_normal((B, NA))).astype(np.float32))
               for _ in range(2)]
    o = Core16(s, params)
    mine = np.zeros(R, np.int64)
    ocnt, osq = np.zeros(R, np.int64), np.zeros(R)
    near = np.zeros(R, bool)
    okl = 0.0
    for i, (obs, tl) in enumerate(batches):
        x, t = torch.as_tensor(obs).cuda(), torch.as_tensor(tl).cuda()
        say("bf16 fc_survey", i)
        call("fc_survey", core.h, x.data_ptr(), t.data_ptr(), B, 0, 1.0, int(i == 0))
        mine += np.concatenate([(core.state(k, 0, rows[k], B) > 0).sum(1) for k in range(len(rows))])
        lg = o.forward(obs)
        states = [(o.states[0][0], None)] + [(h, bf16(z)) for h, z in o.states[1:]]
        c, q = ot.survey_sums(states)
        ocnt += c
        osq += q
        near |= np.concatenate([((h > 0) & (h < 1e-2)).any(1) for h, _ in states])
        lp = lg - lg.max(1, keepdims=True)
        lp = lp - np.log(np.exp(lp).sum(1, keepdims=True))
        tp = tl - tl.max(1, keepdims=True)
        tp = tp - np.log(np.exp(tp).sum(1, keepdims=True))
        okl += float((np.exp(tp) * (tp - lp)).sum())
    cnt, sq, (kl, agree, samples) = _survey_read(core.h, R)
    assert samples == 2 * B
    assert np.array_equal(cnt, mine)                                   # the counts of the library's own states
    assert np.array_equal(cnt[~near], ocnt[~near]), int((cnt != ocnt).sum())
    assert (sq[:rows[0]] == 0).all()
    assert rel(sq, osq) <= 1e-3, rel(sq, osq)
    assert abs(kl - okl) <= 1e-3 * max(abs(okl), 1.0), (kl, okl)


def _dead_case(seed=0):
    """A toy network with silent neurons: gain 0 for a tenth of the neurons past the sensory layer."""
    s, params = toy_net("a", 3, 5, seed)
    rng = np.random.default_rng(seed)
    sens = set(np.asarray(s["n0"]).tolist())
    cand = sorted({int(g) for h in s["hop"] for g in h["nid"]} - sens)
    dead = rng.choice(cand, max(3, len(cand) // 10), replace=False)
    params[1][dead] = 0.0
    return s, params, dead


def test_revive_matches_oracle(gpu_lib):
    s, params, forced = _dead_case(0)
    B, nb = 64, 2
    core = Core(s, params, max_batch=B)
    rng = np.random.default_rng(5)
    m = [rng.standard_normal(n).astype(np.float32) * 1e-3 for n in param_sizes(s)]
    v = [np.abs(rng.standard_normal(n)).astype(np.float32) * 1e-6 for n in param_sizes(s)]
    for a in v:
        a[::7] = 0                                                     # median_positive skips zeros
    ema = [p + np.float32(0.01) for p in params]
    core.set(1, ema)
    core.set(2, m)
    core.set(3, v)
    obs = rng.standard_normal((nb * B, OD)).astype(np.float32)
    tl = (2 * rng.standard_normal((nb * B, NA))).astype(np.float32)
    d_obs, d_tl = torch.as_tensor(obs).cuda(), torch.as_tensor(tl).cuda()
    before = core.forward(obs[:B])
    rep = ctypes.create_string_buffer(1024)
    seed, target = 99991 * 12 + 3, 0.4
    say("fc_revive", s["n_neurons"], len(forced))
    n = call("fc_revive", core.h, d_obs.data_ptr(), d_tl.data_ptr(), B, nb, target, seed, 12, rep, 1024)
    report = rep.value.decode()
    say(report)
    after = core.forward(obs[:B])
    assert np.array_equal(before.view(np.uint32), after.view(np.uint32))      # the output unchanged, bit for bit
    k = re.search(r"kl ([-0-9.]+) -> ([-0-9.]+) \(must be equal\)", report)
    assert k and k.group(1) == k.group(2)
    P, E, M, V = (core.get(i) for i in range(4))

    batches = [(obs[i * B:(i + 1) * B], tl[i * B:(i + 1) * B]) for i in range(nb)]

    def survey(p):
        c, q, smp, kl, _, _ = _oracle_survey(s, p, batches)
        return c, q, smp, kl / smp
    want = ot.revive(s, params, ema, m, v, survey, target, seed)
    assert n == want["n_dead"] and n >= len(forced)
    assert f"{want['n_dead']} of {want['n_play']} neurons" in report
    assert f"new sign for {want['n_in']} incoming" in report and f"zero for {want['n_out']} outgoing" in report
    mark = want["mark"]
    W, W0 = P[0], want["P"][0]
    assert np.array_equal(W[mark == 0], params[0][mark == 0])
    assert (W[mark == 2] == 0).all() and (W0[mark == 2] == 0).all()
    assert np.array_equal(np.sign(W[mark == 1]), np.sign(W0[mark == 1]))
    assert rel(W[mark == 1], W0[mark == 1]) <= 1e-4
    for i in (1, 2, 3, 4, 5, 6):
        assert np.array_equal(P[i], want["P"][i]), i
    assert np.array_equal(E[0][mark == 0], ema[0][mark == 0]) and rel(E[0], want["EMA"][0]) <= 1e-4
    for i in range(1, 7):
        assert np.array_equal(E[i], want["EMA"][i]), i
    for i in range(7):
        assert np.array_equal(M[i], want["M"][i]) and np.array_equal(V[i], want["V"][i]), i
    # every revived neuron fires now (the surgery's purpose), as the oracle's surveys also find
    assert f"| {want['still']} still silent" in report


def test_bf16_revive_keeps_the_output(gpu_lib):
    """fc_revive on a bfloat16-state handle: the network's output is bit-identical before and after, the silent
    neurons are those of the library's own stored states, and every connection the surgery touches gets what the
    rules say (a new sign into a silent neuron, zero from a silent one into a live one, gain 1 and threshold -4)."""
    s, params, forced = _dead_case(2)
    B, nb = 64, 2
    core = Core(s, params, max_batch=B, flags=1)
    rng = np.random.default_rng(6)
    obs = rng.standard_normal((nb * B, OD)).astype(np.float32)
    tl = (2 * rng.standard_normal((nb * B, NA))).astype(np.float32)
    d_obs, d_tl = torch.as_tensor(obs).cuda(), torch.as_tensor(tl).cuda()
    # the silent neurons, from the library's own stored states over the same batches
    fired = np.zeros(s["n_neurons"], np.int64)
    play = np.zeros(s["n_neurons"], bool)
    sens = np.zeros(s["n_neurons"], bool)
    sens[np.asarray(s["n0"])] = True
    for i in range(nb):
        core.forward(obs[i * B:(i + 1) * B])
        for k, h in enumerate(s["hop"], start=1):
            nid = np.asarray(h["nid"])
            play[nid] = True
            np.add.at(fired, nid, (core.state(k, 0, len(nid), B) > 0).sum(1))
    dead = play & ~sens & (fired == 0)
    before = core.forward(obs[:B])
    rep = ctypes.create_string_buffer(1024)
    say("bf16 fc_revive", len(forced))
    n = call("fc_revive", core.h, d_obs.data_ptr(), d_tl.data_ptr(), B, nb, 0.4, 99991 * 5 + 3, 5, rep, 1024)
    report = rep.value.decode()
    say(report)
    after = core.forward(obs[:B])
    assert np.array_equal(before.view(np.uint32), after.view(np.uint32))
    assert n == int(dead.sum()) and n >= len(forced)
    W = core.get(0)[0]
    pre, post = np.full(s["n_w"], -1), np.full(s["n_w"], -1)
    below = np.asarray(s["n0"])
    for h in s["hop"]:
        nid = np.asarray(h["nid"])
        tgt = np.repeat(np.arange(len(nid)), np.diff(h["crow"]))
        pre[np.asarray(h["widx"])] = below[np.asarray(h["col"])]
        post[np.asarray(h["widx"])] = nid[tgt]
        below = nid
    into = dead[post]
    out_of = dead[pre] & ~into
    assert (W[out_of] == 0).all()
    assert np.array_equal(W[~into & ~out_of], params[0][~into & ~out_of])
    assert (np.abs(W[into]) > 0).all()
    gain, theta = core.get(0)[1], core.get(0)[2]
    assert (gain[dead] == 1).all() and (theta[dead] == -4).all()


# ---------------------------------------------------------------------------------------------------- whole runs
def _setup(tmp_path, s, params, sizes=(50, 70, 90), seed=11):
    d = tmp_path / "data"
    d.mkdir()
    rng = np.random.default_rng(seed)
    chunks = {}
    t0 = 1_700_000_000 * 10 ** 9
    for i, n in enumerate(sizes):
        name = f"chunk_{i:04d}.bin"
        o = rng.standard_normal((n, OD)).astype(np.float16)
        l = (2 * rng.standard_normal((n, NA))).astype(np.float16)
        ot.write_chunk(d / name, o, l)
        os.utime(d / name, ns=(t0 + i * 10 ** 9, t0 + i * 10 ** 9))
        chunks[name] = (o.astype(np.float32), l.astype(np.float32))
    (tmp_path / "net.bin").write_bytes(net_bytes(s))
    write_params(params, tmp_path / "init.bin", 0)
    return d, chunks


def _run(*args):
    argv = [b"flyguy_train"] + [str(a).encode() for a in args]
    arr = (ctypes.c_char_p * len(argv))(*argv)
    say("ft_main", " ".join(str(a) for a in args[4:]))
    return lib().ft_main(len(argv), arr)


def _replay(core, ring, chunks, g, steps, first, B, lr, lrn, lrp, lmin, hl, clip, ema, it=1.0):
    sizes = [chunks[n][0].shape[0] for n in ring]
    for k in range(steps):
        sel = ot.draw(g, sizes, B)
        obs = np.stack([chunks[ring[c]][0][i] for c, i in sel])
        tl = np.stack([chunks[ring[c]][1][i] for c, i in sel])
        x, t = torch.as_tensor(obs).cuda(), torch.as_tensor(tl).cuda()
        l = ot.lr(first + k + 1, lr, lrn, lrp, lmin, hl)
        call("fc_teach_step", core.h, x.data_ptr(), t.data_ptr(), B, it, float(l[0]), float(l[1]), float(l[2]), clip, ema,
             None)
    torch.cuda.synchronize()


def _saved(tmp_path, s, out="out"):
    sz = param_sizes(s)
    step, P = ot.read_params(tmp_path / f"{out}.bin", sz)
    step_e, E = ot.read_params(tmp_path / f"{out}.ema.bin", sz)
    step_o, adam_t, M, V = ot.read_opt(tmp_path / f"{out}.opt.bin", sz)
    assert step == step_e == step_o
    return step, adam_t, [P, E, M, V]


def _same(core, saved):
    for which in range(4):
        got = core.get(which)
        for i in range(7):
            assert np.array_equal(got[i].view(np.uint32), saved[which][i].view(np.uint32)), (which, i)


OPTS = dict(lr=1e-3, lrn=3e-4, lrp=1e-3, lmin=1e-4, hl=3.0, ema=0.9)


def _opts(B, steps, **kw):
    o = ["--batch", B, "--steps", steps, "--lr", OPTS["lr"], "--lr-neuron", OPTS["lrn"], "--lr-plug", OPTS["lrp"],
         "--lr-min", OPTS["lmin"], "--half-life", OPTS["hl"], "--ema", OPTS["ema"], "--save-sec", 1e9, "--ring", 2]
    for k, v in kw.items():
        o += ["--" + k.replace("_", "-"), v]
    return o


def test_trainer_run_matches_replay(gpu_lib, tmp_path, capfd):
    s, params = toy_net("b", 3, 8, seed=2)
    data, chunks = _setup(tmp_path, s, params)
    B, steps = 64, 5
    rc = _run(tmp_path / "net.bin", tmp_path / "init.bin", data, tmp_path / "out", *_opts(B, steps, log=2, eval_batches=2))
    out = capfd.readouterr().out
    say(out)
    assert rc == 0
    assert "start step 0" in out and "ring of 2 chunks" in out
    assert re.search(r"eval step 0 \| kl [0-9.]+ agree [0-9.]+ \| raw kl .* \| chunk_0002\.bin at the start", out)
    assert re.search(r"step 2 \| [0-9]+ samples/s \| kl [0-9.]+ agree [0-9.]+ \| lr .* \| ring 2, newest chunk_0002\.bin", out)
    assert "saved" in out and "done at step 5" in out
    step, adam_t, saved = _saved(tmp_path, s)
    assert step == 5 and adam_t == 5
    ring = ot.scan_order(data, 2)
    assert ring == ["chunk_0001.bin", "chunk_0002.bin"]
    core = Core(s, params, max_batch=B)
    _replay(core, ring, chunks, ot.MT19937_64(12345), steps, 0, B, OPTS["lr"], OPTS["lrn"], OPTS["lrp"], OPTS["lmin"],
            OPTS["hl"], 0.0, OPTS["ema"])
    _same(core, saved)



@pytest.mark.parametrize("hops", [1, 5])
def test_trainer_run_matches_replay_other_depths(gpu_lib, tmp_path, capfd, hops):
    """The trainer on networks of one and of five hops: weights, running average and both Adam moments after four
    steps bit-identical to the same draws fed through fc_teach_step."""
    s, params = toy_net("b", hops, 8, seed=2)
    data, chunks = _setup(tmp_path, s, params)
    B, steps = 64, 4
    rc = _run(tmp_path / "net.bin", tmp_path / "init.bin", data, tmp_path / "out", *_opts(B, steps))
    say(capfd.readouterr().out)
    assert rc == 0
    step, adam_t, saved = _saved(tmp_path, s)
    assert step == steps and adam_t == steps
    ring = ot.scan_order(data, 2)
    core = Core(s, params, max_batch=B)
    _replay(core, ring, chunks, ot.MT19937_64(12345), steps, 0, B, OPTS["lr"], OPTS["lrn"], OPTS["lrp"], OPTS["lmin"],
            OPTS["hl"], 0.0, OPTS["ema"])
    _same(core, saved)

def test_bf16_trainer_run_matches_replay(gpu_lib, tmp_path, capfd):
    """--bf16 1: the trainer on a bfloat16-state handle, step for step what fc_teach_step does on one."""
    s, params = toy_net("b", 3, 8, seed=2)
    data, chunks = _setup(tmp_path, s, params)
    B, steps = 64, 4
    assert _run(tmp_path / "net.bin", tmp_path / "init.bin", data, tmp_path / "out",
                *_opts(96, steps, bf16=1)) == 2                 # the batch must be a multiple of 64
    rc = _run(tmp_path / "net.bin", tmp_path / "init.bin", data, tmp_path / "out",
              *_opts(B, steps, log=2, eval_batches=2, bf16=1))
    out = capfd.readouterr().out
    say(out)
    assert rc == 0
    assert "bfloat16 states" in out and "done at step 4" in out
    assert re.search(r"eval step 0 \| kl [0-9.]+ agree [0-9.]+ \| raw kl", out)
    step, adam_t, saved = _saved(tmp_path, s)
    assert step == 4 and adam_t == 4
    ring = ot.scan_order(data, 2)
    core = Core(s, params, max_batch=B, flags=1)
    _replay(core, ring, chunks, ot.MT19937_64(12345), steps, 0, B, OPTS["lr"], OPTS["lrn"], OPTS["lrp"], OPTS["lmin"],
            OPTS["hl"], 0.0, OPTS["ema"])
    _same(core, saved)


def test_trainer_resume_clip_and_stop(gpu_lib, tmp_path, capfd):
    s, params = toy_net("a", 3, 5, seed=4)
    data, chunks = _setup(tmp_path, s, params, sizes=(40, 33))
    B = 32
    common = dict(clip=0.05, temp=2.0, eval_batches=0)
    assert _run(tmp_path / "net.bin", tmp_path / "init.bin", data, tmp_path / "out", *_opts(B, 3, **common)) == 0
    assert _run(tmp_path / "net.bin", tmp_path / "out.bin", data, tmp_path / "out", *_opts(B, 2, **common)) == 0
    out = capfd.readouterr().out
    assert "start step 3, optimiser state restored" in out and "done at step 5" in out
    step, adam_t, saved = _saved(tmp_path, s)
    assert step == 5 and adam_t == 5
    ring = ot.scan_order(data, 2)
    core = Core(s, params, max_batch=B)
    args = (B, OPTS["lr"], OPTS["lrn"], OPTS["lrp"], OPTS["lmin"], OPTS["hl"], 0.05, OPTS["ema"], 0.5)
    _replay(core, ring, chunks, ot.MT19937_64(12345), 3, 0, *args)
    _replay(core, ring, chunks, ot.MT19937_64(12345 + 3), 2, 3, *args)     # a restart seeds with its start step
    _same(core, saved)
    # a STOP file ends the run after the next step's save
    (tmp_path / "out.STOP").write_text("")
    assert _run(tmp_path / "net.bin", tmp_path / "out.bin", data, tmp_path / "out", *_opts(B, 100, **common)) == 0
    out = capfd.readouterr().out
    assert "stopped on request at step 6" in out
    assert (tmp_path / "out.STOP.done").exists() and not (tmp_path / "out.STOP").exists()
    assert _saved(tmp_path, s)[0] == 6


def test_trainer_revives_in_the_loop(gpu_lib, tmp_path, capfd):
    s, params, forced = _dead_case(1)
    data, chunks = _setup(tmp_path, s, params, sizes=(64, 64))
    rc = _run(tmp_path / "net.bin", tmp_path / "init.bin", data, tmp_path / "out",
              *_opts(32, 3, revive_every=2, revive_batches=2, revive_first=1, eval_batches=1))
    out = capfd.readouterr().out
    say(out)
    assert rc == 0
    lines = [l for l in out.splitlines() if l.startswith("revive step")]
    assert len(lines) == 2                                     # at the start (--revive-first) and two steps later
    first = re.search(r"revive step 0 \| (\d+) of \d+ neurons", lines[0])
    assert first and int(first.group(1)) >= len(forced)
    for l in lines:
        if "no silent neuron" in l:
            continue
        k = re.search(r"kl ([-0-9.]+) -> ([-0-9.]+) \(must be equal\)", l)
        assert k and k.group(1) == k.group(2), l
    assert "done at step 3" in out


def test_check_mode_matches_oracle(gpu_lib, tmp_path):
    s, params = toy_net("c", 3, 16, seed=3)
    B = 64
    rng = np.random.default_rng(8)
    x = (0.7 * rng.standard_normal((B, OD))).astype(np.float32)
    t = (2 * rng.standard_normal((B, NA))).astype(np.float32)
    (tmp_path / "net.bin").write_bytes(net_bytes(s))
    write_params(params, tmp_path / "p.bin", 0)
    (tmp_path / "batch.bin").write_bytes(b"FLYB" + struct.pack("<i", B) + x.tobytes() + t.tobytes())
    exe = lib()._name.replace("libflyguy_core.so", "flyguy_train")
    say("flyguy_train --check", exe)
    r = subprocess.run([exe, "--check", tmp_path / "net.bin", tmp_path / "p.bin", tmp_path / "batch.bin"],
                       capture_output=True, text=True, timeout=120)
    say(r.stdout, r.stderr)
    assert r.returncode == 0
    o = Oracle(net_bytes(s), params, "f64")
    lg = o.forward(x)
    dl, kl, agree = o.loss(lg, t, 1.0)
    grads = o.backward(dl)
    m = re.search(r"native: loss ([-0-9.e+]+) agree ([0-9.]+)", r.stdout)
    assert abs(float(m.group(1)) - kl / B) <= 1e-5 * max(abs(kl / B), 1e-3) + 1e-6
    assert abs(float(m.group(2)) - agree / B) <= 1.5 / B
    first = [float(v) for v in re.search(r"logits\[0\]\[:5\] (.*)", r.stdout).group(1).split()]
    assert np.allclose(first, lg[0, :5], atol=2e-6 * max(1.0, np.abs(lg).max()))
    for name, g in zip(("W", "gain", "theta", "in_w", "in_b", "out_w", "out_b"), grads):
        mm = re.search(rf"grad {name}\s+norm ([-0-9.e+]+) sum ([-+0-9.e]+)", r.stdout)
        norm, tot = float(mm.group(1)), float(mm.group(2))
        n0 = float(np.linalg.norm(g.astype(np.float64)))
        assert abs(norm - n0) <= 1e-4 * max(n0, 1e-12) + 1e-9, (name, norm, n0)
        assert abs(tot - float(g.astype(np.float64).sum())) <= 1e-4 * float(np.abs(g).sum()) + 1e-9, name


def test_export_batch_then_check(gpu_lib, tmp_path):
    """The reference's workflow for checking the library against PyTorch (export.py net / params / batch, then
    flyguy_train --check NET PARAMS BATCH): the library's loss, first logits and gradient norms and sums agree with
    the PyTorch path's, as the converter printed them."""
    from conftest import GOLDEN
    from flyguy_amd.export import main as export_main
    graph = GOLDEN / "toy_b.npz"
    torch.manual_seed(4)
    f = lively(FlyActor(str(graph), OD, NA, hops=3, fan=16), 4)
    ck = {"model": {"actor." + k: v.detach().clone() for k, v in f.state_dict().items()},
          "config": {"model": {"fly_graph": str(graph), "fly_hops": 3}}}
    torch.save(ck, tmp_path / "ck.pt")
    net, p, b = tmp_path / "net.bin", tmp_path / "p.bin", tmp_path / "batch.bin"
    import contextlib
    import io
    torch.manual_seed(4)
    assert export_main(["net", str(graph), str(net), "--hops", "3", "--fan", "16"]) == 0
    assert export_main(["params", str(tmp_path / "ck.pt"), str(p)]) == 0
    out = io.StringIO()
    with contextlib.redirect_stdout(out):
        assert export_main(["batch", str(tmp_path / "ck.pt"), str(b), "--n", "64"]) == 0
    ref = out.getvalue()
    exe = lib()._name.replace("libflyguy_core.so", "flyguy_train")
    say("export batch -> flyguy_train --check")
    r = subprocess.run([exe, "--check", net, p, b], capture_output=True, text=True, timeout=120)
    say(ref, r.stdout, r.stderr)
    assert r.returncode == 0
    lt = float(re.search(r"torch: loss ([-0-9.e+]+)", ref).group(1))
    ln = float(re.search(r"native: loss ([-0-9.e+]+)", r.stdout).group(1))
    assert abs(ln - lt) <= 1e-5 * max(1.0, abs(lt))
    first_t = [float(v) for v in re.search(r"logits\[0\]\[:5\] (.*)", ref).group(1).split()]
    first_n = [float(v) for v in re.search(r"logits\[0\]\[:5\] (.*)", r.stdout).group(1).split()]
    assert np.allclose(first_n, first_t, atol=1e-5, rtol=1e-5)
    for name in ("W", "gain", "theta", "in_w", "in_b", "out_w", "out_b"):
        pat = rf"grad {name}\s+norm ([-0-9.e+]+) sum ([-+0-9.e]+)"
        nt, st = (float(v) for v in re.search(pat, ref).groups())
        nn, sn = (float(v) for v in re.search(pat, r.stdout).groups())
        assert abs(nn - nt) <= 1e-4 * max(nt, 1e-12), (name, nn, nt)
        assert abs(sn - st) <= 1e-4 * max(nt, 1e-12) * 64, (name, sn, st)
