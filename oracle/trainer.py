"""ORACLE - test infrastructure only: the teaching trainer's host-side arithmetic restated in plain Python / numpy.

Restates flyguy/native/flyguy_train.cu:
  * the batch draw, draw_batch (:412-424), over the C++ standard's std::mt19937_64 ([rand.predef]) and the bounded
    draw of libstdc++'s std::uniform_int_distribution<long long> for a 64-bit engine (bits/uniform_int_dist.h of
    GCC 11: Lemire's nearly divisionless method with a 128-bit product);
  * the learning-rate schedule of a step (:764-769);
  * the chunk selection of a scan (Loader::scan, :392-404) and the FLYD reader's checks (read_chunk, :372-384);
  * the FLYP / FLYO files (:258-307);
  * survey sums (k_fired :181-187, survey :436-454, per_neuron :456-461, firing_line :462-471);
  * the revive surgery (:472-551), given a survey function.

Pinned by tests/test_trainer_cpu.py: mt19937_64 against the standard's known answer (the 10000th output of a
default-seeded engine is 9981545732273789042) and a seeded g++ probe; the bounded draw against
std::uniform_int_distribution compiled with g++; the schedule against closed forms.  The revive restatement is
pinned by its invariants (the network's output unchanged, revived neurons firing, marks and signs) in the GPU
tests, and the survey sums by brute force over the oracle's states.
"""
from __future__ import annotations

import math
import os
import struct
from pathlib import Path

import numpy as np

M64 = (1 << 64) - 1


class MT19937_64:
    """std::mt19937_64: w=64, n=312, m=156, r=31, a=0xB5026F5AA96619E9, u=29, d=0x5555555555555555, s=17,
    b=0x71D67FFFEDA60000, t=37, c=0xFFF7EEE000000000, l=43, f=6364136223846793005."""
    N, M = 312, 156
    A = 0xB5026F5AA96619E9
    UPPER, LOWER = (~((1 << 31) - 1)) & M64, (1 << 31) - 1

    def __init__(self, seed: int = 5489):
        mt = [0] * self.N
        mt[0] = seed & M64
        for i in range(1, self.N):
            x = mt[i - 1]
            mt[i] = (6364136223846793005 * (x ^ (x >> 62)) + i) & M64
        self.mt, self.i = mt, self.N

    def _twist(self):
        mt, N, M = self.mt, self.N, self.M
        for k in range(N):
            y = (mt[k] & self.UPPER) | (mt[(k + 1) % N] & self.LOWER)
            v = y >> 1
            if y & 1:
                v ^= self.A
            mt[k] = mt[(k + M) % N] ^ v
        self.i = 0

    def __call__(self) -> int:
        if self.i >= self.N:
            self._twist()
        y = self.mt[self.i]
        self.i += 1
        y ^= (y >> 29) & 0x5555555555555555
        y ^= (y << 17) & 0x71D67FFFEDA60000 & M64
        y ^= (y << 37) & 0xFFF7EEE000000000 & M64
        y ^= y >> 43
        return y & M64


def uniform(g: MT19937_64, lo: int, hi: int) -> int:
    """std::uniform_int_distribution<long long>(lo, hi)(g) for a 64-bit engine (libstdc++)."""
    urange = (hi - lo) & M64
    if urange == M64:
        return lo + g()
    erange = urange + 1
    product = g() * erange
    low = product & M64
    if low < erange:
        threshold = ((1 << 64) - erange) % erange
        while low < threshold:
            product = g() * erange
            low = product & M64
    return lo + (product >> 64)


def draw(g: MT19937_64, sizes, B: int) -> np.ndarray:
    """draw_batch (flyguy_train.cu:412-424): [B][2] = {chunk, sample}."""
    total = int(sum(sizes))
    out = np.zeros((B, 2), np.int64)
    for i in range(B):
        s = uniform(g, 0, total - 1)
        c = 0
        while s >= sizes[c]:
            s -= sizes[c]
            c += 1
        out[i] = (c, s)
    return out


def draws(seed: int, sizes, B: int, n_batches: int) -> np.ndarray:
    g = MT19937_64(seed)
    return np.concatenate([draw(g, sizes, B) for _ in range(n_batches)]) if n_batches else np.zeros((0, 2), np.int64)


def lr(step: int, lr0: float, lr_neuron: float, lr_plug: float, lr_min: float, half_life: float) -> np.ndarray:
    """The three group learning rates of step `step` (flyguy_train.cu:764-769), in float32 as the trainer computes
    them: sched = (float) 0.5^(step / half_life); max(lr_min * base / lr, base * sched)."""
    f = np.float32
    sched = f(math.pow(0.5, step / half_life))
    out = []
    for base in (f(lr0), f(lr_neuron), f(lr_plug)):
        out.append(max(f(f(f(lr_min) * base) / f(lr0)), f(base * sched)))
    return np.array(out, np.float32)


def scan_order(d: Path, keep: int) -> list[str]:
    """Loader::scan's choice on a first scan (flyguy_train.cu:392-404): chunk_*.bin by (modification time, path),
    of several only the newest `keep`."""
    files = []
    for e in os.scandir(d):
        name = e.name
        if not name.startswith("chunk_") or os.path.splitext(name)[1] != ".bin":
            continue
        files.append((e.stat().st_mtime_ns, str(Path(d) / name), name))
    files.sort()
    return [n for _, _, n in files[max(0, len(files) - keep):]]


# ---- files
def write_chunk(path: Path, obs16: np.ndarray, lg16: np.ndarray) -> None:
    """A FLYD chunk (flyguy/native/gen_data.py:151-176 writes this layout)."""
    obs16, lg16 = np.ascontiguousarray(obs16, np.float16), np.ascontiguousarray(lg16, np.float16)
    with open(path, "wb") as fh:
        fh.write(b"FLYD" + struct.pack("<qii", obs16.shape[0], obs16.shape[1], lg16.shape[1]))
        fh.write(obs16.tobytes())
        fh.write(lg16.tobytes())


def chunk_samples(path: Path, obs_dim: int, n_act: int) -> int:
    """read_chunk's checks (flyguy_train.cu:372-384): -1 unless the whole file is a FLYD chunk of these sizes."""
    try:
        raw = Path(path).read_bytes()
    except OSError:
        return -1
    if len(raw) < 20 or raw[:4] != b"FLYD":
        return -1
    n, od, na = struct.unpack("<qii", raw[4:20])
    if od != obs_dim or na != n_act or n <= 0:
        return -1
    if len(raw) - 20 < 2 * n * (od + na):
        return -1
    return n


def read_params(path: Path, sizes) -> tuple[int, list[np.ndarray]]:
    raw = Path(path).read_bytes()
    assert raw[:4] == b"FLYP"
    step = struct.unpack("<q", raw[4:12])[0]
    out, off = [], 12
    for n in sizes:
        out.append(np.frombuffer(raw, np.float32, n, off).copy())
        off += 4 * n
    assert off == len(raw)
    return step, out


def read_opt(path: Path, sizes) -> tuple[int, int, list[np.ndarray], list[np.ndarray]]:
    """FLYO (flyguy_train.cu:288-294): step, adam_t, then per array m and v."""
    raw = Path(path).read_bytes()
    assert raw[:4] == b"FLYO"
    step, adam_t = struct.unpack("<qq", raw[4:20])
    m, v, off = [], [], 20
    for n in sizes:
        m.append(np.frombuffer(raw, np.float32, n, off).copy())
        off += 4 * n
        v.append(np.frombuffer(raw, np.float32, n, off).copy())
        off += 4 * n
    assert off == len(raw)
    return step, adam_t, m, v


# ---- survey and revive
def survey_sums(states: list[tuple[np.ndarray, np.ndarray | None]]):
    """k_fired (flyguy_train.cu:181-187) over each layer's (h, z) [rows][B]: fires = #(h > 0), sq = sum z^2 (0 for
    a layer without z)."""
    cnt, sq = [], []
    for h, z in states:
        cnt.append((h > 0).sum(1).astype(np.int64))
        sq.append((z.astype(np.float64) ** 2).sum(1) if z is not None else np.zeros(h.shape[0]))
    return np.concatenate(cnt), np.concatenate(sq)


def per_neuron(s: dict, cnt: np.ndarray):
    """fired / play / sens per neuron (flyguy_train.cu:456-461)."""
    N = s["n_neurons"]
    fired = np.zeros(N, np.int64)
    play = np.zeros(N, bool)
    sens = np.zeros(N, bool)
    sens[np.asarray(s["n0"])] = True
    off = s["sizes"][0]
    for h in s["hop"]:
        nid = np.asarray(h["nid"])
        play[nid] = True
        np.add.at(fired, nid, cnt[off:off + len(nid)])
        off += len(nid)
    return fired, play, sens


def median_positive(v: np.ndarray) -> np.float32:
    p = np.sort(v[v > 0])
    return np.float32(p[len(p) // 2]) if len(p) else np.float32(0)


def revive(s: dict, P: list[np.ndarray], EMA: list[np.ndarray], M: list[np.ndarray], V: list[np.ndarray],
           survey, target: float, seed: int) -> dict:
    """The revive surgery (flyguy_train.cu:486-551) on copies of the arrays.  survey(P) -> (cnt, sq, samples, kl).
    Returns the new arrays and the report's counts."""
    f = np.float32
    P, EMA, M, V = ([a.copy() for a in x] for x in (P, EMA, M, V))
    N, K, n_dn, n_act = s["n_neurons"], s["hops"], s["n_dn"], s["n_act"]
    cnt0, _, samples0, kl0 = survey(P)
    fired, play, sens = per_neuron(s, cnt0)
    dead = play & ~sens & (fired == 0)
    out = {"n_dead": int(dead.sum()), "n_play": int((play & ~sens).sum()), "kl0": kl0}
    if not dead.any():
        out.update(P=P, EMA=EMA, M=M, V=V)
        return out
    W, gain, theta, ow = P[0], P[1], P[2], P[5]
    mark = np.zeros(s["n_w"], np.int8)
    r = MT19937_64((seed * 7919 + 17) & M64)
    n_in = n_out = 0
    for k, h in enumerate(s["hop"]):
        below = np.asarray(s["hop"][k - 1]["nid"]) if k else np.asarray(s["n0"])
        nid, crow, col, widx = (np.asarray(h[x]) for x in ("nid", "crow", "col", "widx"))
        for t in range(len(nid)):
            dpost = dead[nid[t]]
            for e in range(int(crow[t]), int(crow[t + 1])):
                wi = int(widx[e])
                if mark[wi]:
                    continue
                if dpost:
                    W[wi] = f(max(abs(W[wi]), f(1e-4))) * (f(1) if (r() & 1) else f(-1))
                    mark[wi] = 1
                    n_in += 1
                elif dead[below[col[e]]]:
                    W[wi] = f(0)
                    mark[wi] = 2
                    n_out += 1
    gain[dead] = 1.0
    theta[dead] = -4.0
    top = np.asarray(s["hop"][K - 1]["nid"])
    dcol = dead[top[np.asarray(s["dn_rows"])]]
    ow.reshape(n_act, n_dn)[:, dcol] = 0.0
    for _ in range(3):
        _, sq, samples, _ = survey(P)
        rms = np.zeros(N, np.float32)
        off = s["sizes"][0]
        for h in s["hop"]:
            nid = np.asarray(h["nid"])
            for t in range(len(nid)):
                rms[nid[t]] = max(rms[nid[t]], f(math.sqrt(float(sq[off + t]) / samples)))
            off += len(nid)
        done = np.zeros(s["n_w"], bool)
        for h in s["hop"]:
            nid, crow, widx = (np.asarray(h[x]) for x in ("nid", "crow", "widx"))
            for t in range(len(nid)):
                g = nid[t]
                if not dead[g] or rms[g] <= 0:
                    continue
                sc = min(f(200), max(f(0.02), f(f(target) / rms[g])))
                for e in range(int(crow[t]), int(crow[t + 1])):
                    wi = int(widx[e])
                    if not done[wi]:
                        W[wi] = f(W[wi] * sc)
                        done[wi] = True
    cnt1, _, _, kl1 = survey(P)
    fired1, _, _ = per_neuron(s, cnt1)
    fill = median_positive(V[0])
    mk = mark > 0
    EMA[0][mk] = W[mk]
    M[0][mk] = 0
    V[0][mk] = fill
    for p, val in ((1, 1.0), (2, -4.0)):
        f2 = median_positive(V[p])
        EMA[p][dead] = val
        M[p][dead] = 0
        V[p][dead] = f2
    EMA[5].reshape(n_act, n_dn)[:, dcol] = 0
    M[5].reshape(n_act, n_dn)[:, dcol] = 0
    out.update(P=P, EMA=EMA, M=M, V=V, mark=mark, dead=dead, n_in=n_in, n_out=n_out, n_dn_dead=int(dcol.sum()),
               still=int((dead & (fired1 == 0)).sum()), kl1=kl1)
    return out
