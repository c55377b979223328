"""ORACLE - test infrastructure only: the library core with bfloat16 states, restated in numpy.

The arithmetic is the reference's (flyguy/native/flyguy_train.cu:73-203: plug, neuron layers, hops, read-out and
their backward, as oracle/fly_oracle.c restates them), done here in float64 with the sums of scipy's sparse products.
What makes it the 16-bit variant is where values are rounded to bfloat16 (round to nearest even): the points where
the library stores a state, and the connection strengths and plug weights its sparse products use (the masters,
their gradients and Adam stay float32):
  x = bf16(obs); drive = in_b + bf16(in_w) . x; h0 = bf16(relu(gain drive - softplus theta)); the stored drive
  bf16(drive);
  hop k: z = bf16(W) . h_{k-1} (+ the stored drive of a re-drive row), h_k = bf16(relu(gain z - softplus theta));
  backward: gz = g gain with g = gh where h > 0, gathered as bf16(gz); the drive's gradient sums the hops' gz before
  rounding; a hop layer's gain gradient is sum g (h + softplus theta) / gain over its stored h (0 when gain = 0), the
  sensory layer's sum g . bf16(drive); per-connection gradients multiply bf16(gz) by the stored source states; the
  gradient of a layer's output is bf16(W)^T . bf16(gz).
softplus is taken in float32 (the library computes it so).

Pinned by tests/test_gpu_core16.py: bit-exact agreement on networks whose every value and sum is exact (integer
states and weights), the rounding against hand-worked ties and special values, and the float32 oracle (fly_oracle.c)
when the rounding is switched off (round=False).
"""
from __future__ import annotations

import numpy as np
import scipy.sparse as sp


def bf16(a: np.ndarray) -> np.ndarray:
    """float64 -> float32 -> bfloat16 (round to nearest even, NaN kept) -> float64."""
    f = np.asarray(a, np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32) << 16
    return r.view(np.float32).astype(np.float64)


def _softplus32(theta: np.ndarray) -> np.ndarray:
    t = np.asarray(theta, np.float32)
    return np.where(t > np.float32(20), t, np.log1p(np.exp(t))).astype(np.float32).astype(np.float64)


def _csr(vals, col, crow, shape):
    return sp.csr_matrix((np.asarray(vals, np.float64), np.asarray(col, np.int64), np.asarray(crow, np.int64)), shape=shape)


class Core16:
    """One network (structure dict of flyguy_amd.export.structure) with its seven weight arrays."""

    def __init__(self, s: dict, params: list[np.ndarray], round: bool = True, round_weights: bool = True):
        """round: the bfloat16 rounding on (states, and the weights of the sparse products unless round_weights is
        False) or off (the float32 / float64 core)."""
        self.s = s
        self.P = [np.asarray(p, np.float64) for p in params]
        ident = lambda a: np.asarray(a, np.float64)                              # noqa: E731
        self.r = bf16 if round else ident
        self.rw = bf16 if round and round_weights else ident

    def forward(self, obs: np.ndarray) -> np.ndarray:
        s, r = self.s, self.r
        W, gain, theta, in_w, in_b, ow, ob = self.P
        spl = _softplus32(theta)
        n_s, od = s["n_s"], s["obs_dim"]
        self.x = r(np.asarray(obs, np.float32).T.astype(np.float64))             # [obs_dim][B]
        drive = in_b[:, None] + _csr(self.rw(in_w), s["in_col"], s["in_crow"], (n_s, od)) @ self.x
        n0 = np.asarray(s["n0"])
        h0 = r(np.maximum(gain[n0][:, None] * drive - spl[n0][:, None], 0.0))
        self.drive = r(drive)
        self.states = [(h0, self.drive)]
        hp = h0
        for k, h in enumerate(s["hop"]):
            rows, src = s["sizes"][k + 1], s["sizes"][k]
            widx = np.asarray(h["widx"])
            z = _csr(self.rw(W[widx]), h["col"], h["crow"], (rows, src)) @ hp
            drow = np.asarray(h["drow"])
            m = drow >= 0
            z[m] += self.drive[drow[m]]
            nid = np.asarray(h["nid"])
            hk = r(np.maximum(gain[nid][:, None] * z - spl[nid][:, None], 0.0))
            self.states.append((hk, z))
            hp = hk
        dn = np.asarray(s["dn_rows"])
        owm = ow.reshape(s["n_act"], s["n_dn"])
        return (ob[None, :] + (owm @ hp[dn]).T)                                  # [B][n_act]

    def backward(self, dl: np.ndarray) -> list[np.ndarray]:
        """Gradients of the seven arrays for d(loss)/d(logits) = dl [B][n_act], after forward."""
        s, r = self.s, self.r
        W, gain, theta, in_w, in_b, ow, ob = self.P
        spl = _softplus32(theta)
        dl = np.asarray(dl, np.float64)
        n_act, n_dn, K = s["n_act"], s["n_dn"], s["hops"]
        dn = np.asarray(s["dn_rows"])
        owm = ow.reshape(n_act, n_dn)
        hK = self.states[K][0]
        gow = dl.T @ hK[dn].T                                                    # [n_act][n_dn]
        gob = dl.sum(0)
        gh = np.zeros_like(hK)
        gh[dn] = owm.T @ dl.T
        N = s["n_neurons"]
        gW, ggain, gsum = np.zeros(s["n_w"]), np.zeros(N), np.zeros(N)
        gdrive = np.zeros((s["n_s"], dl.shape[0]))
        for k in range(K, 0, -1):
            h = s["hop"][k - 1]
            hk = self.states[k][0]
            nid = np.asarray(h["nid"])
            g = np.where(hk > 0, gh, 0.0)
            gn = gain[nid]
            gz = g * gn[:, None]
            sg = g.sum(1)
            with np.errstate(divide="ignore", invalid="ignore"):
                pg = np.where(gn != 0, ((g * hk).sum(1) + spl[nid] * sg) / np.where(gn != 0, gn, 1.0), 0.0)
            np.add.at(ggain, nid, pg)
            np.add.at(gsum, nid, sg)
            drow = np.asarray(h["drow"])
            m = drow >= 0
            np.add.at(gdrive, drow[m], gz[m])
            gz16 = r(gz)
            below = self.states[k - 1][0]
            crow, col, widx = (np.asarray(h[x]) for x in ("crow", "col", "widx"))
            tgt = np.repeat(np.arange(len(crow) - 1), np.diff(crow))
            np.add.at(gW, widx, (gz16[tgt] * below[col]).sum(1))
            A = _csr(self.rw(W[widx]), col, crow, (s["sizes"][k], s["sizes"][k - 1]))
            gh = A.T @ gz16
        h0, dr = self.states[0]
        n0 = np.asarray(s["n0"])
        g0 = np.where(h0 > 0, gh, 0.0)
        gz0 = g0 * gain[n0][:, None]
        np.add.at(ggain, n0, (g0 * dr).sum(1))
        np.add.at(gsum, n0, g0.sum(1))
        gd = gdrive + gz0
        gin_b = gd.sum(1)
        in_crow, in_col = np.asarray(s["in_crow"]), np.asarray(s["in_col"])
        tgt = np.repeat(np.arange(len(in_crow) - 1), np.diff(in_crow))
        gin_w = (gd[tgt] * self.x[in_col]).sum(1)
        sig = 1.0 / (1.0 + np.exp(-np.asarray(theta, np.float64)))
        gtheta = -sig * gsum
        return [gW, ggain, gtheta, gin_w, gin_b, gow.reshape(-1), gob]
