"""Write the golden index vectors of the fly actor from the reference implementation itself.

The graph indexing of the reference (FlyActor.__init__, flyguy/fly.py:78-154, and export.structure /
export.write_net, flyguy/native/export.py:32-65) must be reproduced bit-exactly, and nothing but the
reference's own code yields its arrays.  This script imports those two functions from the reference checkout
(read-only, no bytecode written), runs them on small toy connectomes generated here, and stores inputs and
outputs as .npz fixtures (no pickles).  For the shipped 3-hop graph it stores SHA-256 digests of every array.

    python tests/golden/make_golden.py /root/reference

Fixtures written (all in tests/golden/):
    toy_<name>.npz        the toy graph (inputs: body, nt, pre, post, syn, sensory, descending[, in_total, hops])
    idx_<name>_h<H>_f<F>.npz   every buffer of FlyActor(graph, 517, 90, hops=H, fan=F) built after
                               torch.manual_seed(0), its initial parameters, structure() arrays and the NET.bin bytes
    shipped_3hop.json     SHA-256 of every buffer / structure array / NET.bin of the shipped graph (hops 3, fan 16)
"""
from __future__ import annotations

import hashlib
import json
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def toy_graph(n: int, n_sens: int, n_dn: int, edges: int, seed: int, sigma: float = 0.0, trimmed: bool = False) -> dict:
    """A random connectome: unique (pre, post) pairs, no self loops; optional lognormal in-degree skew."""
    rng = np.random.default_rng(seed)
    if sigma > 0:
        pdeg = rng.lognormal(0.0, sigma, n)
        pdeg /= pdeg.sum()
    else:
        pdeg = None
    pairs: set[tuple[int, int]] = set()
    while len(pairs) < edges:
        b = int(rng.choice(n, p=pdeg)) if pdeg is not None else int(rng.integers(n))
        a = int(rng.integers(n))
        if a != b:
            pairs.add((a, b))
    order = rng.permutation(len(pairs))                     # edges in random order, not sorted
    arr = np.array(sorted(pairs), np.int64)[order]
    pre, post = arr[:, 0].astype(np.int32), arr[:, 1].astype(np.int32)
    ids = rng.permutation(n)
    g = dict(body=(np.arange(n) + 1000).astype(np.int64),
             nt=rng.choice(np.array(["acetylcholine", "gaba", "glutamate", "histamine", "serotonin"]), n),
             pre=pre, post=post, syn=rng.integers(2, 40, len(pre)).astype(np.int32),
             sensory=np.sort(ids[:n_sens]).astype(np.int32),
             descending=np.sort(ids[n_sens:n_sens + n_dn]).astype(np.int32))
    if trimmed:                                             # the trimmed-file form: whole-graph in_total kept beside
        tot = np.zeros(n, np.int64)
        np.add.at(tot, post, g["syn"])
        g["in_total"] = tot + rng.integers(0, 5, n)        # (as if some connections were cut away)
        g["hops"] = np.int64(4)
    return g


TOYS = {
    "a": dict(n=80, n_sens=14, n_dn=7, edges=420, seed=0),
    "b": dict(n=600, n_sens=60, n_dn=25, edges=6000, seed=1, sigma=1.0),
    "c": dict(n=300, n_sens=40, n_dn=12, edges=2500, seed=2, sigma=1.5, trimmed=True),
}
CASES = [("a", 2, 5), ("a", 3, 5), ("a", 4, 5), ("a", 3, 16), ("b", 3, 16), ("b", 2, 8), ("c", 3, 16), ("c", 4, 6)]
BUFS = ["e", "r", "c", "crow", "tcrow", "tcol", "tperm", "ci", "tci", "n", "s", "d"]
PLUG = ["in_r", "in_c", "in_crow", "in_tcrow", "in_tcol", "in_tperm", "in_ci", "in_tci", "n0", "dn_rows"]
PARAMS = ["w", "gain", "theta", "in_w", "in_b", "out.weight", "out.bias"]


def collect(f, write_net, structure) -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for k in range(1, f.hops + 1):
        for b in BUFS:
            out[f"{b}{k}"] = getattr(f, f"{b}{k}").numpy()
    for b in PLUG:
        out[b] = getattr(f, b).numpy()
    sd = f.state_dict()
    for p in PARAMS:
        out["param_" + p] = sd[p].numpy()
    out["sizes"] = np.array(f.sizes, np.int64)
    out["counts"] = np.array([f.n_neurons, f.n_conn, f.used, f.in_play], np.int64)
    s = structure(f)
    out["wmap"] = np.asarray(s["wmap"])
    for k, h in enumerate(s["hop"], 1):
        for name in ("widx", "twidx", "drow"):
            out[f"st_{name}{k}"] = np.asarray(h[name])
    with tempfile.TemporaryDirectory() as tmp:
        write_net(f, Path(tmp) / "net.bin")
        out["net_bin"] = np.frombuffer((Path(tmp) / "net.bin").read_bytes(), np.uint8).copy()
    return out


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.dont_write_bytecode = True
    sys.path.insert(0, str(ref))
    import torch
    from flyguy.fly import FlyActor                         # the reference's index build (fly.py:78-154)
    from flyguy.native.export import structure, write_net   # the reference's NET.bin writer (export.py:32-65)

    for name, kw in TOYS.items():
        g = toy_graph(**kw)
        np.savez_compressed(HERE / f"toy_{name}.npz", **g)
    for name, hops, fan in CASES:
        torch.manual_seed(0)
        f = FlyActor(HERE / f"toy_{name}.npz", 517, 90, hops=hops, fan=fan)
        np.savez_compressed(HERE / f"idx_{name}_h{hops}_f{fan}.npz", **collect(f, write_net, structure))
        print(f"toy {name} hops {hops} fan {fan}: sizes {f.sizes}, used {f.used}, in play {f.in_play}")

    shipped = ref / "flyguy" / "graphs" / "male_cns_min2_3hop.npz"
    if shipped.exists():
        torch.manual_seed(0)
        f = FlyActor(shipped, 517, 90, hops=3, fan=16)
        arrs = collect(f, write_net, structure)
        digest = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() for k, v in arrs.items()
                  if not k.startswith("param_")}
        digest["_dtypes"] = {k: str(v.dtype) for k, v in arrs.items() if not k.startswith("param_")}
        digest["_shapes"] = {k: list(v.shape) for k, v in arrs.items() if not k.startswith("param_")}
        digest["_sizes"] = [int(x) for x in arrs["sizes"]]
        digest["_counts"] = [int(x) for x in arrs["counts"]]
        (HERE / "shipped_3hop.json").write_text(json.dumps(digest, indent=1, sort_keys=True))
        print(f"shipped graph: sizes {f.sizes}, used {f.used}, in play {f.in_play}")


if __name__ == "__main__":
    main()
