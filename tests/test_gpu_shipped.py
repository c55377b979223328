"""The shipped network through the HIP library: the reference's 3-hop graph (flyguy/graphs/male_cns_min2_3hop.npz)
with its trained actor (bot/model.pt), as the reference's own parity harness checks its library
(flyguy/native/core_check.py:22-76), here against the float64 oracle instead of the PyTorch path.

The two files are data, copied from the reference checkout by `make -C oracle shipped` into oracle/_ref/shipped
(built with the oracle, travels with the tree); the graph is read by np.load (no pickles) and the checkpoint by
torch.load(weights_only=True).  The actor is built by FlyActor from the graph file, its weights loaded from the
checkpoint, and the network handed to the library as NET.bin bytes.

  * B = 64 through the C-ABI: logits and every layer's states <= 1e-5, argmax identical, the seven gradients of
    core_check's made-up loss (sum(l * r) + 0.1 sum(l^2)) <= 1e-4, relative to the largest entry;
  * NativeFlyActor at B = 160 in pieces of max_batch 64 (core_check.py:40-56): logits the same bar; gradients within
    1e-4 of float64 on the samples whose firing pattern the library and both oracles share, and over the whole batch
    within 1e-4 or no further from float64 than 1.1 x the float32 oracle's distance + 1e-6; then one Adam step at 1e-3 with core_check's move bounds (core_check.py:64-73): a strength moves between 5e-4
    and 2e-3, a gain between 1e-4 and 6e-4 (rate 0.3x), strengths not in play not at all;
  * B = 4096 (the benchmark batch): logits <= 1e-5 against float64 and <= 4e-6 against the float32 oracle, argmax
    identical off near-ties; 64-sample slices give the same logits bit for bit;
  * a teaching step (KL loss against teacher logits 2 N(0,1)) at B = 512 and 4096: the gradients held as at the
    synthetic network's benchmark batch (tests/test_gpu_configs.py);
  * B = 4096: gradients of four 1024-sample pieces add up to the whole batch's (<= 1e-5), pieces' logits bit for bit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from flyguy_amd.export import actor_of, net_bytes, params_from_torch, structure
from gpu_helpers import NAMES, Core, argmax_agrees, rel, say
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu
SHIPPED = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "shipped"
GRAPH, MODEL = SHIPPED / "male_cns_min2_3hop.npz", SHIPPED / "model.pt"


def _checkpoint() -> dict:
    if not (GRAPH.exists() and MODEL.exists()):
        pytest.skip("the shipped network's data files are not in oracle/_ref/shipped (make -C oracle shipped)")
    return torch.load(MODEL, map_location="cpu", weights_only=True)


@pytest.fixture(scope="module")
def shipped():
    say("shipped network: graph, index, trained weights")
    f = actor_of(_checkpoint(), graph=str(GRAPH))
    s = structure(f)
    return f, s, params_from_torch(f, s)


def _core_check_inputs(n: int) -> tuple[np.ndarray, np.ndarray]:
    """core_check.py:37-39: torch seed 0, observations 0.5 N(0,1), the loss's weights N(0,1)."""
    torch.manual_seed(0)
    obs = torch.randn(n, 517) * 0.5
    R = torch.randn(n, 90)
    return obs.numpy(), R.numpy()


def test_shipped_network_is_the_published_one(shipped):
    f, s, params = shipped
    assert s["sizes"] == [16_894, 46_393, 37_748, 1_332]
    assert [len(h["col"]) for h in s["hop"]] == [771_482, 2_569_085, 347_491]
    assert s["n_w"] == 2_992_734 and params[3].size == 270_304
    assert all(np.isfinite(p).all() for p in params)


def test_shipped_b64_against_oracle(gpu_lib, shipped):
    f, s, params = shipped
    B = 64
    obs, R = _core_check_inputs(B)
    core = Core(s, params, max_batch=B)
    got = core.forward(obs)
    o64 = Oracle(net_bytes(s), params, "f64")
    want = o64.forward(obs)
    r = rel(got, want)
    ok, ties = argmax_agrees(got, want)
    say(f"   logits rel {r:.2e} (logits up to {np.abs(want).max():.2f}), near ties {ties}")
    assert r <= 1e-5 and ok
    assert np.array_equal(got.argmax(1), want.argmax(1))
    for layer in range(s["hops"] + 1):
        rows = s["sizes"][layer]
        g, w = core.state(layer, 0, rows, B), o64.state(layer, 0, rows)
        say(f"   layer {layer} h rel {rel(g, w):.2e}, silent (row, sample) share {(w <= 0).mean():.3f}")
        assert rel(g, w) <= 1e-5, layer
    dl = (R + 0.2 * got).astype(np.float32)
    core.zero_grad()
    core.backward(dl)
    for name, g, w in zip(NAMES, core.get(4), o64.backward(dl)):
        r = rel(g, w)
        say(f"   grad {name:6s} rel {r:.2e}")
        assert r <= 1e-4, (name, r)


def test_shipped_native_actor_pieces_and_adam(gpu_lib):
    """NativeFlyActor as core_check drives it: B = 160 in pieces of 64 (the last one padded to 32 samples), the
    gradients added over the pieces, then one step of the library's Adam."""
    from flyguy_amd.fly_native import NativeFlyActor, grad_arrays
    say("shipped network: NativeFlyActor, max_batch 64")
    nat = actor_of(_checkpoint(), graph=str(GRAPH), cls=NativeFlyActor, max_batch=64)
    s = structure(nat)
    params = params_from_torch(nat, s)
    nat = nat.cuda()
    B = 160
    obs, R = _core_check_inputs(B)
    opt = nat.native_adam(1e-3, 0.0)
    assert opt is not None
    opt.zero_grad()
    x, r = torch.as_tensor(obs).cuda(), torch.as_tensor(R).cuda()
    ln = nat(x)
    ((ln * r).sum() + 0.1 * ln.pow(2).sum()).backward()
    got_lg = ln.detach().cpu().numpy()
    o64 = Oracle(net_bytes(s), params, "f64")
    want = o64.forward(obs)
    r_lg = rel(got_lg, want)
    say(f"   logits rel {r_lg:.2e}")
    assert r_lg <= 1e-5 and argmax_agrees(got_lg, want)[0]
    dl = (R + 0.2 * got_lg).astype(np.float32)       # the made-up loss's gradient at the library's logits
    o32 = Oracle(net_bytes(s), params, "f32")
    o32.forward(obs)
    # the whole batch: within 1e-4 of float64, or no further from it than the reference's float32 arithmetic is
    # (here one layer-2 neuron of sample 145 sits 2.3e-7 above its threshold in float32 and at 0 in float64, which
    # moves the float32 oracle's threshold gradient by 2.2e-4 of its largest entry)
    for name, g, a, w in zip(NAMES, grad_arrays(nat), o32.backward(dl), o64.backward(dl)):
        rr, r_ref = rel(g.reshape(-1), w), rel(a, w)
        say(f"   grad {name:6s} rel {rr:.2e} (float32 oracle {r_ref:.2e})")
        assert rr <= 1e-4 or rr <= 1.1 * r_ref + 1e-6, (name, rr, r_ref)
    # the samples whose firing pattern the library (one handle over the whole batch) and both oracles share: 1e-4
    core = Core(s, params, max_batch=B)
    core.forward(obs)
    bad = _flipped(core, o64, s, B) | _flipped(o32, o64, s, B)
    say(f"   samples with a neuron on the other side of its threshold: {np.flatnonzero(bad).tolist()}")
    assert bad.sum() <= 4
    del core
    d = dl.copy()
    d[bad] = 0.0
    opt.zero_grad()
    ln = nat(x)
    ln.backward(torch.as_tensor(d).cuda())
    for name, g, a, w in zip(NAMES, grad_arrays(nat), o32.backward(d), o64.backward(d)):
        rr, r_32 = rel(g.reshape(-1), w), rel(g.reshape(-1), a)
        say(f"   shared pattern: grad {name:6s} rel {rr:.2e} (float64), {r_32:.2e} (float32 oracle)")
        assert rr <= 1e-4 and r_32 <= 1e-4, (name, rr, r_32)
    before = [t.clone() for t in (nat.w.data, nat.gain.data, nat.out.weight.data)]
    opt.step()
    after = [nat.w.data, nat.gain.data, nat.out.weight.data]
    moved = [float((a - b).abs().max()) for a, b in zip(after, before)]
    out_of_play = torch.ones(nat.w.numel(), dtype=torch.bool, device="cuda")
    out_of_play[nat._wmap] = False
    still = float((nat.w.data - before[0])[out_of_play].abs().max()) if bool(out_of_play.any()) else 0.0
    say(f"   Adam at 1e-3: strength moved {moved[0]:.2e}, gain {moved[1]:.2e}, read-out {moved[2]:.2e}; "
        f"not in play {still:.1e}")
    assert 5e-4 < moved[0] < 2e-3 and still == 0.0 and 1e-4 < moved[1] < 6e-4
    sd = opt.state_dict()
    assert sd["adam_t"] == 1 and len(sd["m"]) == 7
    nat._session.close()


def _flipped(a, b, s: dict, B: int) -> np.ndarray:
    """Per sample: some neuron fires in one forward and not in the other (the state getters of Core / Oracle)."""
    bad = np.zeros(B, bool)
    for layer in range(s["hops"] + 1):
        rows = s["sizes"][layer]
        ha = a.state(layer, 0, rows, B) if isinstance(a, Core) else a.state(layer, 0, rows)
        hb = b.state(layer, 0, rows)
        bad |= ((ha > 0) != (hb > 0)).any(0)
    return bad


def test_shipped_b4096_forward_against_oracle(gpu_lib, shipped):
    """The benchmark batch on the shipped network: logits against both oracles, argmax, and 64-sample slices bit for
    bit against the whole batch."""
    f, s, params = shipped
    B = 4096
    obs = (0.5 * np.random.default_rng(50).standard_normal((B, 517))).astype(np.float32)
    core = Core(s, params, max_batch=B)
    got = core.forward(obs)
    say("shipped B 4096: oracles forward")
    raw = net_bytes(s)
    w32 = Oracle(raw, params, "f32").forward(obs)
    w64 = Oracle(raw, params, "f64").forward(obs)
    r32, r64 = rel(got, w32), rel(got, w64)
    ok, ties = argmax_agrees(got, w64)
    say(f"   logits rel {r32:.2e} (float32 oracle), {r64:.2e} (float64), near ties {ties}, "
        f"argmax differs on {int((got.argmax(1) != w64.argmax(1)).sum())}")
    assert r32 <= 4e-6 and r64 <= 1e-5 and ok
    for start in (0, 2048, B - 64):
        assert np.array_equal(core.forward(obs[start:start + 64]), got[start:start + 64]), start


@pytest.mark.parametrize("B", [512, 4096])
def test_shipped_teaching_step_against_oracle(gpu_lib, shipped, B):
    """Forward, KL loss and backward on the shipped network at B = 512 and at the benchmark batch, 4096.  Gradients:
    on the samples whose firing
    pattern the library, the float32 oracle and the float64 oracle share, within 1e-4 of float64 and of the float32
    oracle; over the whole batch within 1e-4 of float64 or no further from it than 1.1 x the float32 oracle's own
    distance + 1e-6 (a pre-activation within rounding of its threshold fires in one float32 sum order and not in
    another, and then the two gradients differ by that neuron's whole term)."""
    f, s, params = shipped
    rng = np.random.default_rng(51)
    obs = (0.5 * rng.standard_normal((B, 517))).astype(np.float32)
    teacher = (rng.standard_normal((B, 90)) * 2).astype(np.float32)
    core = Core(s, params, max_batch=B)
    got = core.forward(obs)
    raw = net_bytes(s)
    o32, o64 = Oracle(raw, params, "f32"), Oracle(raw, params, "f64")
    w32 = o32.forward(obs)
    o64.forward(obs)
    dl, _, _ = o32.loss(w32, teacher, 1.0)
    bad = _flipped(core, o64, s, B) | _flipped(o32, o64, s, B)
    say(f"   samples with a neuron on the other side of its threshold (library or float32 oracle): {int(bad.sum())}")
    assert bad.sum() <= B // 50
    d = dl.copy()
    d[bad] = 0.0
    core.zero_grad()
    core.backward(d)
    for name, g, a, w in zip(NAMES, core.get(4), o32.backward(d), o64.backward(d)):
        r, r_32 = rel(g, w), rel(g, a)
        say(f"   shared pattern: grad {name:6s} rel {r:.2e} (float64), {r_32:.2e} (float32 oracle)")
        assert r <= 1e-4 and r_32 <= 1e-4, (name, r, r_32)
    core.zero_grad()
    core.backward(dl)
    for name, g, a, w in zip(NAMES, core.get(4), o32.backward(dl), o64.backward(dl)):
        r, r_ref = rel(g, w), rel(a, w)
        say(f"   whole batch: grad {name:6s} rel {r:.2e} (float32 oracle {r_ref:.2e})")
        assert r <= 1e-4 or r <= 1.1 * r_ref + 1e-6, (name, r, r_ref)


def test_shipped_b4096_gradients_add_up_over_pieces(gpu_lib, shipped):
    """The benchmark batch's gradients on the shipped network equal the sum of those of its four 1024-sample
    pieces (each sum in its own tile order) to 1e-5, and a piece's logits are those of the whole batch bit for bit:
    no sample's result depends on the batch it is in."""
    f, s, params = shipped
    B = 4096
    rng = np.random.default_rng(52)
    obs = (0.5 * rng.standard_normal((B, 517))).astype(np.float32)
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    core = Core(s, params, max_batch=B)
    whole_lg = core.forward(obs)
    core.zero_grad()
    core.backward(dl)
    whole = core.get(4)
    core.zero_grad()
    for i in range(0, B, 1024):
        assert np.array_equal(core.forward(obs[i:i + 1024]), whole_lg[i:i + 1024]), i
        core.backward(dl[i:i + 1024])
    for name, a, b in zip(NAMES, core.get(4), whole):
        r = rel(a, b)
        say(f"   grad {name:6s} 4 x 1024 vs 4096 rel {r:.2e}")
        assert r <= 1e-5, (name, r)
