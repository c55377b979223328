"""The benchmark configurations at their own sizes, and the reference's own entry path, on the GPU.

  * float32 at B = 4096 on the synthetic 3-hop network (the benchmark batch): logits, KL loss, its logits gradient
    and all seven weight gradients against the float32 oracle (the reference's arithmetic); gradient additivity of
    eight pieces of 512 against the whole batch;
  * float32 at B = 16384 on the synthetic network and its Erdos-Renyi control: batch independence of the logits
    and additivity of the gradients over four pieces of 4096;
  * bfloat16 states on the full-size synthetic network and on its Erdos-Renyi control: logits and all seven
    gradients against the bfloat16 restatement (oracle/core16.py) at B = 128; at B = 16384 (the bfloat16 benchmark
    batch) batch independence of the logits and additivity of the gradients over four pieces of 4096;
  * the whole-connectome graph at its configured B = 1024: batch independence bit-exact against 64-sample slices,
    gradient additivity of four pieces of 256;
  * NativeFlyActor on the whole-connectome graph at B = 1 and B = 37: batches that are padded to 32 in the forward
    (the last observation repeated) and in the backward (zero rows), fly_native.py:53,200, against the float64
    oracle at the unpadded batch;
  * fc_create(path) on a NET.bin file, with the library opened by ctypes exactly as the reference binds it
    (fly_native.py:136-145): the ten argtypes, then forward, backward, gradient length and one Adam step.

Bars (relative to the largest entry, as flyguy/native/core_check.py:59 measures): float32 logits <= 1e-5 (4e-6 vs
the float32 oracle), gradients <= 1e-4; bfloat16 logits <= 1e-3, gradients <= 1e-2 (a float32 sum and the float64
restatement may round a state to neighbouring bfloat16 values); additivity <= 1e-5; batch independence bit-exact.
"""
from __future__ import annotations

import ctypes
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch

from flyguy_amd._lib import LIB_PATH, call
from flyguy_amd.export import net_bytes, param_sizes, params_from_torch, structure
from flyguy_amd.synth import synth_3hop, whole_connectome
from gpu_helpers import NAMES, Core, argmax_agrees, rel, say
from oracle.core16 import Core16
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu
BF16 = 1


@pytest.fixture(scope="module")
def lognormal():
    say("synthetic 3-hop network (lognormal in-degree)")
    return synth_3hop()


@pytest.fixture(scope="module")
def er():
    say("synthetic 3-hop network (Erdos-Renyi control)")
    return synth_3hop(kind="er")


def _grads(core: Core, dl: np.ndarray) -> list[np.ndarray]:
    core.zero_grad()
    core.backward(dl)
    return core.get(4)


# ------------------------------------------------------------------------------------------------ float32, B = 4096
def _flipped(core: Core, o: Oracle, s: dict, B: int) -> np.ndarray:
    """Per sample: whether some neuron fires (h > 0) in the library's forward and not in the oracle's, or the other
    way round.  A neuron's gradient passes only where it fires, so at such a (neuron, sample) the two backward passes
    differ by a whole term, however small the two pre-activations' difference was."""
    bad = np.zeros(B, bool)
    for layer in range(s["hops"] + 1):
        rows = s["sizes"][layer]
        bad |= ((core.state(layer, 0, rows, B) > 0) != (o.state(layer, 0, rows) > 0)).any(0)
    return bad


def test_fp32_b4096_teaching_step_against_oracle(gpu_lib, lognormal):
    """The benchmark's teaching step at its batch: forward, KL loss, backward.  Logits and the loss against the
    oracle; the gradients against the float64 and the float32 oracle on the samples whose firing pattern the library
    and both oracles share (at B = 4096 a handful of (neuron, sample) pre-activations sit within rounding of the
    threshold, and the reference's own float32 arithmetic flips them too: its gradients then differ from float64 by
    up to 9e-4), and over the whole batch within 1e-4 of float64 or no further from it than 1.1 x the float32
    oracle's own distance + 1e-6."""
    s, params = lognormal
    B = 4096
    rng = np.random.default_rng(40)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    teacher = (rng.standard_normal((B, 90)) * 2).astype(np.float32)
    core = Core(s, params, max_batch=B)
    x, t = torch.as_tensor(obs).cuda(), torch.as_tensor(teacher).cuda()
    lg = torch.empty(B, 90, device="cuda")
    call("fc_forward", core.h, x.data_ptr(), B, lg.data_ptr(), 0)
    dl = torch.empty(B, 90, device="cuda")
    st = torch.zeros(2, device="cuda")
    call("fc_kl_loss", core.h, lg.data_ptr(), t.data_ptr(), B, 1.0, dl.data_ptr(), st.data_ptr())
    got_lg, got_dl = lg.cpu().numpy(), dl.cpu().numpy()
    say("fp32 B 4096: oracles forward")
    raw = net_bytes(s)
    o32, o64 = Oracle(raw, params, "f32"), Oracle(raw, params, "f64")
    w32, w64 = o32.forward(obs), o64.forward(obs)
    r32, r64 = rel(got_lg, w32), rel(got_lg, w64)
    say(f"   logits rel {r32:.2e} (float32 oracle), {r64:.2e} (float64)")
    assert r32 <= 4e-6 and r64 <= 1e-5
    ok, ties = argmax_agrees(got_lg, w64)
    assert ok, ties
    want_dl, want_kl, _ = o32.loss(w32, teacher, 1.0)
    assert rel(got_dl, want_dl) <= 1e-5
    assert abs(float(st[0]) - want_kl) <= 1e-5 * abs(want_kl)
    bad = _flipped(core, o64, s, B)
    bad32 = _flipped_oracles(o32, o64, s, B)
    say(f"   samples with a neuron on the other side of its threshold: {int(bad.sum())} (library), "
        f"{int(bad32.sum())} (float32 oracle), {int((bad | bad32).sum())} (either), of {B}")
    assert bad.sum() <= B // 100
    # (1) the samples whose firing pattern the library and both oracles share: the gradients to the 1e-4 bar against
    # float64, and against the float32 oracle (the reference's own arithmetic) directly
    d = got_dl.copy()
    d[bad | bad32] = 0.0
    core.zero_grad()
    core.backward(d)
    say("fp32 B 4096: oracles backward, shared firing pattern")
    for name, g, a, w in zip(NAMES, core.get(4), o32.backward(d), o64.backward(d)):
        r, r_32 = rel(g, w), rel(g, a)
        say(f"   grad {name:6s} rel {r:.2e} (float64), {r_32:.2e} (float32 oracle)")
        assert r <= 1e-4 and r_32 <= 1e-4, (name, r, r_32)
    # (2) the whole batch: within 1e-4 of float64, or no further from it than the reference's own float32 arithmetic
    # is (1.1 x its distance + 1e-6): a threshold flip changes a gradient by the neuron's whole term
    core.zero_grad()
    core.backward(got_dl)
    got = core.get(4)
    say("fp32 B 4096: whole batch")
    for name, g, a, w in zip(NAMES, got, o32.backward(got_dl), o64.backward(got_dl)):
        r, r_ref = rel(g, w), rel(a, w)
        say(f"   grad {name:6s} rel {r:.2e} (float32 oracle {r_ref:.2e})")
        assert r <= 1e-4 or r <= 1.1 * r_ref + 1e-6, (name, r, r_ref)


def _flipped_oracles(a: Oracle, b: Oracle, s: dict, B: int) -> np.ndarray:
    bad = np.zeros(B, bool)
    for layer in range(s["hops"] + 1):
        rows = s["sizes"][layer]
        bad |= ((a.state(layer, 0, rows) > 0) != (b.state(layer, 0, rows) > 0)).any(0)
    return bad


def test_fp32_b4096_gradients_add_up_over_eight_pieces(gpu_lib, lognormal):
    s, params = lognormal
    B = 4096
    core = Core(s, params, max_batch=B)
    rng = np.random.default_rng(41)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    core.forward(obs)
    whole = _grads(core, dl)
    core.zero_grad()
    for i in range(0, B, 512):
        core.forward(obs[i:i + 512])
        core.backward(dl[i:i + 512])
    pieces = core.get(4)
    for name, a, b in zip(NAMES, pieces, whole):
        r = rel(a, b)
        say(f"   grad {name:6s} 8 x 512 vs 4096 rel {r:.2e}")
        assert r <= 1e-5, (name, r)


# ------------------------------------------------------------------------------------------------ bfloat16
@pytest.mark.parametrize("graph", ["lognormal", "er"])
def test_bf16_full_size_against_oracle(gpu_lib, request, graph):
    s, params = request.getfixturevalue(graph)
    B = 128
    say(f"bf16 full-size {graph}, B {B}")
    obs = np.random.default_rng(42).standard_normal((B, 517)).astype(np.float32)
    core = Core(s, params, max_batch=B, flags=BF16)
    got = core.forward(obs)
    o = Core16(s, params)
    want = o.forward(obs)
    assert np.isfinite(got).all()
    r = rel(got, want)
    ok, ties = argmax_agrees(got, want, margin=1e-2 * np.abs(want).max())
    say(f"   logits rel {r:.2e}, near ties {ties}")
    assert r <= 1e-3 and ok
    dl = ((np.random.default_rng(43).standard_normal(got.shape) + 0.2 * got) / B).astype(np.float32)
    for name, g, w in zip(NAMES, _grads(core, dl), o.backward(dl)):
        r = rel(g, w)
        say(f"   grad {name:6s} rel {r:.2e}")
        assert r <= 1e-2, (name, r)


@pytest.mark.parametrize("graph", ["lognormal", "er"])
def test_bf16_b16384_batch_independence_and_additivity(gpu_lib, request, graph):
    s, params = request.getfixturevalue(graph)
    B = 16384
    say(f"bf16 full-size {graph}, B {B}")
    core = Core(s, params, max_batch=B, flags=BF16)
    rng = np.random.default_rng(44)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    big = core.forward(obs)
    for start in (0, 8192, B - 64):
        assert np.array_equal(core.forward(obs[start:start + 64]), big[start:start + 64]), start
    perm = rng.permutation(B)
    assert np.array_equal(core.forward(obs[perm]), big[perm])
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    core.forward(obs)
    whole = _grads(core, dl)
    core.zero_grad()
    for i in range(0, B, 4096):
        core.forward(obs[i:i + 4096])
        core.backward(dl[i:i + 4096])
    for name, a, b in zip(NAMES, core.get(4), whole):
        r = rel(a, b)
        say(f"   grad {name:6s} 4 x 4096 vs 16384 rel {r:.2e}")
        assert r <= 1e-5, (name, r)



@pytest.mark.parametrize("graph", ["lognormal", "er"])
def test_fp32_b16384_batch_independence_and_additivity(gpu_lib, request, graph):
    """Float32 at B = 16384 (512 tiles: the plug's LDS split, the last hop's LDS backward and the XCD mapping at four
    times the benchmark's tiles): a sample's logits bit-identical in 32-sample slices and under a permutation of the
    batch; the gradients of four pieces of 4096 add up to the whole batch's (<= 1e-5)."""
    s, params = request.getfixturevalue(graph)
    B = 16384
    say(f"float32 full-size {graph}, B {B}")
    core = Core(s, params, max_batch=B)
    rng = np.random.default_rng(45)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    big = core.forward(obs)
    assert np.isfinite(big).all()
    for start in (0, 8192, B - 32):
        assert np.array_equal(core.forward(obs[start:start + 32]), big[start:start + 32]), start
    perm = rng.permutation(B)
    assert np.array_equal(core.forward(obs[perm]), big[perm])
    dl = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    core.forward(obs)
    whole = _grads(core, dl)
    core.zero_grad()
    for i in range(0, B, 4096):
        core.forward(obs[i:i + 4096])
        core.backward(dl[i:i + 4096])
    for name, a, b in zip(NAMES, core.get(4), whole):
        r = rel(a, b)
        say(f"   grad {name:6s} 4 x 4096 vs 16384 rel {r:.2e}")
        assert r <= 1e-5, (name, r)

# ------------------------------------------------------------------------------------------------ whole connectome
@pytest.fixture(scope="module")
def connectome():
    """A NativeFlyActor (on the CPU) over the whole-connectome graph, with its structure and initial weights."""
    from flyguy_amd.fly_native import NativeFlyActor
    say("whole connectome: graph and index")
    torch.manual_seed(0)
    f = NativeFlyActor(whole_connectome(), 517, 90, hops=3, fan=16, max_batch=64)
    s = structure(f)
    return f, s, params_from_torch(f, s)


def test_whole_connectome_against_oracle(gpu_lib, connectome):
    """The whole-connectome case: a synthetic graph of 166,700 neurons and 15,283,167 connections (lognormal(1.8)
    in-degree), indexed by FlyActor as the reference indexes a graph file (hops of 1.55M, 6.0M and 121k
    connections, 6.76M strengths in play), its initial weights; B = 64, through the C-ABI."""
    f, s, params = connectome
    assert s["n_neurons"] == 166_700 and f.n_conn == 15_283_167
    say(f"   hops {[len(h['col']) for h in s['hop']]}, strengths {s['n_w']:,}")
    obs = np.random.default_rng(21).standard_normal((64, 517)).astype(np.float32)
    core = Core(s, params, max_batch=64)
    got = core.forward(obs)
    o64 = Oracle(net_bytes(s), params, "f64")
    want = o64.forward(obs)
    assert rel(got, want) <= 1e-5
    assert rel(got, Oracle(net_bytes(s), params, "f32").forward(obs)) <= 4e-6
    for layer in range(s["hops"] + 1):
        rows = s["sizes"][layer]
        assert rel(core.state(layer, 0, rows, 64), o64.state(layer, 0, rows)) <= 1e-5, layer
    say("whole connectome: backward")
    dl = (np.random.default_rng(22).standard_normal(got.shape) + 0.2 * got).astype(np.float32)
    for name, g, w in zip(NAMES, _grads(core, dl), o64.backward(dl)):
        r = rel(g, w)
        say(f"   grad {name:6s} rel {r:.2e}")
        assert r <= 1e-4, (name, r)


def test_whole_connectome_b1024_independence_and_additivity(gpu_lib, connectome):
    """The whole-connectome case at its configured batch, B = 1024: 64-sample slices give the logits of the whole
    batch bit for bit (so do a permuted batch's), and the gradients of four pieces of 256 add up to the whole
    batch's within 1e-5 (relative to the largest entry)."""
    f, s, params = connectome
    B = 1024
    say(f"whole connectome, B {B}")
    core = Core(s, params, max_batch=B)
    rng = np.random.default_rng(23)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    big = core.forward(obs)
    assert np.isfinite(big).all()
    for start in range(0, B, 64):
        assert np.array_equal(core.forward(obs[start:start + 64]), big[start:start + 64]), start
    perm = rng.permutation(B)
    assert np.array_equal(core.forward(obs[perm]), big[perm])
    dl = ((rng.standard_normal((B, 90)) + 0.2 * big) / B).astype(np.float32)
    core.forward(obs)
    whole = _grads(core, dl)
    core.zero_grad()
    for i in range(0, B, 256):
        core.forward(obs[i:i + 256])
        core.backward(dl[i:i + 256])
    for name, a, b in zip(NAMES, core.get(4), whole):
        r = rel(a, b)
        say(f"   grad {name:6s} 4 x 256 vs 1024 rel {r:.2e}")
        assert r <= 1e-5, (name, r)


@pytest.mark.parametrize("B", [1, 37])
def test_native_actor_padded_batches(gpu_lib, connectome, B):
    """NativeFlyActor.forward with gradients at a batch that is not a multiple of 32 (padded to 32 / 64 inside),
    then the logits' gradient back through the library: logits and the seven gradients against the float64
    oracle at the unpadded batch; and the same forward without gradients."""
    from flyguy_amd.fly_native import grad_arrays
    f, s, params = connectome
    nat = f.cuda()
    say(f"native actor, whole connectome, B {B}")
    rng = np.random.default_rng(100 + B)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    R = rng.standard_normal((B, 90)).astype(np.float32)
    opt = nat.native_adam(1e-3)
    opt.zero_grad()
    x = torch.as_tensor(obs).cuda()
    out = nat(x)
    assert out.shape == (B, 90)
    (out * torch.as_tensor(R).cuda()).sum().backward()
    o = Oracle(net_bytes(s), params, "f64")
    want = o.forward(obs)
    r = rel(out.detach().cpu().numpy(), want)
    say(f"   logits rel {r:.2e}")
    assert r <= 1e-5
    for name, g, w in zip(NAMES, grad_arrays(nat), o.backward(R)):
        r = rel(g.reshape(-1), w)
        say(f"   grad {name:6s} rel {r:.2e}")
        assert r <= 1e-4, (name, r)
    with torch.no_grad():
        again = nat(x)
    assert torch.equal(again, out.detach())


# ------------------------------------------------------------------------------------------------ fc_create(path)
def _reference_binding() -> ctypes.CDLL:
    """The library opened and typed as the reference's NativeFlyActor._ready does it (fly_native.py:136-145)."""
    L = ctypes.CDLL(str(LIB_PATH))
    vp, ci = ctypes.c_void_p, ctypes.c_int
    L.fc_create.restype, L.fc_create.argtypes = vp, [ctypes.c_char_p, ci]
    L.fc_sizes.restype, L.fc_sizes.argtypes = None, [vp, ctypes.POINTER(ctypes.c_longlong)]
    L.fc_copy.restype, L.fc_copy.argtypes = None, [vp, ci, ci, ctypes.POINTER(vp)]
    L.fc_forward.restype, L.fc_forward.argtypes = None, [vp, vp, ci, vp, ci]
    L.fc_zero_grad.restype, L.fc_zero_grad.argtypes = None, [vp]
    L.fc_backward.restype, L.fc_backward.argtypes = None, [vp, vp, ci]
    L.fc_grad_norm.restype, L.fc_grad_norm.argtypes = ctypes.c_float, [vp]
    L.fc_step.restype, L.fc_step.argtypes = ctypes.c_float, [vp] + [ctypes.c_float] * 5
    L.fc_adam_t.restype, L.fc_adam_t.argtypes = ctypes.c_longlong, [vp, ctypes.c_longlong]
    return L


def test_fc_create_from_path_with_the_reference_binding(gpu_lib, lognormal):
    s, params = lognormal
    B = 256
    L = _reference_binding()
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "net.bin"
        path.write_bytes(net_bytes(s))
        core = L.fc_create(str(path).encode(), B)
    if not core:
        call("fc_create")
    sizes = (ctypes.c_longlong * 10)()
    L.fc_sizes(core, sizes)
    assert [int(v) for v in sizes[:7]] == param_sizes(s)
    assert [int(v) for v in sizes[7:]] == [517, 90, B]
    ts = [torch.as_tensor(np.ascontiguousarray(p, np.float32)).cuda() for p in params]
    ptrs = (ctypes.c_void_p * 7)(*[t.data_ptr() for t in ts])
    L.fc_copy(core, 0, 1, ptrs)
    L.fc_copy(core, 1, 1, ptrs)
    rng = np.random.default_rng(45)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    R = (rng.standard_normal((B, 90)) / B).astype(np.float32)
    x, d = torch.as_tensor(obs).cuda(), torch.as_tensor(R).cuda()
    lg = torch.empty(B, 90, device="cuda")
    L.fc_forward(core, x.data_ptr(), B, lg.data_ptr(), 0)
    lg_ema = torch.empty(B, 90, device="cuda")
    L.fc_forward(core, x.data_ptr(), B, lg_ema.data_ptr(), 1)      # the running average starts as the weights
    L.fc_forward(core, x.data_ptr(), B, lg.data_ptr(), 0)          # (the backward follows the last forward of ema 0)
    L.fc_zero_grad(core)
    L.fc_backward(core, d.data_ptr(), B)
    norm = float(L.fc_grad_norm(core))
    grads = [torch.empty_like(t) for t in ts]
    L.fc_copy(core, 4, 0, (ctypes.c_void_p * 7)(*[t.data_ptr() for t in grads]))
    o = Oracle(net_bytes(s), params, "f64")
    want = o.forward(obs)
    assert rel(lg.cpu().numpy(), want) <= 1e-5
    assert torch.equal(lg, lg_ema)
    want_g = o.backward(R)
    for name, g, w in zip(NAMES, grads, want_g):
        assert rel(g.cpu().numpy(), w) <= 1e-4, name
    want_norm = float(np.sqrt(sum(float((w.astype(np.float64) ** 2).sum()) for w in want_g)))
    assert abs(norm - want_norm) <= 1e-4 * want_norm
    assert float(L.fc_step(core, 1e-3, 3e-4, 1e-3, 0.0, 0.999)) == 0.0
    assert int(L.fc_adam_t(core, -1)) == 1
    after = [torch.empty_like(t) for t in ts]
    L.fc_copy(core, 0, 0, (ctypes.c_void_p * 7)(*[t.data_ptr() for t in after]))
    moved = max(float((a - t).abs().max()) for a, t in zip(after, ts))
    assert 5e-4 < moved < 2e-3                                      # Adam's first step moves by about lr
    call("fc_free", core)
