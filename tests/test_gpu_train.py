"""The KL loss, Adam, the fused teaching step and the Python API (NativeFlyActor / NativeAdam / HopHip) on the GPU,
against the oracle and against PyTorch in float64."""
from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from conftest import lively, toy
from flyguy_amd._lib import LibraryError, call
from flyguy_amd.export import net_bytes, params_from_torch, structure
from flyguy_amd.fly import FlyActor
from flyguy_amd.fly_native import NativeFlyActor, grad_arrays
from flyguy_amd.synth import scaled_3hop
from gpu_helpers import NAMES, Core, rel, say
from oracle.oracle import Oracle

pytestmark = pytest.mark.gpu


def test_kl_loss(gpu_lib):
    say("kl loss")
    s, params = scaled_3hop(64)
    core = Core(s, params, max_batch=256)
    rng = np.random.default_rng(0)
    lg = (rng.standard_normal((256, 90)) * 3).astype(np.float32)
    tl = (rng.standard_normal((256, 90)) * 2).astype(np.float32)
    lg[3, 4] = lg[3, 8] = 30.0
    o = Oracle(net_bytes(s), params, "f64")
    lg_d, tl_d = torch.as_tensor(lg).cuda(), torch.as_tensor(tl).cuda()      # (kept alive while the kernel runs)
    for it in (1.0, 0.5):
        dl = torch.empty(256, 90, device="cuda")
        st = torch.zeros(2, device="cuda")
        call("fc_kl_loss", core.h, lg_d.data_ptr(), tl_d.data_ptr(), 256, it, dl.data_ptr(), st.data_ptr())
        want_dl, want_kl, want_agree = o.loss(lg, tl, it)
        assert rel(dl.cpu().numpy(), want_dl) <= 1e-5
        assert abs(float(st[0]) - want_kl) <= 1e-5 * abs(want_kl)
        assert float(st[1]) == want_agree


def test_adam_step(gpu_lib):
    say("adam")
    s, params = scaled_3hop(64)
    core = Core(s, params, max_batch=64)
    rng = np.random.default_rng(2)
    o = Oracle(net_bytes(s), params, "f32")
    p = [a.astype(np.float32).copy() for a in params]
    m = [np.zeros_like(a) for a in p]
    v = [np.zeros_like(a) for a in p]
    ema = [a.copy() for a in p]
    lrs = [1e-3, 3e-4, 3e-4, 1e-3, 1e-3, 1e-3, 1e-3]
    for t in range(1, 4):
        g = [rng.standard_normal(a.shape).astype(np.float32) for a in p]
        core.set(4, g)
        norm = float(call("fc_step", core.h, 1e-3, 3e-4, 1e-3, 0.0, 0.99))
        assert norm == 0.0
        for i in range(7):
            o.adam(p[i], g[i], m[i], v[i], ema[i], lrs[i], t, 1.0, 0.99)
    for i, (gp, ge, gm, gv) in enumerate(zip(core.get(0), core.get(1), core.get(2), core.get(3))):
        assert np.abs(gp - p[i]).max() <= 1e-6, NAMES[i]
        assert np.abs(ge - ema[i]).max() <= 1e-6, NAMES[i]
        assert np.abs(gm - m[i]).max() <= 1e-6 and np.abs(gv - v[i]).max() <= 1e-6
    assert int(call("fc_adam_t", core.h, -1)) == 3
    # clipping: the norm is reported and the step scaled
    g = [np.full(a.shape, 10.0, np.float32) for a in p]
    core.set(4, g)
    want = float(np.sqrt(sum(float((x.astype(np.float64) ** 2).sum()) for x in g)))
    got = float(call("fc_grad_norm", core.h))
    assert abs(got - want) <= 1e-4 * want
    assert abs(float(call("fc_step", core.h, 1e-3, 3e-4, 1e-3, 1.0, 0.99)) - want) <= 1e-4 * want


def test_teach_step_matches_its_parts(gpu_lib):
    say("teach step")
    s, params = scaled_3hop(32)
    B = 128
    rng = np.random.default_rng(4)
    obs = rng.standard_normal((B, 517)).astype(np.float32)
    tl = (rng.standard_normal((B, 90)) * 2).astype(np.float32)
    a = Core(s, params, max_batch=B)
    b = Core(s, params, max_batch=B)
    st = torch.zeros(2, device="cuda")
    x, t = torch.as_tensor(obs).cuda(), torch.as_tensor(tl).cuda()
    for _ in range(2):
        call("fc_teach_step", a.h, x.data_ptr(), t.data_ptr(), B, 1.0, 1e-3, 3e-4, 1e-3, 0.0, 0.999, st.data_ptr())
        lg = torch.as_tensor(b.forward(obs)).cuda()
        dl = torch.empty(B, 90, device="cuda")
        st2 = torch.zeros(2, device="cuda")
        call("fc_kl_loss", b.h, lg.data_ptr(), t.data_ptr(), B, 1.0, dl.data_ptr(), st2.data_ptr())
        b.zero_grad()
        b.backward(dl.cpu().numpy())
        call("fc_step", b.h, 1e-3, 3e-4, 1e-3, 0.0, 0.999)
        assert torch.equal(st, st2)
    for pa, pb in zip(a.get(0), b.get(0)):
        assert np.array_equal(pa, pb)
    # against the oracle: the loss of the first step
    o = Oracle(net_bytes(s), params, "f64")
    _, kl, _ = o.loss(o.forward(obs), tl)
    c = Core(s, params, max_batch=B)
    call("fc_teach_step", c.h, x.data_ptr(), t.data_ptr(), B, 1.0, 1e-3, 3e-4, 1e-3, 0.0, 0.999, st.data_ptr())
    assert abs(float(st[0]) - kl) <= 1e-5 * abs(kl)


def test_bad_batches_are_refused(gpu_lib):
    s, params = scaled_3hop(64)
    core = Core(s, params, max_batch=64)
    for B in (48, 96, 0):
        with pytest.raises(LibraryError):
            core.forward(np.zeros((B, 517), np.float32)) if B else call("fc_forward", core.h, 0, 0, 0, 0)


def _torch_reference(f, obs, R):
    """Logits and gradients of the PyTorch formulation in float64 on the CPU."""
    g = copy.deepcopy(f).double()
    g.zero_grad()
    out = g(torch.as_tensor(obs).double())
    ((out * torch.as_tensor(R).double()).sum() + 0.1 * out.pow(2).sum()).backward()
    return out.detach().numpy(), g


def test_native_actor_like_core_check(gpu_lib):
    """The checks of flyguy/native/core_check.py: logits and the seven gradients against the PyTorch path, one
    piece and several pieces (batch 160, max_batch 64), then one Adam step (strengths not in play unchanged) and
    the optimiser state round trip."""
    say("native actor")
    torch.manual_seed(0)
    base = lively(FlyActor(toy("b"), 517, 90, hops=3, fan=16))
    nat = NativeFlyActor(toy("b"), 517, 90, hops=3, fan=16, max_batch=64)
    nat.load_state_dict(base.state_dict())
    nat = nat.cuda()
    rng = np.random.default_rng(0)
    obs = (rng.standard_normal((160, 517)) * 0.5).astype(np.float32)
    R = rng.standard_normal((160, 90)).astype(np.float32)
    opt = nat.native_adam(1e-3, 0.0)
    assert opt is not None
    for n in (64, 160):
        want_lg, ref = _torch_reference(base, obs[:n], R[:n])
        opt.zero_grad()
        ln = nat(torch.as_tensor(obs[:n]).cuda())
        ((ln * torch.as_tensor(R[:n]).cuda()).sum() + 0.1 * ln.pow(2).sum()).backward()
        assert rel(ln.detach().cpu().numpy(), want_lg) <= 1e-5
        got = grad_arrays(nat)
        want = [ref.w.grad.numpy()[nat._wmap.cpu().numpy()], ref.gain.grad.numpy(), ref.theta.grad.numpy(),
                ref.in_w.grad.numpy(), ref.in_b.grad.numpy(), ref.out.weight.grad.numpy().reshape(-1),
                ref.out.bias.grad.numpy()]
        for name, g, w in zip(NAMES, got, want):
            assert rel(g.reshape(-1), w) <= 1e-4, (n, name, rel(g.reshape(-1), w))
    before = nat.w.data.clone()
    opt.step()
    moved = (nat.w.data - before).abs()
    out_of_play = torch.ones(nat.w.numel(), dtype=torch.bool, device="cuda")
    out_of_play[nat._wmap] = False
    assert float(moved[out_of_play].max()) == 0.0
    assert 5e-4 < float(moved.max()) < 2e-3
    sd = opt.state_dict()
    assert sd["adam_t"] == 1 and len(sd["m"]) == 7
    opt.load_state_dict(copy.deepcopy(sd))
    assert int(call("fc_adam_t", nat._core, -1)) == 1
    # a copy is a plain FlyActor with the same weights
    cp = copy.deepcopy(nat)
    assert type(cp) is FlyActor and torch.equal(cp.w, nat.w)
    # without gradients: the library, pieces of max_batch
    with torch.no_grad():
        a = nat(torch.as_tensor(obs).cuda())
    want_lg, _ = _torch_reference(cp.cpu(), obs, R)
    assert rel(a.cpu().numpy(), want_lg) <= 1e-5


@pytest.mark.parametrize("hops", [1, 5])
def test_native_actor_other_depths(gpu_lib, hops):
    """NativeFlyActor on networks of one and five hops: logits and the seven gradients against the PyTorch path in
    float64, in one piece and in pieces of max_batch (batch 160, max_batch 64)."""
    say(f"native actor, {hops} hops")
    torch.manual_seed(1)
    base = lively(FlyActor(toy("b"), 517, 90, hops=hops, fan=16), seed=hops)
    nat = NativeFlyActor(toy("b"), 517, 90, hops=hops, fan=16, max_batch=64)
    nat.load_state_dict(base.state_dict())
    nat = nat.cuda()
    rng = np.random.default_rng(hops)
    obs = (rng.standard_normal((160, 517)) * 0.5).astype(np.float32)
    R = rng.standard_normal((160, 90)).astype(np.float32)
    opt = nat.native_adam(1e-3, 0.0)
    assert opt is not None
    for n in (64, 160):
        want_lg, ref = _torch_reference(base, obs[:n], R[:n])
        opt.zero_grad()
        ln = nat(torch.as_tensor(obs[:n]).cuda())
        ((ln * torch.as_tensor(R[:n]).cuda()).sum() + 0.1 * ln.pow(2).sum()).backward()
        assert rel(ln.detach().cpu().numpy(), want_lg) <= 1e-5
        got = grad_arrays(nat)
        want = [ref.w.grad.numpy()[nat._wmap.cpu().numpy()], ref.gain.grad.numpy(), ref.theta.grad.numpy(),
                ref.in_w.grad.numpy(), ref.in_b.grad.numpy(), ref.out.weight.grad.numpy().reshape(-1),
                ref.out.bias.grad.numpy()]
        for name, g, w in zip(NAMES, got, want):
            assert rel(g.reshape(-1), w) <= 1e-4, (hops, n, name, rel(g.reshape(-1), w))


@pytest.mark.parametrize("hops", [3, 1, 2, 5])
def test_hop_hip_matches_torch(gpu_lib, hops):
    """HopHip (the HopCuda interface): output and both gradients of every hop against the sparse product in float64,
    then the whole actor through HopHip against the PyTorch path, on networks of one to five hops."""
    say(f"hop hip, {hops} hops")
    from flyguy_amd.fly_hip import HopHip
    torch.manual_seed(0)
    f = lively(FlyActor(toy("b"), 517, 90, hops=hops, fan=16))
    B = 64
    for k in range(1, hops + 1):
        n_src = f.sizes[k - 1]
        h = torch.rand(n_src, B, dtype=torch.float64)
        w = f.w.detach()[getattr(f, f"e{k}")].double()
        crow, col = getattr(f, f"crow{k}"), getattr(f, f"ci{k}")
        a = torch.sparse_csr_tensor(crow, col.long(), w, size=(len(crow) - 1, n_src))
        want = (a @ h).numpy()
        gz = torch.randn(len(crow) - 1, B, dtype=torch.float64)
        want_gh = (a.t() @ gz).numpy()
        r, c = getattr(f, f"r{k}"), getattr(f, f"c{k}")
        want_gw = (gz[r] * h[c]).sum(1).numpy()
        wd = w.float().cuda().requires_grad_(True)
        hd = h.float().cuda().requires_grad_(True)
        out = HopHip.apply(wd, hd, crow.cuda(), col.cuda(), getattr(f, f"tcrow{k}").cuda(), getattr(f, f"tci{k}").cuda(),
                           getattr(f, f"tperm{k}").cuda(), False)
        out.backward(gz.float().cuda())
        assert rel(out.detach().cpu().numpy(), want) <= 1e-5
        assert rel(hd.grad.cpu().numpy(), want_gh) <= 1e-5
        assert rel(wd.grad.cpu().numpy(), want_gw) <= 1e-5
    # the whole actor through HopHip against the PyTorch path
    f.kernel = "hip"
    x = torch.randn(64, 517)
    g = copy.deepcopy(f).cuda()
    got = g(x.cuda())
    ref = copy.deepcopy(f)
    ref.kernel = "torch"
    ref_out = ref.double()(x.double())
    assert rel(got.detach().cpu().numpy(), ref_out.detach().numpy()) <= 1e-5


def _half_case(a, r, c, w, n_src, n_rows, B, crow, col, tcrow, tcol, tperm, seed):
    """One HopHip(half=True) product and its backward against the reference's half arithmetic in float64:
    states rounded to binary16, the output gradient divided by its largest magnitude and rounded to binary16,
    products rescaled (fly_cuda.py:93, 100-114)."""
    from flyguy_amd.fly_hip import HopHip
    g = torch.Generator().manual_seed(seed)
    h32 = torch.rand(n_src, B, generator=g)
    gz32 = torch.randn(n_rows, B, generator=g)
    hs = h32.half().double()
    scale = gz32.abs().max().clamp_min(1e-30)
    gzs = (gz32 / scale).half().double()
    want = (a @ hs).numpy()
    want_gh = ((a.t() @ gzs) * float(scale)).numpy()
    want_gw = ((gzs[r] * hs[c]).sum(1) * float(scale)).numpy()
    wd = w.float().cuda().requires_grad_(True)
    hd = h32.cuda().requires_grad_(True)
    out = HopHip.apply(wd, hd, crow.cuda(), col.cuda(), tcrow.cuda(), tcol.cuda(), tperm.cuda(), True)
    out.backward(gz32.cuda())
    for name, got, ref in (("out", out, want), ("gh", hd.grad, want_gh), ("gw", wd.grad, want_gw)):
        r_ = rel(got.detach().cpu().numpy(), ref)
        say(f"      half B {B} {name} rel {r_:.2e}")
        assert r_ <= 1e-5, (name, B, r_)


@pytest.mark.parametrize("hops", [3, 5])
def test_hop_hip_half_matches_reference_rounding(gpu_lib, hops):
    """HopHip(half=True), the fp16 variant of HopCuda: relative to the largest entry <= 1e-5 (float32 sums of the
    same binary16 operands), on every hop of toy networks of three and five hops and on a hop of the scaled benchmark
    shape whose heavy rows are split, at B = 64 and at B = 96 (a 64-sample tile that is half past the batch)."""
    say(f"hop hip half, {hops} hops")
    from flyguy_amd.synth import scaled_3hop
    torch.manual_seed(0)
    f = lively(FlyActor(toy("b"), 517, 90, hops=hops, fan=16))
    for B in (64, 96):
        for k in range(1, hops + 1):
            n_src, crow, col = f.sizes[k - 1], getattr(f, f"crow{k}"), getattr(f, f"ci{k}")
            w = f.w.detach()[getattr(f, f"e{k}")].double()
            a = torch.sparse_csr_tensor(crow, col.long(), w, size=(len(crow) - 1, n_src))
            _half_case(a, getattr(f, f"r{k}"), getattr(f, f"c{k}"), w, n_src, len(crow) - 1, B, crow, col,
                       getattr(f, f"tcrow{k}"), getattr(f, f"tci{k}"), getattr(f, f"tperm{k}"), 10 * B + k)
    if hops != 3:
        return
    s, params = scaled_3hop(16)
    h = s["hop"][1]
    crow = torch.as_tensor(np.asarray(h["crow"], np.int64))
    col = torch.as_tensor(np.asarray(h["col"], np.int32))
    E = len(col)
    widx, twidx = np.asarray(h["widx"]), np.asarray(h["twidx"])
    inv = np.full(int(widx.max()) + 1, -1, np.int64)
    inv[widx] = np.arange(E)                                  # weight index -> CSR edge
    tperm = torch.as_tensor(inv[twidx])                       # CSC position -> CSR edge
    assert (tperm >= 0).all()
    rows_t = np.repeat(np.arange(len(crow) - 1), np.diff(np.asarray(h["crow"])))
    w = torch.as_tensor(params[0][widx].astype(np.float64))
    n_src, n_rows = s["sizes"][1], s["sizes"][2]
    a = torch.sparse_csr_tensor(crow, col.long(), w, size=(n_rows, n_src))
    _half_case(a, torch.as_tensor(rows_t), col.long(), w, n_src, n_rows, 96, crow, col,
               torch.as_tensor(np.asarray(h["tcrow"], np.int64)), torch.as_tensor(np.asarray(h["tcol"], np.int32)),
               tperm, 7)
