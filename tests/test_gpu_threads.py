"""Reentrancy of the stack steps: two host threads, each with its own stream, step object
(outputs and workspace) and inputs, call pd_moe_stack_step / pd_lm_stack_step at the same
time; every output must be bit-identical to the same call made alone. The stack steps
fork work onto a per-device helper stream with a shared event pool, so this is the case
where one call's event records could land between another call's record and wait."""

import threading

import pytest
import torch

pytestmark = pytest.mark.gpu

ROUNDS = 4


def _run_pair(device, steps, calls):
    """calls[i]() enqueues thread i's step on the current stream. Runs both once alone,
    then ROUNDS times concurrently from two threads; returns (alone, [concurrent...])."""

    def snapshot(step):
        return {name: t.clone() for name, t in step.outputs().items()}

    alone = []
    for step, call in zip(steps, calls):
        call()
        torch.cuda.synchronize()
        alone.append(snapshot(step))
    streams = [torch.cuda.Stream(device=device) for _ in steps]  # default priority
    errors = []

    def worker(i, barrier):
        try:
            with torch.cuda.stream(streams[i]):
                barrier.wait()
                calls[i]()
        except Exception as e:  # surfaced below
            errors.append(e)

    results = []
    for _ in range(ROUNDS):
        for step in steps:  # poison the outputs so a skipped write cannot pass
            for t in step.outputs().values():
                t.fill_(7 if t.dtype in (torch.int32,) else float("nan"))
        torch.cuda.synchronize()
        barrier = threading.Barrier(len(steps))
        ths = [threading.Thread(target=worker, args=(i, barrier)) for i in range(len(steps))]
        for th in ths:
            th.start()
        for th in ths:
            th.join()
        torch.cuda.synchronize()
        assert not errors, errors
        results.append([snapshot(s) for s in steps])
    return alone, results


def _assert_same(alone, results):
    for r in results:
        for i, (want, got) in enumerate(zip(alone, r)):
            for name in want:
                assert torch.equal(got[name], want[name]), f"thread {i}: {name} differs from the call alone"


class _MoEOut:
    def __init__(self, step):
        self.s = step

    def outputs(self):
        s = self.s
        out = {"losses": s.losses, "d_ci_pre": s.d_ci_pre, "top_idx": s.top_idx}
        for site in ("gate", "up", "down"):
            out["dV_" + site], out["dU_" + site] = s.dV[site], s.dU[site]
        return out


class _LMOut:
    def __init__(self, step):
        self.s = step

    def outputs(self):
        s = self.s
        out = {"losses": s.losses}
        for k in s.dV:
            out["dV_" + k], out["dU_" + k], out["dci_" + k] = s.dV[k], s.dU[k], s.d_ci_pre[k]
        return out


def test_moe_stack_step_two_threads(device):
    from param_decomp_amd.moe_step import MoEStackStep, MoEWeights

    T, d, f, E, k, c, Ln = 1024, 128, 64, 16, 4, 64, 3
    g = torch.Generator(device=device).manual_seed(3)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)

    def weights():
        return MoEWeights(ln=torch.randn(Ln, d, device=device, generator=g) * 0.1,
                          router=rn(Ln, E, d, scale=d**-0.5), Wg=rn(Ln, E, d, f, scale=d**-0.5),
                          Wu=rn(Ln, E, d, f, scale=d**-0.5), Wd=rn(Ln, E, f, d, scale=f**-0.5),
                          Vg=rn(Ln, E, d, c, scale=d**-0.5), Ug=rn(Ln, E, c, f, scale=(E * c)**-0.5),
                          Vu=rn(Ln, E, d, c, scale=d**-0.5), Uu=rn(Ln, E, c, f, scale=(E * c)**-0.5),
                          Vd=rn(Ln, E, f, c, scale=f**-0.5), Ud=rn(Ln, E, c, d, scale=(E * c)**-0.5))

    inputs = []
    for key in ((0, 1), (4, 9)):
        x0 = rn(T, d, scale=1.0)
        ci = (torch.rand(Ln, 3, T, k, c, device=device, generator=g) * 1.6 - 0.3).to(torch.bfloat16)
        inputs.append((x0, weights(), ci, key))
    steps = [MoEStackStep(T, d, f, E, k, c, Ln, device=device) for _ in inputs]
    calls = [lambda s=s, a=a: s.step(*a) for s, a in zip(steps, inputs)]
    alone, results = _run_pair(device, [_MoEOut(s) for s in steps], calls)
    assert not torch.equal(alone[0]["losses"], alone[1]["losses"])
    _assert_same(alone, results)


def test_lm_stack_step_two_threads(device):
    from param_decomp_amd.lm_step import KINDS as K, LMStackStep, LMWeights, site_dims

    B, T, d, H, f, V, Ln = 2, 256, 128, 2, 256, 1000, 2
    C = {"q_proj": 64, "k_proj": 48, "v_proj": 64, "o_proj": 32, "c_fc": 128, "down_proj": 96}
    g = torch.Generator(device=device).manual_seed(5)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)

    def weights():
        Wd, Vd, Ud = {}, {}, {}
        for kk in K:
            din, dout = site_dims(kk, d, H, H, f)
            Wd[kk] = rn(Ln, dout, din, scale=din**-0.5)
            Vd[kk] = rn(Ln, din, C[kk], scale=din**-0.5)
            Ud[kk] = rn(Ln, C[kk], dout, scale=C[kk]**-0.5)
        return LMWeights(wte=rn(V, d, scale=d**-0.5), ln1=torch.ones(Ln, d, device=device),
                         ln2=torch.ones(Ln, d, device=device), norm=torch.ones(d, device=device), W=Wd, V=Vd, U=Ud)

    inputs = []
    for key in ((0, 1), (2, 7)):
        ci = {kk: (torch.rand(Ln, B * T, C[kk], device=device, generator=g) * 1.6 - 0.3).to(torch.bfloat16)
              for kk in K}
        tok = torch.randint(0, V, (B * T,), device=device, generator=g, dtype=torch.int32)
        inputs.append((tok, weights(), ci, key))
    steps = [LMStackStep(B, T, d, H, H, f, V, Ln, C, device=device, n_kl_chunks=2) for _ in inputs]
    calls = [lambda s=s, a=a: s.step(*a) for s, a in zip(steps, inputs)]
    alone, results = _run_pair(device, [_LMOut(s) for s in steps], calls)
    assert not torch.equal(alone[0]["losses"], alone[1]["losses"])
    _assert_same(alone, results)


def test_moe_and_lm_steps_on_two_threads(device):
    """The two step kinds share the device's helper stream: an MoE call and an LM call
    from two threads at once."""
    from param_decomp_amd.lm_step import KINDS as K, LMStackStep, LMWeights, site_dims
    from param_decomp_amd.moe_step import MoEStackStep, MoEWeights

    g = torch.Generator(device=device).manual_seed(11)

    def rn(*shape, scale):
        return (torch.randn(*shape, device=device, generator=g) * scale).to(torch.bfloat16)

    T, d, f, E, k, c, Ln = 512, 64, 32, 8, 2, 32, 2
    w = MoEWeights(ln=torch.zeros(Ln, d, device=device), router=rn(Ln, E, d, scale=d**-0.5),
                   Wg=rn(Ln, E, d, f, scale=d**-0.5), Wu=rn(Ln, E, d, f, scale=d**-0.5),
                   Wd=rn(Ln, E, f, d, scale=f**-0.5), Vg=rn(Ln, E, d, c, scale=d**-0.5),
                   Ug=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vu=rn(Ln, E, d, c, scale=d**-0.5),
                   Uu=rn(Ln, E, c, f, scale=(E * c)**-0.5), Vd=rn(Ln, E, f, c, scale=f**-0.5),
                   Ud=rn(Ln, E, c, d, scale=(E * c)**-0.5))
    moe_in = (rn(T, d, scale=1.0), w,
              (torch.rand(Ln, 3, T, k, c, device=device, generator=g) * 1.6 - 0.3).to(torch.bfloat16), (1, 2))
    moe = MoEStackStep(T, d, f, E, k, c, Ln, device=device)

    B, Tl, dl, H, fl, V, Ll = 1, 256, 128, 2, 256, 512, 2
    C = {kk: 32 for kk in K}
    Wd, Vd, Ud = {}, {}, {}
    for kk in K:
        din, dout = site_dims(kk, dl, H, H, fl)
        Wd[kk], Vd[kk], Ud[kk] = rn(Ll, dout, din, scale=din**-0.5), rn(Ll, din, C[kk], scale=din**-0.5), rn(
            Ll, C[kk], dout, scale=C[kk]**-0.5)
    lw = LMWeights(wte=rn(V, dl, scale=dl**-0.5), ln1=torch.ones(Ll, dl, device=device),
                   ln2=torch.ones(Ll, dl, device=device), norm=torch.ones(dl, device=device), W=Wd, V=Vd, U=Ud)
    lm_in = (torch.randint(0, V, (B * Tl,), device=device, generator=g, dtype=torch.int32), lw,
             {kk: (torch.rand(Ll, B * Tl, C[kk], device=device, generator=g) * 1.6 - 0.3).to(torch.bfloat16)
              for kk in K}, (3, 4))
    lm = LMStackStep(B, Tl, dl, H, H, fl, V, Ll, C, device=device, n_kl_chunks=1)
    alone, results = _run_pair(device, [_MoEOut(moe), _LMOut(lm)], [lambda: moe.step(*moe_in), lambda: lm.step(*lm_in)])
    _assert_same(alone, results)
