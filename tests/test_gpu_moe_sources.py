"""Persistent (adversarial) source tables in the MoE stack step against the MoE oracle
(pinned by torch autograd with the tables as leaves, tests/test_moe_oracle.py): the
`c`, `bc` and `bsc` source shapes, f32 / bf16 / uint16 storage, with and without the
delta leaf; losses, every model gradient and both source gradients within rtol 2e-2 of
the oracle's bf16 storage model, and the warmup form (no weight gradients) giving the
same source gradients. Then a whole persistent-PGD step (warmups + final ascent)."""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from routing_checks import assert_routing_matches
from test_gpu_moe import _close, _make

pytestmark = pytest.mark.gpu


def _tables(cfg, rps, dtype, with_delta, seed, device):
    rng = np.random.default_rng(seed)
    S = cfg.T // rps
    src = rng.uniform(size=(cfg.L, 3, S, cfg.E, cfg.c))
    srcd = rng.uniform(size=(cfg.L, 3, S))
    if dtype == torch.uint16:
        q = np.round(src * 65535.0)
        src = q / 65535.0
        t_src = torch.tensor(q.astype(np.int32), device=device).to(torch.uint16)
    else:
        t_src = torch.tensor(src.astype(np.float32), device=device).to(dtype)
        src = t_src.float().cpu().numpy().astype(np.float64)
    t_d = torch.tensor(srcd.astype(np.float32), device=device) if with_delta else None
    src_l = [{s: src[l, i] for i, s in enumerate(mo.SITES)} for l in range(cfg.L)]
    srcd_l = [{s: (srcd[l, i] if with_delta else np.zeros(S)) for i, s in enumerate(mo.SITES)} for l in range(cfg.L)]
    return t_src, t_d, src_l, srcd_l


@pytest.mark.parametrize("rps,dtype,with_delta", [(256, torch.float32, True), (64, torch.bfloat16, True),
                                                  (1, torch.float32, True), (32, torch.uint16, True),
                                                  (64, torch.float32, False)])
def test_moe_step_with_source_tables_matches_oracle(device, rps, dtype, with_delta):
    from param_decomp_amd.moe_step import MoEStackStep

    cfg = mo.MoEConfig(T=256, d=64, f=32, E=8, k=2, c=16, L=2)
    params, x0, ci, w, ci_t, x0_t = _make(cfg, 0, device)
    t_src, t_d, src_l, srcd_l = _tables(cfg, rps, dtype, with_delta, 7 + rps, device)
    step = MoEStackStep(cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L, device=device, p=2.0, imp_coeff=0.0,
                        recon_coeff=1.5, rows_per_source=rps)
    step.step_sources(x0_t, w, ci_t, t_src, t_d)
    torch.cuda.synchronize()
    got_idx = step.top_idx.cpu().numpy()
    ref = mo.moe_stack_step(cfg, params, x0, ci, (0, 17), p=2.0, imp_coeff=0.0, recon_coeff=1.5, bf16_storage=True,
                            use_delta=with_delta, pinned_top_idx=got_idx, sources=(src_l, srcd_l, rps))
    for l in range(cfg.L):
        assert_routing_matches(got_idx[l], ref, l, cfg.k)
    np.testing.assert_allclose(step.losses.cpu().numpy()[:2], [ref["loss"], ref["recon"]], rtol=2e-2)
    d_src = step.d_src.cpu().numpy()
    d_srcd = step.d_src_delta.cpu().numpy()
    for l in range(cfg.L):
        for s, vn, un in (("gate", "Vg", "Ug"), ("up", "Vu", "Uu"), ("down", "Vd", "Ud")):
            _close(step.dV[s][l].cpu().numpy(), ref["grads"][l][vn], 2e-2, 1e-2, f"{vn}[{l}]")
            _close(step.dU[s][l].cpu().numpy(), ref["grads"][l][un], 2e-2, 1e-2, f"{un}[{l}]")
        for si, s in enumerate(mo.SITES):
            _close(d_src[l, si], ref["d_src"][l][s], 2e-2, 1e-2, f"d_src[{l}][{s}]")
            if with_delta:
                _close(d_srcd[l, si], ref["d_src_delta"][l][s], 2e-2, 1e-2, f"d_src_delta[{l}][{s}]")
    # the warmup form: no weight gradients, the same source gradients bit for bit
    first = {k: v.clone() for k, v in (("losses", step.losses), ("dVd", step.dV["down"]), ("dUg", step.dU["gate"]),
                                        ("dci", step.d_ci_pre))}
    step.step_sources(x0_t, w, ci_t, t_src, t_d, want_weight_grads=False)
    torch.cuda.synchronize()
    assert np.array_equal(step.d_src.cpu().numpy(), d_src)
    if with_delta:
        assert np.array_equal(step.d_src_delta.cpu().numpy(), d_srcd)
    # the clean pass taken from the workspace (same x0 and frozen weights): identical
    step.step_sources(x0_t, w, ci_t, t_src, t_d, reuse_clean=True)
    torch.cuda.synchronize()
    assert torch.equal(step.losses, first["losses"]) and torch.equal(step.d_ci_pre, first["dci"])
    assert torch.equal(step.dV["down"], first["dVd"]) and torch.equal(step.dU["gate"], first["dUg"])
    assert np.array_equal(step.d_src.cpu().numpy(), d_src)
    assert np.array_equal(step.top_idx.cpu().numpy(), got_idx)


def test_moe_persistent_pgd_step(device):
    """Warmup ascents then the final step: after each ascent the sources moved along
    their gradient inside [0, 1], the final model gradients are those of a direct call
    at the ascended sources, and the recon loss did not decrease over the warmups
    (ascent on the adversary's objective)."""
    from param_decomp_amd.adversary import AdamPGDConfig, MoEPPGDStep, PersistentAdversary
    from param_decomp_amd.moe_step import MoEStackStep

    cfg = mo.MoEConfig(T=256, d=64, f=32, E=8, k=2, c=16, L=2)
    params, x0, ci, w, ci_t, x0_t = _make(cfg, 1, device)
    rps = 64
    t_src, t_d, _, _ = _tables(cfg, rps, torch.float32, True, 3, device)
    step = MoEStackStep(cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L, device=device, p=2.0, imp_coeff=0.0,
                        recon_coeff=1.0, rows_per_source=rps)
    adv = PersistentAdversary(t_src.clone(), AdamPGDConfig(), n_warmup=3, rows_per_source=rps)
    dadv = PersistentAdversary(t_d.clone(), AdamPGDConfig(), n_warmup=3, rows_per_source=rps, leaf_index=1)
    res = MoEPPGDStep(step, adv, dadv).step(x0_t, w, ci_t, lr=0.05, key=(0, 9))
    torch.cuda.synchronize()
    wl = [float(x) for x in res.warmup_losses]
    assert len(wl) == 3 and wl[-1] >= wl[0] * (1 - 1e-3), wl
    assert float(adv.sources.min()) >= 0.0 and float(adv.sources.max()) <= 1.0
    assert not torch.equal(adv.sources, t_src)
    dV, dci = step.dV["down"].clone(), step.d_ci_pre.clone()
    assert torch.isfinite(dV).all() and float(dV.abs().max()) > 0
    # the same procedure spelled out (fp32 sources: the keys only drive uint16 rounding):
    # three source-only steps and ascents, then the final step at the warmed sources
    adv2 = PersistentAdversary(t_src.clone(), AdamPGDConfig(), n_warmup=3, rows_per_source=rps)
    dadv2 = PersistentAdversary(t_d.clone(), AdamPGDConfig(), n_warmup=3, rows_per_source=rps, leaf_index=1)
    for _ in range(3):
        step.step_sources(x0_t, w, ci_t, adv2.sources, dadv2.sources, want_weight_grads=False)
        adv2.after_one_ascent(step.d_src, 0.05, (0, 0))
        dadv2.after_one_ascent(step.d_src_delta, 0.05, (0, 0))
    step.step_sources(x0_t, w, ci_t, adv2.sources, dadv2.sources)
    torch.cuda.synchronize()
    assert torch.equal(step.dV["down"], dV) and torch.equal(step.d_ci_pre, dci)
