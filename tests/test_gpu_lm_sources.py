"""GPU parity of the LM step with persistent source tables (`pd_lm_stack_step_sources`)
against the LM oracle's source arm (oracle/lm_oracle.py, pinned by the draw path and by
finite differences): losses, the model gradients and the tables' gradients within the LM
step's bf16 tolerance, for every table storage, the three row shapes (one token per row,
one sample per row, one row for the batch) and with and without the delta table; the
warmup form (no weight gradients) and the reused clean pass give the same results bit for
bit."""

import numpy as np
import pytest
import torch

from oracle import lm_oracle as lo
from tests.test_gpu_lm import KINDS, _close, _setup

pytestmark = pytest.mark.gpu


def _tables(cfg, N, rps, dtype, with_delta, seed, device):
    rng = np.random.default_rng(seed)
    S = N // rps
    src_f, src_t = [{} for _ in range(cfg.n_layers)], {}
    for k in KINDS:
        u = rng.uniform(0.0, 1.0, size=(cfg.n_layers, S, cfg.C[k]))
        if dtype == torch.uint16:
            q = np.round(u * 65535).astype(np.int32)
            src_t[k] = torch.tensor(q, device=device).to(torch.uint16)
            val = q / 65535.0
        else:
            src_t[k] = torch.tensor(u, dtype=torch.float32, device=device).to(dtype)
            val = src_t[k].float().cpu().numpy().astype(np.float64)
        for l in range(cfg.n_layers):
            src_f[l][k] = val[l]
    dl_f, dl_t = None, None
    if with_delta:
        d = rng.uniform(0.0, 1.0, size=(cfg.n_layers, len(KINDS), S))
        dl_t = torch.tensor(d, dtype=torch.float32, device=device)
        dl_f = [{k: d[l, i] for i, k in enumerate(KINDS)} for l in range(cfg.n_layers)]
    return src_f, src_t, dl_f, dl_t


@pytest.mark.parametrize("dtype,rps_kind,with_delta", [(torch.float32, "bsc", True), (torch.bfloat16, "bc", True),
                                                       (torch.uint16, "c", True), (torch.float32, "bc", False)])
def test_lm_sources_step_matches_oracle(device, dtype, rps_kind, with_delta):
    from param_decomp_amd.lm_step import LMStackStep
    from oracle import pd_oracle as po
    from param_decomp_amd.losses import ImpMin

    B, T = 2, 128
    N = B * T
    rps = {"bsc": 1, "bc": T, "c": N}[rps_kind]
    cfg = lo.LMConfig(n_layers=2, d=128, n_head=2, n_kv_head=1, d_mlp=256, vocab=384,
                      C={"q_proj": 64, "k_proj": 48, "v_proj": 64, "o_proj": 32, "c_fc": 128, "down_proj": 96})
    params, tokens, ci, w, ci_t, tok_t = _setup(cfg, B, T, 17, device)
    src_f, src_t, dl_f, dl_t = _tables(cfg, N, rps, dtype, with_delta, 3, device)
    spec = po.ImpMin("pnorm", p=2.0, coeff=0.05)
    step = LMStackStep(B, T, cfg.d, cfg.n_head, cfg.n_kv_head, cfg.d_mlp, cfg.vocab, cfg.n_layers, cfg.C,
                       device=device, use_delta=with_delta, n_kl_chunks=3, recon_coeff=3.0,
                       imp_min=ImpMin("pnorm", 2.0, 0.05), rows_per_source=rps)
    print(f"lm sources {dtype} rps={rps} delta={with_delta}", flush=True)
    step.step_sources(tok_t, w, ci_t, src_t, dl_t)
    torch.cuda.synchronize()
    ref = lo.lm_stack_step(cfg, params, tokens, ci, (0, 0), bf16_storage=True, recon_coeff=3.0, imp_min=spec,
                           sources=(src_f, dl_f, rps))
    np.testing.assert_allclose(step.losses.cpu().numpy(), [ref["loss"], ref["recon"], ref["imp"], ref["freq"]],
                               rtol=2e-2, atol=1e-7)
    stats = []
    for l in range(cfg.n_layers):
        for k in KINDS:
            _close(step.dV[k][l].cpu().numpy(), ref["dV"][l][k], f"dV[{l}][{k}]", stats)
            _close(step.dU[k][l].cpu().numpy(), ref["dU"][l][k], f"dU[{l}][{k}]", stats)
            _close(step.d_ci_pre[k][l].float().cpu().numpy(), ref["d_ci_pre"][l][k], f"d_ci_pre[{l}][{k}]", stats)
            _close(step.d_src[k][l].cpu().numpy(), ref["d_src"][l][k], f"d_src[{l}][{k}]", stats)
            if with_delta:
                _close(step.d_src_delta[l, KINDS.index(k)].cpu().numpy(), ref["d_src_delta"][l][k],
                       f"d_src_delta[{l}][{k}]", stats)
    worst = max(stats, key=lambda x: x[1])
    print(f"worst element/scale {worst[1]:.3e} ({worst[0]}), worst relative norm {max(x[2] for x in stats):.3e}")
    # the warmup form: the same source gradients without the model gradients, then the
    # clean pass taken from the workspace: identical results
    first = {"losses": step.losses.clone(), "dci": {k: step.d_ci_pre[k].clone() for k in KINDS},
             "dsrc": {k: step.d_src[k].clone() for k in KINDS}, "dsd": step.d_src_delta.clone(),
             "dV": {k: step.dV[k].clone() for k in KINDS}}
    step.step_sources(tok_t, w, ci_t, src_t, dl_t, want_weight_grads=False, reuse_clean=True)
    torch.cuda.synchronize()
    for k in KINDS:
        assert torch.equal(step.d_src[k], first["dsrc"][k]), k
    if with_delta:
        assert torch.equal(step.d_src_delta, first["dsd"])
    step.step_sources(tok_t, w, ci_t, src_t, dl_t, reuse_clean=True)
    torch.cuda.synchronize()
    assert torch.equal(step.losses, first["losses"])
    for k in KINDS:
        assert torch.equal(step.dV[k], first["dV"][k]) and torch.equal(step.d_ci_pre[k], first["dci"][k]), k


def test_lm_persistent_pgd_step(device):
    """Warmup ascents then the final step (Adam on fp32 `bc` tables, with the delta leaf):
    the sources move inside [0, 1], the recon term does not fall over the warmups (ascent),
    and the final gradients equal those of the same procedure spelled out call by call."""
    from param_decomp_amd.adversary import AdamPGDConfig, LMPPGDStep, PersistentAdversary
    from param_decomp_amd.lm_step import LMStackStep
    from param_decomp_amd.losses import ImpMin

    B, T = 2, 64
    cfg = lo.LMConfig(n_layers=2, d=128, n_head=2, n_kv_head=2, d_mlp=256, vocab=384,
                      C={"q_proj": 32, "k_proj": 32, "v_proj": 32, "o_proj": 32, "c_fc": 64, "down_proj": 48})
    params, tokens, ci, w, ci_t, tok_t = _setup(cfg, B, T, 21, device)
    _, src_t, _, dl_t = _tables(cfg, B * T, T, torch.float32, True, 5, device)

    def make():
        advs = {k: PersistentAdversary(src_t[k].clone(), AdamPGDConfig(), n_warmup=2, rows_per_source=T, leaf_index=i)
                for i, k in enumerate(KINDS)}
        dadv = PersistentAdversary(dl_t.clone(), AdamPGDConfig(), n_warmup=2, rows_per_source=T, leaf_index=len(KINDS))
        return advs, dadv

    step = LMStackStep(B, T, cfg.d, cfg.n_head, cfg.n_kv_head, cfg.d_mlp, cfg.vocab, cfg.n_layers, cfg.C,
                       device=device, use_delta=True, n_kl_chunks=2, imp_min=ImpMin("pnorm", 2.0, 0.0),
                       rows_per_source=T)
    advs, dadv = make()
    res = LMPPGDStep(step, advs, dadv).step(tok_t, w, ci_t, lr=0.05, key=(0, 9))
    torch.cuda.synchronize()
    wl = [float(x) for x in res.warmup_losses]
    assert len(wl) == 2 and wl[-1] >= wl[0] * (1 - 1e-3), wl
    for k in KINDS:
        s = advs[k].sources
        assert float(s.min()) >= 0.0 and float(s.max()) <= 1.0 and not torch.equal(s, src_t[k])
    dV = {k: step.dV[k].clone() for k in KINDS}
    dci = {k: step.d_ci_pre[k].clone() for k in KINDS}
    # the same procedure spelled out: source-only calls and ascents, then the final call
    advs2, dadv2 = make()
    from param_decomp_amd import prng

    warm_key = prng.fold_in(prng.fold_in((0, 9), 0x51C), 0)
    for ascent_key in prng.split(warm_key, 2):
        step.step_sources(tok_t, w, ci_t, {k: a.sources for k, a in advs2.items()}, dadv2.sources,
                          want_weight_grads=False)
        for k in KINDS:
            advs2[k].after_one_ascent(step.d_src[k], 0.05, ascent_key)
        dadv2.after_one_ascent(step.d_src_delta, 0.05, ascent_key)
    step.step_sources(tok_t, w, ci_t, {k: a.sources for k, a in advs2.items()}, dadv2.sources)
    torch.cuda.synchronize()
    for k in KINDS:
        assert torch.equal(step.dV[k], dV[k]) and torch.equal(step.d_ci_pre[k], dci[k]), k
