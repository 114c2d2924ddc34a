"""GPU parity at the widths the measured workloads run, so every kernel instantiation
those workloads select is compared against the oracle, not only checked for finiteness:

- the MoE stack at its full widths (d=512, f=256, c=512, 42 experts, top-8): the
  256x256 grouped tiles of the N=512 component products (`grouped_gemm_pair`) and of
  every paired weight gradient (`grouped_gemm_dw_kmajor_pair`), K=512 main loops over
  several k stages, and ragged per-expert contraction lengths;
- the dense products' 256x256 buffer-fed tile (`CfgDtlBig`, taken once the grid has >= 256
  such tiles) in every operand layout, and the 128x128 one just below that size;
- the public grouped products at K = N = 512 with ragged and empty groups;
- the LM stack at the Llama-4L widths (the streamed KL's dual products at V = 50277) and
  the dense step at 768 -> 3072, C = 4096.

Reference semantics: `pd/targets/qwen36_moe.py:2752-2837` (decomposed experts in job
space), `pd/routed/experts.py:209-348` (grouped products and the ragged dW),
`pd/targets/transformer.py:1031-1140` and `pd/targets/losses.py:102-163` (the LM step),
`pd/core/decomposed_linear.py:142-175` (the dense site).
"""

import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from oracle import pd_oracle as po
from routing_checks import assert_routing_matches

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _bf(a, device):
    return torch.tensor(np.asarray(a, np.float32), device=device).to(torch.bfloat16)


def _close(got, want, rtol, floor, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got - want)
    bad = err > rtol * np.abs(want) + floor * scale
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} off, worst {err.max():.3e} scale {scale:.3e}"


def test_moe_stack_step_full_width_matches_oracle(device):
    """T=1024 tokens through 2 layers at the benchmark's widths, with the frozen delta
    channel: routing bit-exact up to bf16 near-ties of the router products, losses and
    every gradient within rtol 2e-2 of the oracle's bf16-storage model on the same
    routing. About 20 s of oracle time."""
    from param_decomp_amd import _lib as L
    from param_decomp_amd.moe_step import MoEStackStep, MoEWeights

    cfg = mo.MoEConfig(T=1024, d=512, f=256, E=42, k=8, c=512, L=2)
    rng = np.random.default_rng(21)
    params, x0, ci = mo.init_moe(cfg, rng)
    rb = po.round_bf16
    params = [{k: (v.astype(np.float32).astype(np.float64) if k == "ln" else rb(v)) for k, v in P.items()}
              for P in params]
    x0 = rb(x0)
    ci = [{s: rb(v) for s, v in layer.items()} for layer in ci]

    def stack(name, dt=torch.bfloat16):
        return torch.tensor(np.stack([P[name] for P in params]).astype(np.float32), device=device).to(dt)

    w = MoEWeights(ln=stack("ln", torch.float32), router=stack("router"), Wg=stack("Wg"), Wu=stack("Wu"),
                   Wd=stack("Wd"), Vg=stack("Vg"), Ug=stack("Ug"), Vu=stack("Vu"), Uu=stack("Uu"), Vd=stack("Vd"),
                   Ud=stack("Ud"))
    ci_t = _bf(np.stack([np.stack([layer[s] for s in mo.SITES]) for layer in ci]), device)
    x0_t = _bf(x0, device)
    key = (3, 29)
    step = MoEStackStep(cfg.T, cfg.d, cfg.f, cfg.E, cfg.k, cfg.c, cfg.L, device=device, p=2.0, imp_coeff=0.5,
                        recon_coeff=1.5, layout=L.LAYOUT_PARTITIONABLE, use_delta=True)
    step.step(x0_t, w, ci_t, key)
    torch.cuda.synchronize()
    got_idx = step.top_idx.cpu().numpy()
    ref = mo.moe_stack_step(cfg, params, x0, ci, key, p=2.0, imp_coeff=0.5, recon_coeff=1.5, bf16_storage=True,
                            partitionable=True, use_delta=True, pinned_top_idx=got_idx)
    for l in range(cfg.L):
        assert_routing_matches(got_idx[l], ref, l, cfg.k)
        sizes = np.bincount(got_idx[l].ravel(), minlength=cfg.E)
        assert sizes.min() > 64  # every expert's rows span several 64-deep k stages of the dW
    np.testing.assert_allclose(step.losses.cpu().numpy(), [ref["loss"], ref["recon"], ref["imp"], 0.0], rtol=2e-2)
    for l in range(cfg.L):
        for s, vn, un in (("gate", "Vg", "Ug"), ("up", "Vu", "Uu"), ("down", "Vd", "Ud")):
            _close(step.dV[s][l].cpu().numpy(), ref["grads"][l][vn], BF16_RTOL, 1e-2, f"{vn}[{l}]")
            _close(step.dU[s][l].cpu().numpy(), ref["grads"][l][un], BF16_RTOL, 1e-2, f"{un}[{l}]")
        got = step.d_ci_pre[l].float().cpu().numpy()
        for si, s in enumerate(mo.SITES):
            _close(got[si], ref["d_ci_pre"][l][s], BF16_RTOL, 1e-2, f"d_ci_pre[{l}][{s}]")


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 768), (4096, 4096, 776), (4000, 4104, 200)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_big_tile_layouts(device, ta, tb, M, N, K):
    """The dense site's shapes in every operand layout: 192 256x256 tiles stay on the
    128x128 buffer-fed kernel; >= 256 (one per CU) select the 256x256 one, here with a
    k-tail stage and ragged M and N edges. fp32 output within fp32 accumulation-order
    error of a float64 product; bf16 output within bf16 rounding."""
    from param_decomp_amd import ops

    assert -(-M // 256) * -(-N // 256) >= 192
    rng = np.random.default_rng(M + N + K + 2 * ta + tb)
    A = _bf(rng.normal(size=(K, M) if ta else (M, K)), device)
    B = _bf(rng.normal(size=(N, K) if tb else (K, N)), device)
    An, Bn = _np(A), _np(B)
    want = (An.T if ta else An) @ (Bn.T if tb else Bn)
    out = ops.gemm(A, B, trans_a=bool(ta), trans_b=bool(tb), out_dtype=torch.float32)
    _close(_np(out), want, 1e-5, 1e-6, f"gemm fp32 out ta={ta} tb={tb}")
    out16 = ops.gemm(A, B, trans_a=bool(ta), trans_b=bool(tb))
    _close(_np(out16), want, BF16_RTOL, 1e-3, f"gemm bf16 out ta={ta} tb={tb}")


def test_grouped_products_at_k_n_512(device):
    """Forward (both rhs layouts), d_input and both dW forms at K = N = 512 over 42
    groups with ragged sizes, three empty groups and trailing rows past the last offset."""
    from param_decomp_amd import ops
    from param_decomp_amd.routed.experts import grouped_matmul, transposed_grouped_matmul

    rng = np.random.default_rng(5)
    E, K, N = 42, 512, 512
    sizes = rng.integers(1, 400, size=E)
    sizes[[3, 17, 41]] = 0
    used = int(sizes.sum())
    J = (used + 13 + 7) // 8 * 8
    offsets = torch.tensor(np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32), device=device)
    lhs = _bf(rng.normal(size=(J, K)), device).requires_grad_(True)
    rhs = _bf(rng.normal(size=(E, K, N)) / 16, device).requires_grad_(True)
    out = grouped_matmul(lhs, rhs, offsets)
    want = po.grouped_matmul(_np(lhs)[:used], _np(rhs), sizes)
    _close(_np(out)[:used], want, BF16_RTOL, 4e-3, "grouped fwd")
    assert torch.count_nonzero(out[used:]) == 0
    outT = ops.grouped_gemm(lhs.detach(), rhs.detach().transpose(1, 2).contiguous(), offsets, trans_rhs=True)
    _close(_np(outT)[:used], want, BF16_RTOL, 4e-3, "grouped fwd, K-contiguous rhs")
    g = _bf(rng.normal(size=(J, N)), device)
    dl, dr = torch.autograd.grad(out, (lhs, rhs), g)
    gn = _np(g)
    gn[used:] = 0.0
    _close(_np(dl)[:used], po.grouped_matmul(gn[:used], np.transpose(_np(rhs), (0, 2, 1)), sizes), BF16_RTOL, 4e-3,
           "grouped d_lhs")
    want_dw = po.transposed_grouped_matmul(_np(lhs)[:used], gn[:used], sizes)
    _close(_np(dr), want_dw, BF16_RTOL, 4e-3, "grouped d_rhs")
    dw = transposed_grouped_matmul(lhs.detach(), g, offsets, out_dtype=torch.float32)
    _close(_np(dw), want_dw, 1e-5, 1e-6, "dw fp32")
    dwk = ops.grouped_gemm_dw_kmajor(lhs.detach().t().contiguous(), g.t().contiguous(), offsets, E,
                                     out_dtype=torch.float32)
    _close(_np(dwk), want_dw, 1e-5, 1e-6, "dw kmajor fp32")
    for e in (3, 17, 41):
        assert torch.count_nonzero(dw[e]) == 0 and torch.count_nonzero(dwk[e]) == 0


def test_lm_stack_step_at_benchmark_widths_matches_oracle(device):
    """The Llama-4L widths (d_model 768, 12 heads, d_mlp 3072, vocab 50277, C = 1024
    attention / 4096 MLP, KL over 3 vocab chunks) on one 512-token sequence through 2
    layers: the KL dual products at V = 50277 and d = 768, the tied head's input
    gradient, and every site product at the benchmark's widths against the LM oracle's
    bf16 storage model (elementwise 2e-2 plus a 2e-2 floor of each tensor's largest
    magnitude, and 2e-2 in relative norm; test_gpu_lm.py states why). About 20 s of
    oracle time."""
    from test_gpu_lm import _close as lm_close
    from test_gpu_lm import _setup

    from oracle import lm_oracle as lo
    from param_decomp_amd.lm_step import KINDS, LMStackStep

    B, T = 1, 512
    cfg = lo.LMConfig(n_layers=2, d=768, n_head=12, n_kv_head=12, d_mlp=3072, vocab=50277,
                      C={"q_proj": 1024, "k_proj": 1024, "v_proj": 1024, "o_proj": 1024, "c_fc": 4096,
                         "down_proj": 4096})
    params, tokens, ci, w, ci_t, tok_t = _setup(cfg, B, T, 31, device)
    key = (9, 41)
    spec = po.ImpMin("pnorm", p=2.0, coeff=1e-3)
    step = LMStackStep(B, T, cfg.d, cfg.n_head, cfg.n_kv_head, cfg.d_mlp, cfg.vocab, cfg.n_layers, cfg.C,
                       device=device, n_kl_chunks=3, recon_coeff=3.0, p=2.0, imp_coeff=1e-3)
    step.step(tok_t, w, ci_t, key)
    torch.cuda.synchronize()
    ref = lo.lm_stack_step(cfg, params, tokens, ci, key, bf16_storage=True, recon_coeff=3.0, imp_min=spec)
    np.testing.assert_allclose(step.losses.cpu().numpy(), [ref["loss"], ref["recon"], ref["imp"], ref["freq"]],
                               rtol=2e-2, atol=1e-7)
    stats = []
    for l in range(cfg.n_layers):
        for k in KINDS:
            lm_close(_np(step.dV[k][l]), ref["dV"][l][k], f"dV[{l}][{k}]", stats)
            lm_close(_np(step.dU[k][l]), ref["dU"][l][k], f"dU[{l}][{k}]", stats)
            lm_close(_np(step.d_ci_pre[k][l]), ref["d_ci_pre"][l][k], f"d_ci_pre[{l}][{k}]", stats)
    worst = max(stats, key=lambda x: x[1])
    print(f"worst element/scale {worst[1]:.3e} ({worst[0]}), worst relative norm {max(x[2] for x in stats):.3e}")


@pytest.mark.parametrize("sl0", [False, True])
def test_dense_step_at_benchmark_widths_matches_oracle(device, sl0):
    """The single-linear widths (768 -> 3072, C = 4096, bf16, the delta channel on) on
    512 tokens: the 256x256 GEMM tiles the step selects at these widths, the tabulated
    gate forward over 4096 components and the gate backward, against the oracle's bf16
    storage model at rtol 2e-2 with a 1e-2 floor of each tensor's largest magnitude."""
    from oracle import threefry as tf
    from param_decomp_amd.dense_step import DenseSiteStep
    from param_decomp_amd.losses import ImpMin

    rng = np.random.default_rng(7)
    T, d_in, d_out, C = 512, 768, 3072, 4096
    x = rng.normal(size=(T, d_in))
    W = rng.normal(size=(d_out, d_in)) / np.sqrt(d_in)
    V = rng.normal(size=(d_in, C)) / np.sqrt(d_in)
    U = rng.normal(size=(C, d_out)) / np.sqrt(C)
    gp = po.GateParams(rng.normal(size=(C, 16)) * 1.4, np.zeros((C, 16)), rng.normal(size=(C, 16)) * 0.35,
                       np.full(C, 0.3))
    tx, tW, tV, tU = (_bf(a, device) for a in (x, W, V, U))
    gate = tuple(torch.tensor(np.asarray(a, np.float32), device=device) for a in (gp.w_in, gp.b_in, gp.w_out,
                                                                                   gp.b_out))
    spec = (po.ImpMin("smooth_l0", coeff=0.7, gamma=0.2, normalize_at_one=True, freq_coeff=0.4, ref_count=4096.0)
            if sl0 else po.ImpMin("pnorm", p=2.0, coeff=0.7))
    imp = ImpMin(spec.kind, spec.p, spec.coeff, spec.gamma, spec.normalize_at_one, spec.freq_coeff, spec.ref_count)
    step = DenseSiteStep(T, d_in, d_out, C, device=device, recon_coeff=1.3, use_delta=True, imp_min=imp)
    draw_key = tf.fold_in(tf.prng_key(11), 2)
    mk, dk = step.site_keys(draw_key, 0)
    g = step.step(tx, tW, tV, tU, gate, mk, dk)
    torch.cuda.synchronize()
    gp64 = po.GateParams(*(_np(t) for t in gate))
    r = po.dense_site_step(_np(tx), _np(tW), _np(tV), _np(tU), gp64, draw_key, recon_coeff=1.3,
                           mask_dtype="bfloat16", use_delta=True, bf16_storage=True, imp_min=spec)
    np.testing.assert_allclose(g.losses.cpu().numpy(), [r.loss, r.recon, r.imp, r.freq], rtol=BF16_RTOL, atol=1e-7)
    _close(_np(g.dU), r.dU, BF16_RTOL, 1e-2, "dU")
    _close(_np(g.dV), r.dV, BF16_RTOL, 1e-2, "dV")
    for got, want, name in zip((g.dw_in, g.db_in, g.dw_out, g.db_out), r.dgate, ("dw_in", "db_in", "dw_out", "db_out")):
        _close(_np(got), want, BF16_RTOL, 1e-2, name)
