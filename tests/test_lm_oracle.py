"""Pins of the LM oracle (oracle/lm_oracle.py) against the reference's own frozen
goldens, library routines and finite differences (CPU)."""

import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import lm_oracle as lo

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _t(a):
    return torch.tensor(np.asarray(a, np.float64), dtype=torch.float64)


def test_tiny_llama_simple_mlp_logits_match_the_reference_fixture():
    """The reference's frozen fp32 logits of a 3-layer LlamaSimpleMLP (GQA repeat 2,
    rotate-half RoPE, GELU-tanh MLP, tied head), held to the reference test's own bound
    (`pd/tests/targets/simple_mlp_equivalence/test_torch_equivalence.py`: max abs 1e-5)."""
    f = np.load(os.path.join(GOLDEN, "simple_mlp_tiny_fixture.npz"))
    c = json.loads(str(f["config_json"]))
    cfg = lo.LMConfig(n_layers=c["n_layer"], d=c["n_embd"], n_head=c["n_head"], n_kv_head=c["n_key_value_heads"],
                      d_mlp=c["n_intermediate"], vocab=c["vocab_size"], mlp="plain", eps=c["rms_norm_eps"],
                      rope_base=c["rotary_base"])
    assert c["rotary_dim"] == cfg.head_dim and not c["rotary_adjacent_pairs"]
    w = lambda k: _t(f["weights." + k])  # noqa: E731
    params = {"head": w("lm_head.weight"), "norm": w("ln_f.weight"), "layers": []}
    for i in range(cfg.n_layers):
        params["layers"].append({
            "ln1": w(f"h.{i}.rms_1.weight"), "ln2": w(f"h.{i}.rms_2.weight"),
            "W_q_proj": w(f"h.{i}.attn.q_proj.weight"), "W_k_proj": w(f"h.{i}.attn.k_proj.weight"),
            "W_v_proj": w(f"h.{i}.attn.v_proj.weight"), "W_o_proj": w(f"h.{i}.attn.o_proj.weight"),
            "W_c_fc": w(f"h.{i}.mlp.c_fc.weight"), "W_down_proj": w(f"h.{i}.mlp.down_proj.weight")})
    idx = torch.as_tensor(f["idx"])
    r0 = w("wte.weight")[idx]
    got = lo.logits(params, lo.forward(cfg, params, r0)).numpy()
    assert got.shape == f["logits"].shape
    assert np.abs(got - f["logits"]).max() < 1e-5


def _equivalence_model():
    f = np.load(os.path.join(GOLDEN, "equivalence_fixtures.npz"))
    s = lambda k: f["_scalar_" + k].item()  # noqa: E731
    d, di, n_dec, n_tail, C = s("N_EMBD"), s("N_INTERMEDIATE"), s("N_DECOMP_LAYERS"), s("N_TAIL"), s("C")
    kinds = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}
    cfg = lo.LMConfig(n_layers=n_dec + n_tail, d=d, n_head=2, n_kv_head=1, d_mlp=di, vocab=f["lm_head"].shape[0],
                      C={k: C for k in kinds.values()}, mlp="glu", eps=s("EPS"))
    z = lambda r, c: torch.zeros(r, c, dtype=torch.float64)  # noqa: E731 (the fixtures zero every attention projection)
    hd = d // 2
    layers = []
    for i in range(n_dec + n_tail):
        pre = "" if i < n_dec else "tail_"
        j = i if i < n_dec else i - n_dec
        P = {"ln1": _t(f[f"{pre}ln1_{j}"]), "ln2": _t(f[f"{pre}ln2_{j}"]), "W_q_proj": z(2 * hd, d),
             "W_k_proj": z(hd, d), "W_v_proj": z(hd, d), "W_o_proj": z(d, 2 * hd),
             "W_gate_proj": _t(f[f"{pre}Wg_{j}"]), "W_up_proj": _t(f[f"{pre}Wu_{j}"]),
             "W_down_proj": _t(f[f"{pre}Wd_{j}"])}
        if i < n_dec:
            for short, kind in kinds.items():
                P["V_" + kind] = _t(f[f"V{short[0]}_{i}"])
                P["U_" + kind] = _t(f[f"U{short[0]}_{i}"])
        layers.append(P)
    params = {"head": _t(f["lm_head"]), "norm": _t(f["norm"]), "layers": layers}
    return f, cfg, params, kinds, n_dec


def test_ppgd_loss_matches_the_reference_golden():
    """`pd/tests/targets/equivalence/jax_equivalence.py:160-196`: masks composed from the
    lower CI and the fixed PPGD sources, `m = ci + (1 - ci) * s[..., :C]`, weight-delta
    mask `s[..., C]` (broadcast over the batch), every decomposed GLU site masked, then
    final norm, head and the per-position KL against the frozen forward. The golden is
    the reference's torch-era value, compared at the reference test's RTOL 2e-4 / ATOL
    1e-5."""
    f, cfg, params, kinds, n_dec = _equivalence_model()
    ref = json.load(open(os.path.join(GOLDEN, "equivalence_torch_reference.json")))
    r0 = _t(f["resid"])
    b, t, _ = r0.shape
    masks, deltas = [], []
    for i in range(cfg.n_layers):
        masks.append({})
        deltas.append({})
        if i >= n_dec:
            continue
        for short, kind in kinds.items():
            ci = _t(f[f"ci_lower_{short}"][:, :, i])
            src = _t(np.broadcast_to(f[f"ppgd_source_{short}"][:, :, i], (b, t, cfg.C[kind] + 1)))
            masks[i][kind] = ci + (1.0 - ci) * src[..., :-1]
            deltas[i][kind] = src[..., -1]
    clean = lo.logits(params, lo.forward(cfg, params, r0))
    masked = lo.logits(params, lo.forward(cfg, params, r0, masks, deltas))
    ppgd = float(lo.kl_per_position(masked, clean))
    assert abs(ppgd - ref["ppgd"]) <= 1e-5 + 2e-4 * abs(ref["ppgd"]), (ppgd, ref["ppgd"])
    # a dropped delta channel or an unbroadcast source would move it far outside the bound
    no_delta = float(lo.kl_per_position(lo.logits(params, lo.forward(
        cfg, params, r0, masks, [{k: None for k in m} for m in masks])), clean))
    assert abs(no_delta - ref["ppgd"]) > 1e-2 * ref["ppgd"]


def test_attention_matches_torch_sdpa_with_gqa():
    """The oracle's causal GQA attention equals torch's scaled_dot_product_attention on
    the same RoPE-rotated heads."""
    rng = np.random.default_rng(0)
    b, t, H, KV, hd = 2, 9, 4, 2, 8
    q, k, v = (_t(rng.normal(size=(b, t, n * hd))) for n in (H, KV, KV))
    got = lo.causal_attention(q, k, v, H, KV, 10000.0)
    cos, sin = lo.rope_cos_sin(t, hd, 10000.0)
    qh = lo.apply_rope(q.reshape(b, t, H, hd).transpose(1, 2), cos, sin)
    kh = lo.apply_rope(k.reshape(b, t, KV, hd).transpose(1, 2), cos, sin).repeat_interleave(H // KV, 1)
    vh = v.reshape(b, t, KV, hd).transpose(1, 2).repeat_interleave(H // KV, 1)
    want = torch.nn.functional.scaled_dot_product_attention(qh, kh, vh, is_causal=True)
    np.testing.assert_allclose(got.numpy(), want.transpose(1, 2).reshape(b, t, H * hd).numpy(), rtol=1e-12,
                               atol=1e-12)


def test_rope_is_a_rotation_with_relative_position_scores():
    # head_dim 2: inv_freq = [1], so position p rotates (x0, x1) by p radians
    cos, sin = lo.rope_cos_sin(3, 2, 10000.0)
    x = _t([[[[1.0, 0.0], [1.0, 0.0], [0.0, 1.0]]]])
    y = lo.apply_rope(x, cos, sin)[0, 0].numpy()
    np.testing.assert_allclose(y[1], [math.cos(1.0), math.sin(1.0)], atol=1e-15)
    np.testing.assert_allclose(y[2], [-math.sin(2.0), math.cos(2.0)], atol=1e-15)
    # scores depend only on the offset between query and key positions
    rng = np.random.default_rng(1)
    hd, T = 16, 12
    q, k = _t(rng.normal(size=(1, 1, 1, hd))), _t(rng.normal(size=(1, 1, 1, hd)))
    cos, sin = lo.rope_cos_sin(T, hd, 10000.0)
    qs = lo.apply_rope(q.expand(1, 1, T, hd), cos, sin)[0, 0]
    ks = lo.apply_rope(k.expand(1, 1, T, hd), cos, sin)[0, 0]
    s = (qs @ ks.T).numpy()
    for off in range(-3, 4):
        diag = np.diagonal(s, offset=off)
        np.testing.assert_allclose(diag, diag[0], rtol=1e-10)


def _small():
    cfg = lo.LMConfig(n_layers=2, d=16, n_head=4, n_kv_head=4, d_mlp=24, vocab=40,
                      C={"q_proj": 6, "k_proj": 5, "v_proj": 6, "o_proj": 4, "c_fc": 8, "down_proj": 7})
    rng = np.random.default_rng(3)
    params = lo.init_lm(cfg, rng)
    tokens = rng.integers(0, cfg.vocab, size=(2, 5))
    ci = lo.init_ci(cfg, 10, rng, 0.05, 0.95)
    return cfg, params, tokens, ci


def test_step_gradients_match_finite_differences():
    """float64 step: dV, dU and the CI-preactivation gradients against central
    differences of the loss (CI kept inside (0, 1), where the custom lower VJP is the
    derivative), with the stochastic masks and the weight-delta channel on."""
    cfg, params, tokens, ci = _small()
    key = (7, 11)
    kw = dict(p=2.0, imp_coeff=0.3, recon_coeff=1.7)
    base = lo.lm_stack_step(cfg, params, tokens, ci, key, **kw)
    rng = np.random.default_rng(5)
    eps = 1e-6
    for l, kind in ((0, "q_proj"), (0, "k_proj"), (1, "o_proj"), (1, "c_fc"), (0, "down_proj")):
        for name, grad in (("V_", base["dV"][l][kind]), ("U_", base["dU"][l][kind])):
            arr = params["layers"][l][name + kind]
            for _ in range(2):
                i = tuple(int(rng.integers(0, s)) for s in arr.shape)
                old = arr[i]
                arr[i] = old + eps
                up = lo.lm_stack_step(cfg, params, tokens, ci, key, **kw)["loss"]
                arr[i] = old - eps
                dn = lo.lm_stack_step(cfg, params, tokens, ci, key, **kw)["loss"]
                arr[i] = old
                assert (up - dn) / (2 * eps) == pytest.approx(grad[i], rel=1e-5, abs=1e-9), (name, kind, l, i)
    for l, kind in ((0, "v_proj"), (1, "down_proj")):
        arr = ci[l][kind]
        for _ in range(3):
            i = tuple(int(rng.integers(0, s)) for s in arr.shape)
            old = arr[i]
            arr[i] = old + eps
            up = lo.lm_stack_step(cfg, params, tokens, ci, key, **kw)["loss"]
            arr[i] = old - eps
            dn = lo.lm_stack_step(cfg, params, tokens, ci, key, **kw)["loss"]
            arr[i] = old
            assert (up - dn) / (2 * eps) == pytest.approx(base["d_ci_pre"][l][kind][i], rel=1e-5, abs=1e-9)


def test_full_masks_reproduce_the_clean_forward():
    """CI = 1 everywhere makes every mask 1: with d = 0 the masked forward must equal
    the clean one exactly when V@U = W^T (here: an exact rank-C factorization), so the
    KL is 0 (the decomposition identity)."""
    cfg = lo.LMConfig(n_layers=1, d=8, n_head=2, n_kv_head=2, d_mlp=8, vocab=11,
                      C={"q_proj": 8, "c_fc": 8})
    rng = np.random.default_rng(9)
    params = lo.init_lm(cfg, rng)
    for kind in cfg.C:
        L_ = params["layers"][0]
        L_["U_" + kind] = np.linalg.solve(L_["V_" + kind], L_["W_" + kind].T)  # V square: V U = W^T
    tokens = rng.integers(0, cfg.vocab, size=(1, 6))
    ci = [{k: np.full((6, cfg.C[k]), 1.0) for k in cfg.C}]
    out = lo.lm_stack_step(cfg, params, tokens, ci, (1, 2), use_delta=False, imp_coeff=0.0)
    assert abs(out["recon"]) < 1e-12


def test_smooth_l0_terms_and_gradient_match_the_reference_formula():
    """The step's smooth-L0 activity and frequency equal the reference formula
    (pd_oracle.importance_minimality_terms, pinned by the reference's closed forms) on
    every site's upper CI, and with recon_coeff = 0 the CI gradient is exactly the
    imp-min pullback (the per-component slope times psi', through the upper VJP)."""
    from oracle import pd_oracle as po

    cfg, params, tokens, ci = _small()
    spec = po.ImpMin("smooth_l0", coeff=0.7, gamma=0.25, normalize_at_one=True, freq_coeff=0.3, ref_count=50.0)
    out = lo.lm_stack_step(cfg, params, tokens, ci, (7, 11), recon_coeff=0.0, imp_min=spec)
    ups = [po.upper_leaky(ci[l][k]) for l in range(cfg.n_layers) for k in cfg.kinds if k in cfg.C]
    act, freq = po.importance_minimality_terms(ups, 0.25, 50.0, True)
    assert out["imp"] == pytest.approx(act, rel=1e-12) and out["freq"] == pytest.approx(freq, rel=1e-12)
    assert out["loss"] == pytest.approx(0.7 * act + 0.3 * freq, rel=1e-12)
    for l in range(cfg.n_layers):
        for k in cfg.C:
            _, _, dup = po.impmin_site_terms(po.upper_leaky(ci[l][k]), spec, 10)
            want = po.upper_leaky_vjp(ci[l][k], dup)
            np.testing.assert_allclose(out["d_ci_pre"][l][k], want, rtol=1e-10, atol=1e-14)


def test_smooth_l0_ema_step_reads_the_debiased_estimate():
    """With the EMA estimate the LM step's frequency term is sum Phi(f_hat) over every
    site (ema_frequency_penalty of the per-site frequencies, itself pinned by the
    reference's closed forms), the new estimates are ema + alpha (f - ema), the batch
    penalty is the batch arm's, and at count 0 from a zero estimate every output equals
    the batch arm's (the first observation reproduces the un-smoothed penalty)."""
    from oracle import pd_oracle as po

    cfg, params, tokens, ci = _small()
    spec = po.ImpMin("smooth_l0", coeff=0.7, gamma=0.25, normalize_at_one=True, freq_coeff=0.3, ref_count=50.0,
                     ema_halflife=7.0)
    rng = np.random.default_rng(3)
    sites = [(l, k) for l in range(cfg.n_layers) for k in cfg.kinds if k in cfg.C]
    ema = [{k: rng.uniform(0.0, 0.5, size=cfg.C[k]) for k in cfg.C} for _ in range(cfg.n_layers)]
    out = lo.lm_stack_step(cfg, params, tokens, ci, (7, 11), recon_coeff=0.0, imp_min=spec, freq_ema=ema,
                           ema_count=2.0)
    freqs = {(l, k): po.smooth_l0_psi(po.upper_leaky(ci[l][k]), 0.25, True).mean(0) for l, k in sites}
    want, new = po.ema_frequency_penalty(freqs, {(l, k): ema[l][k] for l, k in sites}, 2.0, 7.0, 50.0)
    assert out["freq"] == pytest.approx(want, rel=1e-12)
    for l, k in sites:
        np.testing.assert_allclose(out["freq_ema"][l][k], new[(l, k)], rtol=1e-12)
    batch = lo.lm_stack_step(cfg, params, tokens, ci, (7, 11), recon_coeff=0.0, imp_min=spec)
    assert out["freq_batch"] == pytest.approx(batch["freq"], rel=1e-12)
    zero = [{k: np.zeros(cfg.C[k]) for k in cfg.C} for _ in range(cfg.n_layers)]
    first = lo.lm_stack_step(cfg, params, tokens, ci, (7, 11), recon_coeff=0.0, imp_min=spec, freq_ema=zero)
    assert first["freq"] == pytest.approx(batch["freq"], rel=1e-12)
    for l, k in sites:
        np.testing.assert_allclose(first["d_ci_pre"][l][k], batch["d_ci_pre"][l][k], rtol=1e-10, atol=1e-15)


def _stacked_model():
    """The reference's stacked-parity target (`pd/tests/targets/stacked_parity/
    stacked_fixtures.npz`, made by `gen_stacked_fixtures.py:95-150`): a residual-fed tiny
    GLU Llama (`tiny_glu_cfg`, `pd/targets/testing.py:107-122`: d 32, 4 heads over 2 kv
    heads, d_mlp 64, vocab 64, RoPE theta 5e5 with Llama-3 scaling (8, 1, 4, 128), eps
    1e-5) from layer 3 to 7, the MLP sites of layers 3-5 decomposed with C = 8."""
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "stacked_forward.npz")
    f = dict(np.load(path))
    first, last = int(f["_scalar_FIRST_LAYER"]), int(f["_scalar_LAST_LAYER"])
    cfg = lo.LMConfig(n_layers=8 - first, d=32, n_head=4, n_kv_head=2, d_mlp=64, vocab=64, mlp="glu", eps=1e-5,
                      rope_base=500000.0, rope_scaling=(8.0, 1.0, 4.0, 128.0),
                      C={k: int(f["_scalar_C"]) for k in ("gate_proj", "up_proj", "down_proj")})
    T = lambda a: torch.tensor(np.asarray(a, np.float64))  # noqa: E731
    names = {"q_proj": "wq", "k_proj": "wk", "v_proj": "wv", "o_proj": "wo", "gate_proj": "Wg", "up_proj": "Wu",
             "down_proj": "Wd"}
    layers, sites = [], []
    for i in range(first, 8):
        P = {"ln1": T(f[f"tgt::layers.{i}.ln1"]), "ln2": T(f[f"tgt::layers.{i}.ln2"])}
        for kind, nm in names.items():
            P["W_" + kind] = T(f[f"tgt::layers.{i}.{nm}"])
        if i <= last:
            for kind in ("gate_proj", "up_proj", "down_proj"):
                name = f"layers.{i}.mlp.{kind}"
                P["V_" + kind], P["U_" + kind] = T(f["vu::V::" + name]), T(f["vu::U::" + name])
                sites.append((i - first, kind, name))
        layers.append(P)
    params = {"layers": layers, "norm": T(f["tgt::norm"]), "head": T(f["tgt::lm_head"])}
    return f, cfg, params, sites


def test_stacked_reference_forward_golden():
    """The reference's frozen forward pins of that model in fp32 (its own test's bar: rtol
    1e-4, atol 1e-5): the clean logits, the masked logits with every decomposed site live
    (fixed masks and weight-delta masks), and the route arm, where only layer 3's sites
    are live, each with per-token routes (`pd/core/decomposed_linear.py:72-85`: unrouted
    positions take the target's x @ W^T) and the other sites run the target."""
    f, cfg, params, sites = _stacked_model()
    resid = torch.tensor(np.asarray(f["resid"], np.float64))
    n = cfg.n_layers

    def run(live, routes=None):
        masks = [dict() for _ in range(n)]
        deltas = [dict() for _ in range(n)]
        rts = [dict() for _ in range(n)]
        for l, kind, name in sites:
            if name in live:
                masks[l][kind] = torch.tensor(np.asarray(f["mask::" + name], np.float64))
                deltas[l][kind] = torch.tensor(np.asarray(f["delta_mask::" + name], np.float64))
                if routes is not None:
                    rts[l][kind] = routes[name]
        act = lo.forward(cfg, params, resid, masks, deltas, routes=rts)
        return lo.logits(params, act).numpy()

    clean = lo.logits(params, lo.forward(cfg, params, resid)).numpy()
    np.testing.assert_allclose(clean, f["out::clean"], rtol=1e-4, atol=1e-5)
    all_live = run({name for _, _, name in sites})
    np.testing.assert_allclose(all_live, f["out::masked_all"], rtol=1e-4, atol=1e-5)
    chunk0 = [name for _, _, name in sites][:3]
    routes = {name: np.asarray(f["route0::" + name]) for name in chunk0}
    assert set(routes) == {f"layers.3.mlp.{k}" for k in ("gate_proj", "up_proj", "down_proj")}
    assert 0 < np.mean([r.mean() for r in routes.values()]) < 1  # both arms taken
    subset = run(set(chunk0), routes)
    np.testing.assert_allclose(subset, f["out::masked_subset"], rtol=1e-4, atol=1e-5)
    # the pins separate the arms: without the routes the subset output moves off its golden
    assert np.abs(run(set(chunk0)) - f["out::masked_subset"]).max() > 1e-3


def test_source_tables_with_the_drawn_values_reproduce_the_draw_step():
    """One token per source row (`bsc`), tables holding exactly the step's own drawn u and
    d: loss and every gradient equal the draw path's (the source arm reads the same masks)."""
    cfg, params, tokens, ci = _small()
    key = (7, 11)
    kw = dict(p=2.0, imp_coeff=0.3, recon_coeff=1.7, bf16_storage=True)
    base = lo.lm_stack_step(cfg, params, tokens, ci, key, **kw)
    src = [{k: base["u"][(l, k)] for k in cfg.C} for l in range(cfg.n_layers)]
    srcd = [{k: base["delta"][(l, k)] for k in cfg.C} for l in range(cfg.n_layers)]
    got = lo.lm_stack_step(cfg, params, tokens, ci, key, sources=(src, srcd, 1), **kw)
    assert got["loss"] == base["loss"]
    for l in range(cfg.n_layers):
        for k in cfg.C:
            np.testing.assert_array_equal(got["dV"][l][k], base["dV"][l][k])
            np.testing.assert_array_equal(got["d_ci_pre"][l][k], base["d_ci_pre"][l][k])
            assert got["d_src"][l][k].shape == src[l][k].shape and got["d_src_delta"][l][k].shape == (10,)


@pytest.mark.parametrize("rps", [5, 10])
def test_source_table_gradients_match_finite_differences(rps):
    """float64: d_src and d_src_delta (rows of 5 tokens: one per sample, `bc`; 10: one
    row for the batch, `c`) against central differences of the loss."""
    cfg, params, tokens, ci = _small()
    rng = np.random.default_rng(9)
    S = 10 // rps
    src = [{k: rng.uniform(0.1, 0.9, size=(S, C)) for k, C in cfg.C.items()} for _ in range(cfg.n_layers)]
    srcd = [{k: rng.uniform(0.1, 0.9, size=S) for k in cfg.C} for _ in range(cfg.n_layers)]
    kw = dict(p=2.0, imp_coeff=0.3, recon_coeff=1.7, sources=(src, srcd, rps))
    base = lo.lm_stack_step(cfg, params, tokens, ci, (1, 2), **kw)
    eps = 1e-6
    for l, kind in ((0, "q_proj"), (1, "c_fc"), (1, "down_proj")):
        for tables, grads in ((src, base["d_src"]), (srcd, base["d_src_delta"])):
            arr = tables[l][kind]
            for _ in range(2):
                i = tuple(int(rng.integers(0, s)) for s in arr.shape)
                old = arr[i]
                arr[i] = old + eps
                up = lo.lm_stack_step(cfg, params, tokens, ci, (1, 2), **kw)["loss"]
                arr[i] = old - eps
                dn = lo.lm_stack_step(cfg, params, tokens, ci, (1, 2), **kw)["loss"]
                arr[i] = old
                assert (up - dn) / (2 * eps) == pytest.approx(grads[l][kind][i], rel=1e-5, abs=1e-9), (l, kind, i)
