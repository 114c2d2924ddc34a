"""Toy-target decomposition steps (TMS, ResidMLP) in float64 NumPy.

Test infrastructure only: the GPU harness in `param_decomp_amd/toys.py` is checked
against these functions; nothing in the product imports them.

Targets, restated:
- TMS (`param_decomp/param_decomp/targets/tms.py:254-258` clean output, `:261-271`
  clean site inputs, `:311-359` masked forward): `hidden = linear1(x)`,
  `out = relu(linear2(hidden) + b2)`; the untrained target ties `W2 = W1^T`
  (`tms.py:569-581`). No hidden layers (the 5-2 configuration).
- ResidMLP (`targets/resid_mlp.py:336-390` masked, `:266-333` clean):
  `resid = x @ W_E`; per layer `resid += mlp_out(act(mlp_in(resid) + b_in)) + b_out`;
  `out = resid @ W_U`; fixed unit-norm embedding with `W_U = W_E^T`
  (`resid_mlp.py:614-628`), Kaiming-uniform blocks (`:596-611`), act = relu (`:158`).

One step (the stochastic-recon + imp-min objective of the engine, `core/train.py:1182-1258`
with `StochasticSources` and `AllRouting` or given routes): clean forward (recon target
and each site's clean input), CI = gate(clean_input @ V) per site (paper form), lower /
upper leaky hard sigmoids, masks from `split(draw_key)` -> `fold_in(., site_idx)` in site
order drawn in the CI dtype (fp32; `core/masking.py:148-167`), masked forward through
`site_forward`, MSE recon (`tms.py:380-388`, `resid_mlp.py:411-418`), p-norm imp-min
summed over sites, and the chain-rule backward to every site's V, U and gate
parameters (the gate reads `clean_input @ V`, so dV has a gate term).

Pinned by: composition of the pinned site / gate / mask / loss functions of
`pd_oracle`, finite differences of the whole step loss (tests/test_toy_oracle.py), and
the clean-target invariants (tied TMS weights, unit-norm embedding rows).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import pd_oracle as po


@dataclass(frozen=True)
class TMSConfig:
    n_features: int = 5
    n_hidden: int = 2
    C: int = 20
    batch: int = 4096
    feature_probability: float = 0.05


@dataclass(frozen=True)
class ResidMLPConfig:
    n_features: int = 100
    d_embed: int = 1000
    d_mlp: int = 50
    n_layers: int = 1
    C: int = 100
    batch: int = 2048
    feature_probability: float = 0.01


@dataclass
class ToySite:
    name: str
    W: np.ndarray  # [d_out, d_in] frozen target weight
    V: np.ndarray  # [d_in, C]
    U: np.ndarray  # [C, d_out]
    gate: po.GateParams


def init_gate(C: int, rng, *, H: int = 16, bias_scale: float = 0.0) -> po.GateParams:
    """Per-component scalar MLP: Kaiming-normal weights (fan-in 1 and H), biases zero
    (or `bias_scale`-wide normal noise for tests that need varied operating points)."""
    return po.GateParams(rng.normal(size=(C, H)) * np.sqrt(2.0), rng.normal(size=(C, H)) * bias_scale,
                         rng.normal(size=(C, H)) * np.sqrt(2.0 / H), rng.normal(size=C) * bias_scale)


def init_site(name: str, W: np.ndarray, C: int, rng, **gate_kw) -> ToySite:
    """V ~ N(0, 1/d_in), U ~ N(0, 1/C) (`core/components.py:650-677`)."""
    d_out, d_in = W.shape
    return ToySite(name, W, rng.normal(size=(d_in, C)) / np.sqrt(d_in), rng.normal(size=(C, d_out)) / np.sqrt(C),
                   init_gate(C, rng, **gate_kw))


def tms_init(cfg: TMSConfig, rng, **gate_kw):
    """Untrained tied TMS target (`tms.py:569-581`, zero bias) and its two sites."""
    b = 1.0 / np.sqrt(cfg.n_features)
    W1 = rng.uniform(-b, b, size=(cfg.n_hidden, cfg.n_features))
    target = {"W1": W1, "b2": np.zeros(cfg.n_features)}
    sites = [init_site("linear1", W1, cfg.C, rng, **gate_kw), init_site("linear2", W1.T.copy(), cfg.C, rng, **gate_kw)]
    return target, sites


def tms_batch(cfg: TMSConfig, rng) -> np.ndarray:
    """`at_least_zero_active` features (`tms.py:584-609`): U(0,1) values gated by
    U(0,1) < p (seeded NumPy draws stand in for the reference's jax.random draws)."""
    v = rng.uniform(0.0, 1.0, size=(cfg.batch, cfg.n_features))
    return v * (rng.uniform(size=v.shape) < cfg.feature_probability)


def resid_mlp_init(cfg: ResidMLPConfig, rng, **gate_kw):
    """Fixed random unit-norm embedding with `W_U = W_E^T` and Kaiming-uniform blocks
    without biases (`resid_mlp.py:596-628`); sites `layers.{i}.mlp_in/mlp_out`."""
    raw = rng.normal(size=(cfg.n_features, cfg.d_embed))
    W_E = raw / np.linalg.norm(raw, axis=-1, keepdims=True)
    target = {"W_E": W_E, "W_U": W_E.T.copy(), "layers": []}
    sites = []
    for i in range(cfg.n_layers):
        bi, bo = 1.0 / np.sqrt(cfg.d_embed), 1.0 / np.sqrt(cfg.d_mlp)
        W_in = rng.uniform(-bi, bi, size=(cfg.d_mlp, cfg.d_embed))
        W_out = rng.uniform(-bo, bo, size=(cfg.d_embed, cfg.d_mlp))
        target["layers"].append({"b_in": None, "b_out": None})
        sites.append(init_site(f"layers.{i}.mlp_in", W_in, cfg.C, rng, **gate_kw))
        sites.append(init_site(f"layers.{i}.mlp_out", W_out, cfg.C, rng, **gate_kw))
    return target, sites


def resid_mlp_batch(cfg: ResidMLPConfig, rng) -> np.ndarray:
    """`at_least_zero_active` (`resid_mlp.py:643-662`): U(-1,1) values gated by U < p."""
    v = rng.uniform(-1.0, 1.0, size=(cfg.batch, cfg.n_features))
    return v * (rng.uniform(size=v.shape) < cfg.feature_probability)


def relu(a):
    return np.maximum(a, 0.0)


def _bias(a, b):
    return a if b is None else a + b


def clean_forward(kind: str, target, sites, x):
    """Clean output and each site's clean input (`tms.py:254-271`; `resid_mlp.py:266-333`)."""
    if kind == "tms":
        hidden = x @ sites[0].W.T
        return relu(hidden @ sites[1].W.T + target["b2"]), [x, hidden]
    r = x @ target["W_E"]
    inputs = []
    for i, lay in enumerate(target["layers"]):
        s_in, s_out = sites[2 * i], sites[2 * i + 1]
        hid = relu(_bias(r @ s_in.W.T, lay["b_in"]))
        inputs += [r, hid]
        r = r + _bias(hid @ s_out.W.T, lay["b_out"])
    return r @ target["W_U"], inputs


def toy_step(kind: str, target, sites, x, draw_key, *, p: float = 1.0, imp_coeff: float = 1.0,
             recon_coeff: float = 1.0, use_delta: bool = False, routes=None, partitionable: bool = True):
    """One fwd+bwd of the toy decomposition objective (see module docstring). Returns a
    dict with loss, recon, imp, out, clean, the per-site CI (g_raw, lower, upper), masks
    and the gradients dV, dU, dgate (w_in, b_in, w_out, b_out) per site."""
    n = len(sites)
    clean, cin = clean_forward(kind, target, sites, x)
    h = [cin[i] @ sites[i].V for i in range(n)]
    g = [po.gate_forward(h[i], sites[i].gate) for i in range(n)]
    lo = [po.lower_leaky(a) for a in g]
    up = [po.upper_leaky(a) for a in g]
    draws = [po.draw_site_mask(lo[i], draw_key, i, "float32", with_delta=use_delta, partitionable=partitionable)
             for i in range(n)]
    m = [d[0] for d in draws]
    dl = [d[1] for d in draws]
    u = [d[2] for d in draws]
    rt = [None if routes is None else routes[i] for i in range(n)]

    def site(i, a):
        return po.site_forward(a, sites[i].W, sites[i].V, sites[i].U, m[i], dl[i], rt[i])[0]

    def site_bwd(i, a, dout):
        return po.site_backward(a, sites[i].W, sites[i].V, sites[i].U, m[i], dl[i], rt[i], dout)

    dV = [None] * n
    dU = [None] * n
    dm = [None] * n
    if kind == "tms":
        s0 = site(0, x)
        pre = site(1, s0) + target["b2"]
        out = relu(pre)
        recon = po.mse(out, clean)
        d_out = recon_coeff * 2.0 * (out - clean) / out.size
        d_pre = d_out * (pre > 0)
        d_s0, dV[1], dU[1], dm[1] = site_bwd(1, s0, d_pre)
        _, dV[0], dU[0], dm[0] = site_bwd(0, x, d_s0)
    else:
        r = x @ target["W_E"]
        saved = []
        for i, lay in enumerate(target["layers"]):
            pre = _bias(site(2 * i, r), lay["b_in"])
            hid = relu(pre)
            saved.append((r, pre, hid))
            r = r + _bias(site(2 * i + 1, hid), lay["b_out"])
        out = r @ target["W_U"]
        recon = po.mse(out, clean)
        d_out = recon_coeff * 2.0 * (out - clean) / out.size
        d_r = d_out @ target["W_U"].T
        for i in reversed(range(len(target["layers"]))):
            r_in, pre, hid = saved[i]
            d_hid, dV[2 * i + 1], dU[2 * i + 1], dm[2 * i + 1] = site_bwd(2 * i + 1, hid, d_r)
            d_pre = d_hid * (pre > 0)
            d_rin, dV[2 * i], dU[2 * i], dm[2 * i] = site_bwd(2 * i, r_in, d_pre)
            d_r = d_r + d_rin
    imp = sum(po.impmin_pnorm(a, p) for a in up)
    loss = recon_coeff * recon + imp_coeff * imp
    dgate = []
    for i in range(n):
        d_lo = dm[i] * (1.0 - u[i])
        dg = po.lower_leaky_vjp(g[i], d_lo) + po.upper_leaky_vjp(g[i], imp_coeff * po.impmin_pnorm_grad(up[i], p))
        dh, dwi, dbi, dwo, dbo = po.gate_backward(h[i], sites[i].gate, dg)
        dV[i] = dV[i] + cin[i].T @ dh
        dgate.append((dwi, dbi, dwo, dbo))
    return dict(loss=loss, recon=recon, imp=imp, out=out, clean=clean, g_raw=g, lower=lo, upper=up, mask=m,
                delta=dl, dV=dV, dU=dU, dgate=dgate)
