"""NumPy restatement of the masked-component path (oracle only; float64 arithmetic).

Every function cites the reference file it follows. Paths are relative to the
reference repository root; `pd/` = `param_decomp/param_decomp/`.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
from scipy.special import erf

from oracle import threefry

ALPHA = 0.01
SQRT1_2 = 1.0 / math.sqrt(2.0)
INV_SQRT_2PI = 1.0 / math.sqrt(2.0 * math.pi)


# ---------------------------------------------------------------- squashing
def lower_leaky(x):
    """`pd/core/ci_fn/squashing.py:8-14`: forward is `clip(x, 0, 1)`."""
    return np.clip(x, 0.0, 1.0)


def lower_leaky_vjp(x, g):
    """`pd/core/ci_fn/squashing.py:17-19` (`_lhs_b`): leak `0.01*g` below zero only when
    `g < 0`; pass `g` on (0, 1] (x=0 takes the lower branch, x=1 the middle); 0 above."""
    leak = np.where(g < 0, ALPHA * g, 0.0)
    return np.where(x <= 0, leak, np.where(x <= 1, g, 0.0))


def upper_leaky(x):
    """`pd/core/ci_fn/squashing.py:41-45`: `x>1 ? 1+0.01(x-1) : clip(x,0,1)`."""
    return np.where(x > 1, 1 + ALPHA * (x - 1), np.clip(x, 0.0, 1.0))


def upper_leaky_vjp(x, g):
    """Plain autodiff of `upper_leaky` as JAX differentiates it: `where` routes the
    cotangent; `clip` is `min(max(x, 0), 1)` and JAX's max/min JVP gives half the
    cotangent to each operand at an exact tie, so x == 0 and x == 1 pass `0.5*g`."""
    clip_grad = np.where((x > 0) & (x < 1), 1.0, np.where((x == 0) | (x == 1), 0.5, 0.0))
    return np.where(x > 1, ALPHA * g, clip_grad * g)


# ---------------------------------------------------------------- gate MLP (paper form)
@dataclass
class GateParams:
    """Per-component gate MLP: `w_in, b_in, w_out` are `[C, H]`, `b_out` is `[C]`
    (`papers/Stochastic_Parameter_Decomposition/spd_paper.md`, appendix "Architecture of
    Causal Importance Function MLPs": one hidden GELU layer of width d_gate per
    component, scalar input h_c, scalar output)."""

    w_in: np.ndarray
    b_in: np.ndarray
    w_out: np.ndarray
    b_out: np.ndarray


def gelu(z):
    """Exact (erf) GELU, the engine's choice (`pd/core/ci_fn/implementations/mlp.py:77`)."""
    return 0.5 * z * (1.0 + erf(z * SQRT1_2))


def gelu_grad(z):
    return 0.5 * (1.0 + erf(z * SQRT1_2)) + z * INV_SQRT_2PI * np.exp(-0.5 * z * z)


def gate_forward(h, p: GateParams):
    """`g_raw[t,c] = b_out[c] + sum_j w_out[c,j] * GELU(w_in[c,j]*h[t,c] + b_in[c,j])`."""
    z = h[..., None] * p.w_in + p.b_in
    return np.sum(gelu(z) * p.w_out, axis=-1) + p.b_out


def gate_backward(h, p: GateParams, dg_raw):
    """VJP of `gate_forward`: returns (dh, dw_in, db_in, dw_out, db_out)."""
    z = h[..., None] * p.w_in + p.b_in
    lead = tuple(range(h.ndim - 1))
    dz = dg_raw[..., None] * p.w_out * gelu_grad(z)
    dh = np.sum(dz * p.w_in, axis=-1)
    dw_in = np.sum(dz * h[..., None], axis=lead)
    db_in = np.sum(dz, axis=lead)
    dw_out = np.sum(dg_raw[..., None] * gelu(z), axis=lead)
    db_out = np.sum(dg_raw, axis=lead)
    return dh, dw_in, db_in, dw_out, db_out


# ---------------------------------------------------------------- masks
def component_mask(ci_lower, u):
    """`pd/core/masking.py:135-136`: `m = g + (1 - g) * u`."""
    return ci_lower + (1.0 - ci_lower) * u


def site_keys(draw_key, site_idx: int, *, partitionable: bool = True):
    """`pd/core/masking.py:148-167` (`materialize_masking`): `mask_key, delta_key =
    split(draw_key)`, then `fold_in(., site_idx)` in CI insertion order."""
    mask_key, delta_key = threefry.split(draw_key, 2, partitionable=partitionable)
    return threefry.fold_in(mask_key, site_idx), threefry.fold_in(delta_key, site_idx)


def draw_site_mask(ci_lower, draw_key, site_idx, dtype="bfloat16", *, with_delta=True, partitionable=True):
    """Site mask and delta exactly as the toy targets draw them
    (`pd/core/masking.py:162-167`; `pd/core/linear_plan.py:80-106`): uniforms in the CI
    dtype, delta drops the trailing component axis."""
    mk, dk = site_keys(draw_key, site_idx, partitionable=partitionable)
    u = threefry.uniform(mk, ci_lower.shape, dtype, partitionable=partitionable)
    m = component_mask(ci_lower, u)
    d = threefry.uniform(dk, ci_lower.shape[:-1], dtype, partitionable=partitionable) if with_delta else None
    return m, d, u


# ---------------------------------------------------------------- decomposed linear
def site_forward(x, W, V, U, mask, delta=None, route=None):
    """`pd/core/decomposed_linear.py:142-175` with `:65-85`:
    `where(route, ((x@V)*(m-d))@U + d*(x@W.T), x@W.T)`. Returns (output, x@V)."""
    xV = x @ V
    coef = mask if delta is None else mask - delta[..., None]
    out = (xV * coef) @ U
    if delta is None and route is None:
        return out, xV
    target = x @ W.T
    blended = out if delta is None else out + delta[..., None] * target
    if route is not None:
        blended = np.where(route[..., None], blended, target)
    return blended, xV


def site_backward(x, W, V, U, mask, delta, route, dout):
    """VJP of `site_forward` w.r.t. (x, V, U, mask) given the output cotangent."""
    xV = x @ V
    coef = mask if delta is None else mask - delta[..., None]
    dcomp = dout if route is None else np.where(route[..., None], dout, 0.0)
    acts = xV * coef
    dU = acts.reshape(-1, acts.shape[-1]).T @ dcomp.reshape(-1, dcomp.shape[-1])
    dacts = dcomp @ U.T
    dmask = dacts * xV
    dxV = dacts * coef
    dV = x.reshape(-1, x.shape[-1]).T @ dxV.reshape(-1, dxV.shape[-1])
    dx = dxV @ V.T
    if delta is not None or route is not None:
        dtarget = np.zeros_like(dout)
        if delta is not None:
            dtarget = dtarget + (dcomp * delta[..., None])
        if route is not None:
            dtarget = dtarget + np.where(route[..., None], 0.0, dout)
        dx = dx + dtarget @ W
    return dx, dV, dU, dmask


def site_delta_grad(x, W, V, U, mask, delta, route, dout):
    """VJP of `site_forward` w.r.t. the per-position delta (`[*lead]`): for a routed
    position `sum_o dout * (x@W.T - (x@V*1)@U)`, i.e. `sum_o dout*target - sum_c
    (dout@U.T)*xV`; 0 where unrouted. The weight-delta sources of adversarial masking
    take this cotangent (`pd/core/source_mask.py:61-63`)."""
    xV = x @ V
    target = x @ W.T
    g = np.sum(dout * target, axis=-1) - np.sum((dout @ U.T) * xV, axis=-1)
    return g if route is None else np.where(route, g, 0.0)


# ---------------------------------------------------------------- block-factored site
def blocked_site_forward(x, W, V, U, mask, delta, route, contraction):
    """`pd/core/decomposed_linear.py:209-271` dense over every block, with the einsums of
    `pd/core/linear_plan.py:149-160`: fused_output `xV = einsum('ti,eij->tej')`,
    `out = einsum('tej,ejk->tek')` flattened; fused_input `xV = einsum('tei,eij->tej')`,
    `out = einsum('tej,ejk->tk')`. mask / delta / route as `site_forward` with the flat
    block-major `C = E*c`. Returns (output, xV_flat)."""
    E, d_in, c = V.shape
    T = x.shape[0]
    if contraction == "fused_output":
        xV = np.einsum("ti,eij->tej", x, V)
    else:
        xV = np.einsum("tei,eij->tej", x.reshape(T, E, d_in), V)
    xV_flat = xV.reshape(T, E * c)
    coef = mask if delta is None else mask - delta[:, None]
    acts = (xV_flat * coef).reshape(T, E, c)
    if contraction == "fused_output":
        out = np.einsum("tej,ejk->tek", acts, U).reshape(T, -1)
    else:
        out = np.einsum("tej,ejk->tk", acts, U)
    if delta is None and route is None:
        return out, xV_flat
    target = x @ W.T
    blended = out if delta is None else out + delta[:, None] * target
    if route is not None:
        blended = np.where(route[:, None], blended, target)
    return blended, xV_flat


def blocked_site_forward_loop(x, W, V, U, mask, delta, route, contraction):
    """The same site written block by block (as `tests/core/test_blocked_factorization.py`'s
    per-block loop reference): the second formulation the einsum form is checked against."""
    E, d_in, c = V.shape
    T = x.shape[0]
    if contraction == "fused_output":
        xV = np.stack([x @ V[e] for e in range(E)], axis=1)
    else:
        xe = x.reshape(T, E, d_in)
        xV = np.stack([xe[:, e] @ V[e] for e in range(E)], axis=1)
    xV_flat = xV.reshape(T, E * c)
    coef = mask if delta is None else mask - delta[:, None]
    acts = (xV_flat * coef).reshape(T, E, c)
    if contraction == "fused_output":
        out = np.concatenate([acts[:, e] @ U[e] for e in range(E)], axis=-1)
    else:
        out = sum(acts[:, e] @ U[e] for e in range(E))
    frozen = x @ W.T
    if delta is not None:
        out = out + delta[:, None] * frozen
    if route is not None:
        out = np.where(route[:, None], out, frozen)
    return out, xV_flat


def blocked_site_backward(x, W, V, U, mask, delta, route, contraction, dout):
    """VJP of `blocked_site_forward` w.r.t. (x, V, U, mask)."""
    E, d_in, c = V.shape
    T = x.shape[0]
    fo = contraction == "fused_output"
    xe = None if fo else x.reshape(T, E, d_in)
    xV = np.einsum("ti,eij->tej", x, V) if fo else np.einsum("tei,eij->tej", xe, V)
    coef = (mask if delta is None else mask - delta[:, None]).reshape(T, E, c)
    dcomp = dout if route is None else np.where(route[:, None], dout, 0.0)
    acts = xV * coef
    if fo:
        g = dcomp.reshape(T, E, -1)
        dU = np.einsum("tej,tek->ejk", acts, g)
        dacts = np.einsum("tek,ejk->tej", g, U)
    else:
        dU = np.einsum("tej,tk->ejk", acts, dcomp)
        dacts = np.einsum("tk,ejk->tej", dcomp, U)
    dmask = (dacts * xV).reshape(T, E * c)
    dxV = dacts * coef
    if fo:
        dV = np.einsum("ti,tej->eij", x, dxV)
        dx = np.einsum("tej,eij->ti", dxV, V)
    else:
        dV = np.einsum("tei,tej->eij", xe, dxV)
        dx = np.einsum("tej,eij->tei", dxV, V).reshape(T, E * d_in)
    if delta is not None or route is not None:
        dtarget = np.zeros_like(dout)
        if delta is not None:
            dtarget = dtarget + dcomp * delta[:, None]
        if route is not None:
            dtarget = dtarget + np.where(route[:, None], 0.0, dout)
        dx = dx + dtarget @ W
    return dx, dV, dU, dmask


# ---------------------------------------------------------------- losses
def blocked_site_delta_grad(x, W, V, U, mask, delta, route, contraction, dout):
    """VJP of `blocked_site_forward` w.r.t. the per-position delta: for a routed position
    `sum_o dout*(x@W.T) - sum_c dmask_c` (the mask cotangent `dacts*xV` of
    `blocked_site_backward`, since the coefficients are `m - d`); 0 where unrouted."""
    _, _, _, dmask = blocked_site_backward(x, W, V, U, mask, delta, route, contraction, dout)
    g = np.sum(dout * (x @ W.T), axis=-1) - np.sum(dmask, axis=-1)
    return g if route is None else np.where(route, g, 0.0)


def impmin_pnorm(ci_upper, p: float, eps: float = 0.0, beta: float = 0.0, world_size: int = 1):
    """L_p importance minimality. Paper algorithm step 4
    (`spd_paper.md`, "Algorithm"): `(1/B) sum_b sum_c |upper|^p`; with the `eps`/`beta`
    extension of `nano_param_decomp/run.py:413-429`:
    `sum_c [mean_c + beta*mean_c*log2(1 + sum_c*world_size)]`, values `(upper+eps)^p`."""
    vals = (ci_upper + eps) ** p
    flat = vals.reshape(-1, vals.shape[-1])
    s = flat.sum(axis=0)
    mean = s / flat.shape[0]
    return float(np.sum(mean + beta * mean * np.log2(1.0 + s * world_size)))


def impmin_pnorm_grad(ci_upper, p: float, eps: float = 0.0, beta: float = 0.0, world_size: int = 1):
    """d impmin_pnorm / d ci_upper."""
    vals = (ci_upper + eps) ** p
    flat = vals.reshape(-1, vals.shape[-1])
    n = flat.shape[0]
    s = flat.sum(axis=0)
    a = s * world_size
    dsum = (1.0 / n) * (1.0 + beta * np.log2(1.0 + a)) + beta * (s / n) * world_size / ((1.0 + a) * math.log(2.0))
    dvals = p * (ci_upper + eps) ** (p - 1.0)
    return dvals * dsum


def smooth_l0_psi(c, gamma: float, normalize_at_one: bool = False):
    """`pd/core/losses.py:388-394`: `c^2/(c^2+gamma^2)` (times `1+gamma^2` when
    normalized at one)."""
    g2 = gamma * gamma
    base = c * c / (c * c + g2)
    return (1.0 + g2) * base if normalize_at_one else base


def smooth_l0_psi_grad(c, gamma: float, normalize_at_one: bool = False):
    g2 = gamma * gamma
    d = 2.0 * c * g2 / (c * c + g2) ** 2
    return (1.0 + g2) * d if normalize_at_one else d


def importance_minimality_terms(ci_upper_sites, gamma, reference_datapoint_count=None, normalize_at_one=False):
    """`pd/core/losses.py:462-485`: activity `sum_sites sum_c mean_t psi`, and the
    frequency penalty `sum f*log2(1 + a'*f)` (`:375-386, 425-458`) when a reference
    datapoint count is given."""
    activity = 0.0
    freq = 0.0
    for v in ci_upper_sites:
        f = smooth_l0_psi(v, gamma, normalize_at_one).reshape(-1, v.shape[-1]).mean(axis=0)
        activity += float(f.sum())
        if reference_datapoint_count is not None:
            freq += float(np.sum(f * np.log2(1.0 + reference_datapoint_count * f)))
    return activity, freq


def frequency_curve(f, reference_datapoint_count):
    """`pd/core/losses.py:375-377`: `Phi(f) = f log2(1 + a' f)`."""
    return f * np.log2(1.0 + reference_datapoint_count * f)


def frequency_curve_slope(f, reference_datapoint_count):
    """`pd/core/losses.py:380-386`: `Phi'(f) = log2(1 + a' f) + a' f / ((1 + a' f) ln 2)`."""
    af = reference_datapoint_count * f
    return np.log2(1.0 + af) + af / ((1.0 + af) * math.log(2.0))


def ema_decay_terms(count: float, halflife_steps: float):
    """`(alpha, debias) = (1 - decay, 1 - decay^(count + 1))`, `decay = 2^(-1/h)`, both
    formed through `expm1` of `log(decay) = -ln 2 / h` (`pd/core/losses.py:449-451`)."""
    log_decay = -math.log(2.0) / halflife_steps
    return -math.expm1(log_decay), -math.expm1(log_decay * (count + 1.0))


def ema_frequency_update(f_batch, ema, count: float, halflife_steps: float):
    """One observation of the running estimate (`pd/core/losses.py:452-455`):
    `new = ema + alpha (f - ema)`, `f_hat = new / debias`. Returns `(new, f_hat)`."""
    alpha, debias = ema_decay_terms(count, halflife_steps)
    new = ema + alpha * (np.asarray(f_batch, np.float64) - ema)
    return new, new / debias


def ema_frequency_penalty(frequencies: dict, ema: dict, count: float, halflife_steps: float,
                          reference_datapoint_count):
    """`pd/core/losses.py:425-458`: `(freq, new_ema)`, the penalty `sum Phi(f_hat)` at the
    debiased estimate after this batch (its gradient, `Phi'(f_hat) df_batch`, is
    `ema_frequency_slope`'s)."""
    freq = 0.0
    new_ema = {}
    for name, f in frequencies.items():
        new_ema[name], f_hat = ema_frequency_update(f, ema[name], count, halflife_steps)
        freq += float(np.sum(frequency_curve(f_hat, reference_datapoint_count)))
    return freq, new_ema


@dataclass(frozen=True)
class ImpMin:
    """The imp-min term of a fused step. `kind="pnorm"`: `coeff * sum upper^p / n` (the
    paper's L_p, the selected arm of `pd/core/losses.py:357-372` for p = smooth-L0's
    stand-in). `kind="smooth_l0"`: the engine's term (`pd/core/objective.py:101-131`):
    `coeff * sum_c f_c + freq_coeff * sum_c f_c log2(1 + ref_count f_c)` with
    `f_c = sum psi(upper) / n` (`pd/core/losses.py:316-330, 375-394`), the frequency term
    off when `ref_count` is 0. `n` is the token count of the batch. `ema_halflife` (the
    config's `ema_halflife_steps`, `pd/core/configs.py:182`) evaluates the frequency term
    at the debiased running estimate (`ema_frequency_penalty`); the steps then take the
    estimate before the batch and its observation count."""

    kind: str = "pnorm"
    p: float = 2.0
    coeff: float = 1.0
    gamma: float = 1.0
    normalize_at_one: bool = False
    freq_coeff: float = 0.0
    ref_count: float = 0.0
    ema_halflife: float | None = None

    def loss(self, activity: float, frequency: float) -> float:
        return self.coeff * activity + (self.freq_coeff * frequency if self.kind == "smooth_l0" else 0.0)


def impmin_site_terms(up, spec: ImpMin, n: int, groups=None, n_groups: int = 1):
    """One site's `(activity, frequency, d loss / d up)` for its upper CI `up` [..., c].
    `groups` (the leading shape of `up`) maps each row to its block of the full
    `[n_groups * c]` component vector, as a selected-emitting site's values map to their
    expert's components (`pd/core/losses.py:316-330`: scatter-add of psi, divided by the
    token count n; unselected pairs add psi(0) = 0). The gradient includes the
    coefficients: `coeff * p up^(p-1) / n` (L_p) or
    `(coeff + freq_coeff * Phi'(f_c)) / n * psi'(up)` (smooth-L0, `Phi'` of
    `pd/core/losses.py:380-386`)."""
    return impmin_site_terms_ema(up, spec, n, groups, n_groups)[:3]


def impmin_site_terms_ema(up, spec: ImpMin, n: int, groups=None, n_groups: int = 1, ema=None, count: float = 0.0):
    """`impmin_site_terms` plus the EMA estimator: with `ema` (the site's `[n_groups * c]`
    estimate before this batch; `spec.ema_halflife` set) the frequency term is
    `sum Phi(f_hat)` and its slope `Phi'(f_hat)` (`pd/core/losses.py:425-458`: the
    surrogate `Phi'(f_hat) (f - sg(f))` keeps the gradient at the batch penalty's scale).
    Returns `(activity, frequency, grad, new_ema, batch_frequency)`; `new_ema` is None
    and `batch_frequency` the frequency term without the EMA."""
    up = np.asarray(up, np.float64)
    if spec.kind == "pnorm":
        return float(np.sum(up**spec.p)) / n, 0.0, spec.coeff * spec.p * up ** (spec.p - 1.0) / n, None, 0.0
    if spec.kind != "smooth_l0":
        raise ValueError(spec.kind)
    c = up.shape[-1]
    psi = smooth_l0_psi(up, spec.gamma, spec.normalize_at_one).reshape(-1, c)
    g = np.zeros(psi.shape[0], np.int64) if groups is None else np.asarray(groups).reshape(-1).astype(np.int64)
    F = np.zeros((n_groups, c))
    np.add.at(F, g, psi)
    f = F / n
    act = float(f.sum())
    freq = batch = 0.0
    new_ema = None
    slope = np.full_like(f, spec.coeff)
    if spec.ref_count > 0:
        fe = f
        batch = float(np.sum(frequency_curve(f, spec.ref_count)))
        if ema is not None:
            if spec.ema_halflife is None:
                raise ValueError("an EMA estimate needs spec.ema_halflife")
            new_ema, fe = ema_frequency_update(f.reshape(-1), np.asarray(ema, np.float64).reshape(-1), count,
                                               spec.ema_halflife)
            fe = fe.reshape(f.shape)
        freq = float(np.sum(frequency_curve(fe, spec.ref_count)))
        slope = slope + spec.freq_coeff * frequency_curve_slope(fe, spec.ref_count)
    elif ema is not None:
        raise ValueError("the EMA estimate needs the frequency term (ref_count > 0)")
    grad = (slope / n)[g].reshape(up.shape) * smooth_l0_psi_grad(up, spec.gamma, spec.normalize_at_one)
    return act, freq, grad, new_ema, batch


def mse(masked, clean):
    """`pd/targets/tms.py:380-388`, `pd/targets/resid_mlp.py:411-418`:
    `mean((masked - clean)^2)` in fp32."""
    return float(np.mean((masked - clean) ** 2))


def relative_squared_error(masked, clean):
    """`pd/core/losses.py:60-76`: mean over positions of `|m-c|^2 / max(|c|^2, 1e-8)`."""
    se = np.sum((masked - clean) ** 2, axis=-1)
    sc = np.sum(clean**2, axis=-1)
    return float(np.mean(se / np.maximum(sc, 1e-8)))


def log_softmax(z):
    z = z - z.max(axis=-1, keepdims=True)
    return z - np.log(np.sum(np.exp(z), axis=-1, keepdims=True))


def kl_per_position(masked_logits, clean_logits):
    """`pd/core/losses.py:80-92`, `pd/targets/losses.py:50-60`: KL(clean || masked) per
    position with the clean distribution frozen."""
    lp = log_softmax(clean_logits)
    lq = log_softmax(masked_logits)
    return np.sum(np.exp(lp) * (lp - lq), axis=-1)


def categorical_kl(masked_logits, clean_logits):
    return float(np.mean(kl_per_position(masked_logits, clean_logits)))


def categorical_kl_grad(masked_logits, clean_logits):
    """d mean_pos KL / d masked_logits = (softmax(masked) - softmax(clean)) / n_pos."""
    n = int(np.prod(masked_logits.shape[:-1]))
    return (np.exp(log_softmax(masked_logits)) - np.exp(log_softmax(clean_logits))) / n


def streamed_position_kl(act_masked, head_masked, act_clean, head_clean, n_chunks: int):
    """`param_decomp/param_decomp/targets/losses.py:101-163` (`streamed_position_kl`):
    per-position KL(softmax(clean) || softmax(masked)) with `z = act @ head.T` streamed
    over `n_chunks` equal vocab chunks through the paired online-softmax accumulators
    (running maxima m_p, m_q, rescaled sums s_p, s_q and the p-weighted cross term a):
    `KL = a/s_p - (m_p + log s_p) + (m_q + log s_q)`. Returns (kl [N], stats [N, 5] =
    (m_p, s_p, a, m_q, s_q))."""
    V = head_masked.shape[0]
    assert V % n_chunks == 0, (V, n_chunks)
    ch = V // n_chunks
    N = act_masked.shape[0]
    m_p = np.full(N, -np.inf)
    m_q = np.full(N, -np.inf)
    s_p = np.zeros(N)
    s_q = np.zeros(N)
    a = np.zeros(N)
    for c in range(n_chunks):
        zp = act_clean @ head_clean[c * ch:(c + 1) * ch].T
        zq = act_masked @ head_masked[c * ch:(c + 1) * ch].T
        mp2 = np.maximum(m_p, zp.max(axis=-1))
        mq2 = np.maximum(m_q, zq.max(axis=-1))
        rp = np.exp(m_p - mp2)
        ep = np.exp(zp - mp2[:, None])
        s_p = s_p * rp + ep.sum(axis=-1)
        a = a * rp + np.sum(ep * (zp - zq), axis=-1)
        s_q = s_q * np.exp(m_q - mq2) + np.exp(zq - mq2[:, None]).sum(axis=-1)
        m_p, m_q = mp2, mq2
    kl = a / s_p - (m_p + np.log(s_p)) + (m_q + np.log(s_q))
    return kl, np.stack([m_p, s_p, a, m_q, s_q], axis=-1)


def streamed_position_kl_vjp(act_masked, head_masked, act_clean, head_clean, g_position):
    """Cotangent of the masked activations: `sum_v (q_v - p_v) g_n head_masked[v]`
    (the exact softmax cotangent the reference's checkpointed scan flows back; the clean
    side is the stop-gradient target)."""
    q = np.exp(log_softmax(act_masked @ head_masked.T))
    p = np.exp(log_softmax(act_clean @ head_clean.T))
    return ((q - p) * g_position[:, None]) @ head_masked


# ---------------------------------------------------------------- dense fused step
@dataclass
class DenseStepResult:
    loss: float
    recon: float
    imp: float
    y: np.ndarray
    h: np.ndarray
    g_raw: np.ndarray
    mask: np.ndarray
    u: np.ndarray
    delta: np.ndarray | None
    dV: np.ndarray
    dU: np.ndarray
    dgate: tuple
    freq: float = 0.0
    freq_ema: np.ndarray | None = None  # the EMA estimate after this step (with freq_ema given)
    freq_batch: float = 0.0  # the batch frequency penalty (the EMA's diagnostic)


def round_bf16(a):
    """Round to bfloat16 (round-to-nearest-even), returned as float64. The float64 value
    is first rounded to fp32 (as a bf16 store of an fp32 accumulator would see it);
    NaNs stay NaN."""
    a32 = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a32.view(np.uint32)
    r = (u >> np.uint32(16)) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u  # uint32 arithmetic; only NaN payloads can wrap, and they are restored below
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32).astype(np.float64)
    nan = np.isnan(a32)
    if nan.any():
        out[nan] = np.nan
    return out


def dense_site_step(x, W, V, U, gate: GateParams, draw_key, *, site_idx=0, p=2.0, imp_coeff=1.0,
                    recon_coeff=1.0, mask_dtype="bfloat16", use_delta=False, partitionable=True, bf16_storage=False,
                    imp_min=None, freq_ema=None, ema_count=0.0):
    """One stochastic-recon + importance-minimality fwd+bwd for ONE decomposed site whose
    input `x` is the clean input (the single-linear workload). It composes:
    clean target `x@W.T` (`pd/core/train.py:578-606`, detached), CI gate on `h = x@V`
    (paper form), lower/upper squashing (`pd/core/ci_fn/interface.py:35-41`), mask draw
    (`pd/core/masking.py:148-167`), `site_forward`, MSE recon and p-norm imp-min, then
    the gradients w.r.t. V, U and the gate parameters. The gate reads `h = x@V` with
    `V` live, so dV carries both the masked product's and the gate's pullback
    (`pd/core/train.py:624-655`: the CI VJP pulls back onto the prepared components).

    `bf16_storage` rounds to bf16 every tensor the reference's bf16 compute stores in
    bf16 (`pd/core/precision.py:9`; `pd/core/model.py:479-483` casts V/U to bf16, so
    `x@V`, `(x@V)*coef`, `@U` and the clean output are bf16, and their cotangents come
    back in bf16); products and reductions are exact (float64) in between. The gate
    MLP itself is evaluated exactly on the bf16 `h` — finer than the reference's bf16
    MLP arithmetic. `imp_min` (an `ImpMin`) replaces the L_p term of p / imp_coeff;
    `freq_ema` ([C], with `imp_min.ema_halflife`) is the EMA frequency estimate before
    this step after `ema_count` observations."""
    rb = round_bf16 if bf16_storage else (lambda a: a)
    spec = imp_min if imp_min is not None else ImpMin("pnorm", p=p, coeff=imp_coeff)
    y_t = rb(x @ W.T)
    h = rb(x @ V)
    g_raw = gate_forward(h, gate)
    lo = lower_leaky(g_raw)
    up = upper_leaky(g_raw)
    m, d, u = draw_site_mask(lo, draw_key, site_idx, mask_dtype, with_delta=use_delta, partitionable=partitionable)
    coef = m if d is None else m - d[:, None]
    acts = rb(h * coef)
    y = rb(acts @ U)
    y_masked = y if d is None else y + d[:, None] * y_t
    recon = mse(y_masked, y_t)
    imp, freq, dup, new_ema, freq_batch = impmin_site_terms_ema(up, spec, up.shape[0], ema=freq_ema, count=ema_count)
    loss = recon_coeff * recon + spec.loss(imp, freq)
    dy = rb(recon_coeff * 2.0 * (y_masked - y_t) / y.size)
    dU = acts.T @ dy
    da = rb(dy @ U.T)
    dh_direct = da * coef
    dlo = da * h * (1.0 - u)
    dgraw = lower_leaky_vjp(g_raw, dlo)
    dgraw = dgraw + upper_leaky_vjp(g_raw, dup)
    dh_gate, dwi, dbi, dwo, dbo = gate_backward(h, gate, dgraw)
    dV = x.T @ rb(dh_direct + dh_gate)
    return DenseStepResult(loss, recon, imp, y_masked, h, g_raw, m, u, d, dV, dU, (dwi, dbi, dwo, dbo), freq, new_ema,
                           freq_batch)


# ---------------------------------------------------------------- MoE routing
def softmax(z, axis=-1):
    z = z - z.max(axis=axis, keepdims=True)
    e = np.exp(z)
    return e / e.sum(axis=axis, keepdims=True)


def select_experts(probs, k: int):
    """`pd/targets/qwen36_moe.py:483-505`: the k most probable experts, descending,
    lowest index on ties (a stable argsort of `-probs`)."""
    order = np.argsort(-probs, axis=-1, kind="stable")
    return order[..., :k].astype(np.int32)


def expert_mixing_weights(probs, idx):
    """`pd/targets/qwen36_moe.py:508-514`: gathered probabilities renormalized over k."""
    sel = np.take_along_axis(probs, idx.astype(np.int64), axis=-1)
    return sel / sel.sum(axis=-1, keepdims=True)


@dataclass
class RoutedJobs:
    top_idx: np.ndarray
    sort_idx: np.ndarray
    inv_sort_idx: np.ndarray
    group_sizes: np.ndarray


def routed_jobs(top_idx, n_experts: int) -> RoutedJobs:
    """`pd/routed/experts.py:115-123`: stable argsort of the flat expert-of-job vector,
    its inverse permutation, and `bincount(length=E)`."""
    flat = top_idx.reshape(-1)
    sort_idx = np.argsort(flat, kind="stable").astype(np.int32)
    inv = np.argsort(sort_idx, kind="stable").astype(np.int32)
    sizes = np.bincount(flat, minlength=n_experts).astype(np.int32)
    return RoutedJobs(top_idx, sort_idx, inv, sizes)


def gather_tokens(x, jobs: RoutedJobs):
    """`pd/routed/experts.py:127-166`: `x[sort_idx // k]`."""
    k = jobs.top_idx.shape[-1]
    return x[jobs.sort_idx // k]


def gather_tokens_vjp(grad, jobs: RoutedJobs):
    """`pd/routed/experts.py:135-138`: inverse gather plus a sum over the k slots."""
    k = jobs.top_idx.shape[-1]
    return grad[jobs.inv_sort_idx].reshape(-1, k, grad.shape[-1]).sum(axis=1)


def unsort_jobs(y, jobs: RoutedJobs):
    """`pd/routed/experts.py:169-172`: `y[inv_sort_idx]` reshaped `[T, k, n]`."""
    T, k = jobs.top_idx.shape
    return y[jobs.inv_sort_idx].reshape(T, k, y.shape[-1])


def sort_jobs(values, jobs: RoutedJobs):
    """`pd/routed/experts.py:175-178`."""
    return values.reshape(-1)[jobs.sort_idx]


def sort_job_values(values, jobs: RoutedJobs):
    """`pd/routed/experts.py:192-199`: `[T, k, n]` rows in expert-sorted job order."""
    T, k = jobs.top_idx.shape
    return values.reshape(T * k, -1)[jobs.sort_idx]


def sum_jobs(y, jobs: RoutedJobs):
    """`pd/routed/experts.py:202-206`: fp32 sum over each token's k job rows."""
    return unsort_jobs(y, jobs).sum(axis=1)


def combine_jobs(y, jobs: RoutedJobs, weights):
    """`pd/routed/experts.py:351-359`: routing-weighted fp32 sum over the k job rows."""
    return (unsort_jobs(y, jobs) * weights[..., None]).sum(axis=1)


def grouped_matmul(lhs, rhs, group_sizes):
    """`pd/routed/experts.py:326-348` (`jax.lax.ragged_dot` semantics): the e-th
    contiguous `group_sizes[e]`-row block of `lhs` times `rhs[e]`. Rows beyond
    `sum(group_sizes)` are zero."""
    out = np.zeros((lhs.shape[0], rhs.shape[-1]), dtype=np.float64)
    start = 0
    for e, n in enumerate(group_sizes):
        n = int(n)
        out[start:start + n] = lhs[start:start + n] @ rhs[e]
        start += n
    return out


def transposed_grouped_matmul(lhs, dout, group_sizes):
    """`pd/routed/experts.py:209-280`: `out[e] = lhs[block_e].T @ dout[block_e]`; empty
    groups are exactly zero."""
    E = len(group_sizes)
    out = np.zeros((E, lhs.shape[1], dout.shape[1]), dtype=np.float64)
    start = 0
    for e, n in enumerate(group_sizes):
        n = int(n)
        if n:
            out[e] = lhs[start:start + n].T @ dout[start:start + n]
        start += n
    return out


def fold_routing_weights(gate, up, weights):
    """`pd/targets/qwen36_moe.py:2272-2282`: `silu(gate) * up * weight` in fp32."""
    return gate / (1.0 + np.exp(-gate)) * up * weights


def routed_decomposed_site(x_jobs, V, U, group_sizes, mask_jobs, delta_jobs=None, frozen=None):
    """One decomposed expert site in job space, `pd/targets/qwen36_moe.py:2790-2818`:
    `acts = gmm(x_jobs, V) * (mask - delta)`; `out = gmm(acts, U) [+ delta*gmm(x, W)]`.
    V is `[E, d_in, c]`, U is `[E, c, d_out]`, mask_jobs `[J, c]`, delta_jobs `[J]`."""
    h = grouped_matmul(x_jobs, V, group_sizes)
    coef = mask_jobs if delta_jobs is None else mask_jobs - delta_jobs[:, None]
    acts = h * coef
    out = grouped_matmul(acts, U, group_sizes)
    if delta_jobs is not None:
        out = out + delta_jobs[:, None] * grouped_matmul(x_jobs, frozen, group_sizes)
    return out, h


# ---------------------------------------------------------------- routing samplers
def uniform_k_routing(key, n_sites: int, leading_shape, *, partitionable: bool = True) -> np.ndarray:
    """`UniformKRouting.__call__` (`param_decomp/param_decomp/core/recon.py:218-231`):
    `k_key, perm_key = split(key)`; `k = randint(k_key, shape, 1, n_sites + 1)`;
    `perms = argsort(uniform(perm_key, (n_sites, *shape)), axis=0)` (stable);
    `routed[j] = perms[j] < k`. Returns bool `[n_sites, *shape]`."""
    k_key, perm_key = threefry.split(key, partitionable=partitionable)
    shape = tuple(int(s) for s in leading_shape)
    k = threefry.randint(k_key, shape, 1, n_sites + 1, partitionable=partitionable)
    u = threefry.uniform(perm_key, (n_sites, *shape), "float32", partitionable=partitionable)
    perms = np.argsort(u, axis=0, kind="stable")
    return perms < k[None]


def static_probability_routing(key, n_sites: int, p: float, leading_shape, *, partitionable: bool = True) -> np.ndarray:
    """`StaticProbabilityRouting.__call__` (`core/recon.py:233-244`):
    `routed[j] = bernoulli(fold_in(key, j), p, shape)` = `uniform_f32 < float32(p)`."""
    shape = tuple(int(s) for s in leading_shape)
    p32 = float(np.float32(p))
    return np.stack([threefry.uniform(threefry.fold_in(key, j), shape, "float32", partitionable=partitionable) < p32
                     for j in range(n_sites)])
