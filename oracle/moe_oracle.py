"""NumPy restatement of the decomposed MoE stack step (oracle only; float64 arithmetic).

The stack is the reference's MoE layer with every routed expert matrix decomposed,
mixers and the shared expert excluded: per layer
`h2 = rms_norm_zero_centered(r)` (`param_decomp/param_decomp/target_ports/qwen3_5_moe.py:33-41`),
router softmax over the router product rounded to the bf16 matmul dtype and widened
(`router_logits`, `pd/targets/qwen36_moe.py:473-475`; the rounding applies with
`bf16_storage`), top-k (`:483-514`), jobs schedule
(`pd/routed/experts.py:115-123`), decomposed expert sites in job space
(`pd/targets/qwen36_moe.py:2752-2837`: `acts = gmm(x_jobs, V) * mask_jobs`,
`out = gmm(acts, U)`, routing weights folded into the down input in fp32,
`_fold_routing_weights` `:2272-2282`, unweighted `sum_jobs`), `r += routed`. The clean
forward runs the frozen expert weights with the weights applied to the down output in
the fp32 combine (`combine_jobs`, `pd/routed/experts.py:351-359`) and pins the masked
pass's expert indices (`_moe_forward`, `pd/targets/qwen36_moe.py:2923-2965`). Masks are
drawn per (kind, layer) from `fold_in(fold_in(split(draw_key)[0], kind_index), layer)`
(`pd/targets/qwen36_moe.py:3374-3401`) over the selected-CI values `[T, k*c]`
(`SelectedCI`, `pd/core/components.py:81-114`). The stochastic recipe also draws the
frozen delta channel (`_entry_masking`, `pd/targets/qwen36_moe.py:2151-2160`): a
per-token `d = uniform(fold_in(fold_in(split(draw_key)[1], kind_index), layer), [T])`
in the CI dtype (`sample_delta_mask`, `pd/core/masking.py:139-140`), component
coefficients `m - d` and site output `gmm(acts, U) + d * gmm(x_jobs, W[e])`
(`pd/targets/qwen36_moe.py:2805-2815`, `pd/core/decomposed_linear.py:65-85`);
`use_delta=False` is `d = 0`. `source_value=v` replaces the draws by the reference's
`ConstantSources(v)` (`pd/core/objective.py:435-449`): `u = v` everywhere and `d = v`
(`_constant_delta_mask`, `pd/core/masking.py:143-145`); `v = 0` is the CI-masked
reconstruction. Loss: MSE between the masked and clean final residual
streams plus the L_p imp-min over the selected upper CI values
(`pd/core/losses.py:357-372` selected arm).

`bf16_storage=True` rounds to bf16 exactly the tensors the GPU step stores in bf16;
everything between is float64. Without source tables the GPU step forms each frozen
product inside its site's second product (one accumulation, `out = rb(acts @ U + bl
frozen)`; gate and up of layer 0 take the clean pass's stored product instead), so the
frozen product is stored, and rounded, only on the source-table path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from oracle import pd_oracle as po
from oracle import threefry as tf

KIND_INDEX = {"gate": 11, "up": 12, "down": 13}
SITES = ("gate", "up", "down")


@dataclass
class MoEConfig:
    T: int
    d: int
    f: int
    E: int
    k: int
    c: int
    L: int
    eps: float = 1e-6


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    return x * sigmoid(x)


def silu_grad(x):
    s = sigmoid(x)
    return s * (1.0 + x * (1.0 - s))


def rms_norm_zero_centered(x, w, eps):
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * (1.0 + w), r


def rms_norm_vjp(x, w, r, dy):
    a = (1.0 + w) * dy
    d = x.shape[-1]
    return r * a - x * r**3 * np.sum(a * x, axis=-1, keepdims=True) / d


def site_mask_keys(draw_key, layer, partitionable=True):
    src_base, _ = tf.split(draw_key, partitionable=partitionable)
    return {s: tf.fold_in(tf.fold_in(src_base, KIND_INDEX[s]), layer) for s in SITES}


def site_delta_keys(draw_key, layer, partitionable=True):
    _, delta_base = tf.split(draw_key, partitionable=partitionable)
    return {s: tf.fold_in(tf.fold_in(delta_base, KIND_INDEX[s]), layer) for s in SITES}


def grouped_T(lhs, rhs, sizes):
    """`lhs[rows_e] @ rhs[e].T` (the grouped matmul's d_input product)."""
    return po.grouped_matmul(lhs, np.transpose(rhs, (0, 2, 1)), sizes)


def moe_stack_step(cfg: MoEConfig, params, x0, ci_pre, draw_key, *, p=2.0, imp_coeff=1.0, recon_coeff=1.0,
                   bf16_storage=False, partitionable=True, use_delta=True, deltas=None, source_value=None,
                   pinned_top_idx=None, imp_min=None, sources=None, freq_ema=None, ema_count=0.0, routes=None):
    """params: list over layers of dicts {ln, router, Wg, Wu, Wd, Vg, Ug, Vu, Uu, Vd, Ud};
    ci_pre[l][site]: [T, k, c]. `deltas[l][site]` ([T]) replaces the drawn delta when
    given. `pinned_top_idx[l]` ([T, k]) replaces the clean pass's own expert selection
    (which is still computed and returned as `own_top_idx`, with the clean pass's router
    products before rounding, `logits_raw`, and the sums of their terms' magnitudes,
    `logits_mag`, that bound an fp32 accumulation's error). Returns dict(loss, recon,
    imp, grads, d_ci_pre, top_idx, own_top_idx, logits_raw, logits_mag, r_final,
    rc_final, deltas). `imp_min` (a `pd_oracle.ImpMin`) replaces the L_p term given by
    p / imp_coeff; each site's selected values map to their expert's block of the
    [E * c] component vector; `freq` is the frequency term. `freq_ema` ([L, 3, E * c],
    with `imp_min.ema_halflife`) is the EMA frequency estimate before this step after
    `ema_count` observations: the frequency term then reads the debiased estimate, and the
    result holds the new estimate (`freq_ema`) and the batch penalty (`freq_batch`).
    `routes[l][site]` ([T] bool) routes the recon term per token: an unrouted token's jobs
    take the frozen output, `where(route, decomposed + d frozen, frozen)`
    (`pd/targets/qwen36_moe.py:2822-2827`).

    `sources = (src, src_delta, rows_per_source)` replaces the draws by persistent
    (adversarial) source tables, the reference's `SourceMaskIngredients` arm
    (`pd/targets/qwen36_moe.py:2151-2163`, `pd/core/source_mask.py:56-63`,
    `pd/core/masking.py:43-68`): src[l][site] [S, E, c], src_delta[l][site] [S], every
    source row covering rows_per_source consecutive tokens (S = T / rows_per_source: the
    `c`, `bc` and `bsc` shapes). A selected value reads its expert's row,
    m = lower + (1 - lower) src[t // rps, idx[t, slot], :], and the site's delta is
    src_delta[t // rps]. The result then also holds the source gradients d_src[l][site]
    (scatter of dm (1 - lower) into [S, E, c]) and d_src_delta[l][site] [S] (the delta
    cotangent sum_o g_out frozen - sum_c dm of every job, summed over each source row's
    tokens)."""
    rb = po.round_bf16 if bf16_storage else (lambda a: a)
    fused = sources is None  # frozen products accumulate with their site's product (see above)
    spec = imp_min if imp_min is not None else po.ImpMin("pnorm", p=p, coeff=imp_coeff)
    T, k, c, E = cfg.T, cfg.k, cfg.c, cfg.E
    # ---------------- clean forward (frozen weights)
    rc = rb(x0)
    tops, own_tops, raws, mags = [], [], [], []
    for l in range(cfg.L):
        P = params[l]
        h2c, _ = rms_norm_zero_centered(rc, P["ln"], cfg.eps)
        h2c = rb(h2c)
        raw = h2c @ P["router"].T
        raws.append(raw)
        mags.append(np.abs(h2c) @ np.abs(P["router"]).T)
        probs = po.softmax(rb(raw))
        own_tops.append(po.select_experts(probs, k))
        idx = own_tops[-1] if pinned_top_idx is None else np.asarray(pinned_top_idx[l]).astype(own_tops[-1].dtype)
        w = po.expert_mixing_weights(probs, idx)
        jobs = po.routed_jobs(idx, E)
        xj = h2c[jobs.sort_idx // k]
        g = rb(po.grouped_matmul(xj, P["Wg"], jobs.group_sizes))
        u = rb(po.grouped_matmul(xj, P["Wu"], jobs.group_sizes))
        din = rb(silu(g) * u)
        down = rb(po.grouped_matmul(din, P["Wd"], jobs.group_sizes))
        routed = rb(po.combine_jobs(down, jobs, w))
        rc = rb(rc + routed)
        tops.append(idx)
    # ---------------- masked forward (pinned indices)
    r = rb(x0)
    saved = []
    imp = 0.0
    freq = 0.0
    freq_batch = 0.0
    new_ema = None if freq_ema is None else np.zeros((cfg.L, len(SITES), E * c))
    for l in range(cfg.L):
        P = params[l]
        h2, rinv = rms_norm_zero_centered(r, P["ln"], cfg.eps)
        h2 = rb(h2)
        probs = po.softmax(rb(h2 @ P["router"].T))
        idx = tops[l]
        w = po.expert_mixing_weights(probs, idx)
        jobs = po.routed_jobs(idx, E)
        keys = site_mask_keys(draw_key, l, partitionable)
        dkeys = site_delta_keys(draw_key, l, partitionable)
        xj = h2[jobs.sort_idx // k]
        tok = jobs.sort_idx // k
        S = {}
        for s in SITES:
            pre = ci_pre[l][s]
            lo = po.lower_leaky(pre)
            up = po.upper_leaky(pre)
            si = SITES.index(s)
            a_, f_, dup, ne, fb = po.impmin_site_terms_ema(
                up, spec, T, idx, E, ema=None if freq_ema is None else np.asarray(freq_ema)[l, si], count=ema_count)
            imp += a_
            freq += f_
            freq_batch += fb
            if new_ema is not None:
                new_ema[l, si] = ne
            if sources is not None:
                src_t, src_d, rps = sources
                # the table is cast to the CI dtype before the select (pd/core/masking.py:57)
                ut = rb(np.asarray(src_t[l][s], np.float64))[(np.arange(T) // rps)[:, None], idx.astype(np.int64)]
            elif source_value is None:
                ut = tf.uniform(keys[s], (T, k * c), "bfloat16", partitionable=partitionable).reshape(T, k, c)
            else:
                ut = np.full((T, k, c), float(source_value))
            m_tok = lo + (1.0 - lo) * ut
            if sources is not None:
                dt = rb(np.asarray(sources[1][l][s], np.float64))[np.arange(T) // sources[2]]
            elif deltas is not None:
                dt = np.asarray(deltas[l][s], np.float64)
            elif use_delta and source_value is not None:
                dt = np.full(T, float(source_value))
            elif use_delta:
                dt = tf.uniform(dkeys[s], (T,), "bfloat16", partitionable=partitionable)
            else:
                dt = np.zeros(T)
            dj = dt[tok][:, None]
            rj = np.ones((T * k, 1)) if routes is None else np.asarray(routes[l][s], bool)[tok][:, None].astype(float)
            S[s] = dict(pre=pre, lo=lo, up=up, dup=dup, u=ut, m=m_tok.reshape(T * k, c)[jobs.sort_idx], delta=dt,
                        dj=dj, rj=rj, bl=np.where(rj > 0, dj, 1.0))
            S[s]["coef"] = (S[s]["m"] - dj) * rj
        wj = w.reshape(-1)[jobs.sort_idx]
        for s in ("gate", "up"):
            S[s]["h"] = rb(po.grouped_matmul(xj, P["V" + s[0]], jobs.group_sizes))
            S[s]["acts"] = rb(S[s]["h"] * S[s]["coef"])
            raw = po.grouped_matmul(xj, P["W" + s[0]], jobs.group_sizes)
            frozen = rb(raw)
            S[s]["frozen"] = frozen
            prod = po.grouped_matmul(S[s]["acts"], P["U" + s[0]], jobs.group_sizes)
            if fused and l > 0:
                S[s]["out"] = rb(prod + S[s]["bl"] * raw)
            else:
                S[s]["out"] = rb(rb(prod) + S[s]["bl"] * frozen)
        gq, uq = S["gate"]["out"], S["up"]["out"]
        din = rb(silu(gq) * uq * wj[:, None])
        S["down"]["h"] = rb(po.grouped_matmul(din, P["Vd"], jobs.group_sizes))
        S["down"]["acts"] = rb(S["down"]["h"] * S["down"]["coef"])
        raw = po.grouped_matmul(din, P["Wd"], jobs.group_sizes)
        S["down"]["frozen"] = rb(raw)
        prod = po.grouped_matmul(S["down"]["acts"], P["Ud"], jobs.group_sizes)
        if fused:
            dout = rb(prod + S["down"]["bl"] * raw)
        else:
            dout = rb(prod) + S["down"]["bl"] * S["down"]["frozen"]
        routed = rb(po.sum_jobs(dout, jobs))
        saved.append(dict(r=r, rinv=rinv, h2=h2, probs=probs, w=w, wj=wj, jobs=jobs, xj=xj, S=S, din=din, idx=idx))
        r = rb(r + routed)
    n = T * cfg.d
    recon = float(np.mean((r - rc) ** 2))
    loss = recon_coeff * recon + spec.loss(imp, freq)
    # ---------------- backward
    dr = rb(recon_coeff * 2.0 * (r - rc) / n)
    grads = [dict() for _ in range(cfg.L)]
    d_pre = [dict() for _ in range(cfg.L)]
    d_src = [dict() for _ in range(cfg.L)]
    d_src_delta = [dict() for _ in range(cfg.L)]
    for l in reversed(range(cfg.L)):
        P, sv = params[l], saved[l]
        jobs, S = sv["jobs"], sv["S"]
        sizes = jobs.group_sizes
        d_dout = dr[jobs.sort_idx // k]
        # down site
        Sd = S["down"]
        Sd["gout"] = d_dout
        d_acts = rb(grouped_T(d_dout, P["Ud"], sizes))
        grads[l]["Ud"] = po.transposed_grouped_matmul(Sd["acts"], d_dout, sizes)
        Sd["dm"] = d_acts * Sd["h"] * Sd["rj"]
        d_h = rb(d_acts * Sd["coef"])
        grads[l]["Vd"] = po.transposed_grouped_matmul(sv["din"], d_h, sizes)
        if fused:
            d_din = rb(grouped_T(d_h, P["Vd"], sizes) + Sd["bl"] * grouped_T(d_dout, P["Wd"], sizes))
        else:
            d_din = rb(grouped_T(d_h, P["Vd"], sizes)) + Sd["bl"] * rb(grouped_T(d_dout, P["Wd"], sizes))
        # SwiGLU fold
        gq, uq, wj = S["gate"]["out"], S["up"]["out"], sv["wj"]
        sg = silu(gq)
        d_g = rb(d_din * uq * wj[:, None] * silu_grad(gq))
        d_u = rb(d_din * sg * wj[:, None])
        d_wj = np.sum(d_din * sg * uq, axis=-1)
        d_xj = np.zeros_like(sv["xj"])
        for s, dgo in (("gate", d_g), ("up", d_u)):
            Ss = S[s]
            Ss["gout"] = dgo
            d_acts = rb(grouped_T(dgo, P["U" + s[0]], sizes))
            grads[l]["U" + s[0]] = po.transposed_grouped_matmul(Ss["acts"], dgo, sizes)
            Ss["dm"] = d_acts * Ss["h"] * Ss["rj"]
            d_h = rb(d_acts * Ss["coef"])
            grads[l]["V" + s[0]] = po.transposed_grouped_matmul(sv["xj"], d_h, sizes)
            if fused:
                d_xj = d_xj + rb(grouped_T(d_h, P["V" + s[0]], sizes) + Ss["bl"] * grouped_T(dgo, P["W" + s[0]], sizes))
            else:
                d_xj = (d_xj + rb(grouped_T(d_h, P["V" + s[0]], sizes))
                        + Ss["bl"] * rb(grouped_T(dgo, P["W" + s[0]], sizes)))
        # mask pullback to the CI preactivations (token-major)
        for s in SITES:
            Ss = S[s]
            dm_tok = np.zeros((T * k, c))
            dm_tok[jobs.sort_idx] = Ss["dm"]
            dm_tok = dm_tok.reshape(T, k, c)
            dlo = dm_tok * (1.0 - Ss["u"])
            d_pre[l][s] = rb(po.lower_leaky_vjp(Ss["pre"], dlo) + po.upper_leaky_vjp(Ss["pre"], Ss["dup"]))
            if sources is not None:
                rps = sources[2]
                Sn = T // rps
                ds = np.zeros((Sn, E, c))
                np.add.at(ds, ((np.arange(T) // rps)[:, None], sv["idx"].astype(np.int64)),
                          dm_tok * (1.0 - Ss["lo"]))
                d_src[l][s] = ds
                # the delta cotangent per job (d enters as acts = h (m - d) and + d frozen)
                qj = np.sum(Ss["gout"] * Ss["frozen"], axis=-1) - np.sum(Ss["dm"], axis=-1)
                d_tok = np.zeros(T)
                np.add.at(d_tok, jobs.sort_idx // k, qj)
                d_src_delta[l][s] = d_tok.reshape(Sn, rps).sum(axis=1)
        # routing weights -> probs -> logits -> h2
        d_w = d_wj[jobs.inv_sort_idx].reshape(T, k)
        w, probs, idx = sv["w"], sv["probs"], sv["idx"]
        Ssum = np.take_along_axis(probs, idx.astype(np.int64), axis=-1).sum(-1, keepdims=True)
        d_psel = (d_w - np.sum(d_w * w, axis=-1, keepdims=True)) / Ssum
        d_probs = np.zeros_like(probs)
        np.put_along_axis(d_probs, idx.astype(np.int64), d_psel, axis=-1)
        d_logits = rb(probs * (d_probs - np.sum(probs * d_probs, axis=-1, keepdims=True)))
        d_h2 = po.gather_tokens_vjp(d_xj, jobs) + d_logits @ P["router"]
        dx = rms_norm_vjp(sv["r"], P["ln"], sv["rinv"], d_h2)
        dr = rb(dr + dx)
    return dict(loss=loss, recon=recon, imp=imp, freq=freq, freq_ema=new_ema, freq_batch=freq_batch, grads=grads,
                d_ci_pre=d_pre, top_idx=tops, d_src=d_src, d_src_delta=d_src_delta, own_top_idx=own_tops,
                logits_raw=raws, logits_mag=mags, r_final=r, rc_final=rc, dx0=dr,
                deltas=[{s: sv["S"][s]["delta"] for s in SITES} for sv in saved])


def selection_within_ulps(raw, got, k, n_ulp=1):
    """True when the expert selection `got` ([k]) is the descending top-k, lowest index
    on ties, of SOME logits within `n_ulp` bf16 ulps of the bf16-rounded router products
    `raw` ([E]). Two products with the same exact value can round to adjacent bf16 values
    when their fp32 accumulation orders (or a bf16 input one step upstream) differ, so a
    selection from another correct implementation may differ from this oracle's exactly
    where two logits are that close."""
    r = po.round_bf16(np.asarray(raw, np.float64))
    ulp = np.abs(r) * 2.0**-7
    got = [int(e) for e in got]
    if len(set(got)) != k:
        return False
    lo, hi = r - n_ulp * ulp, r + n_ulp * ulp
    tiny = 1e-12

    def lift(e, floor, floor_idx):
        """Smallest admissible value of expert e ranked above a value `floor` held by
        expert floor_idx (equal values rank the lower index first), or None."""
        z = max(lo[e], floor)
        if z == floor and floor_idx is not None and e > floor_idx:
            z = floor + tiny
        return z if z <= hi[e] else None

    # the selected values must all stay at or above every unselected expert's lowest value
    rest = [e for e in range(len(r)) if e not in got]
    z, z_idx = -np.inf, None
    for e in sorted(rest, key=lambda e: (lo[e], -e)):
        z, z_idx = lo[e], e  # the binding constraint: the largest lower bound (lowest index on equal)
    for e in reversed(got):  # then each selected expert above the next one down
        zz = lift(e, z, z_idx)
        if zz is None:
            return False
        z, z_idx = zz, e
    return True


def init_moe(cfg: MoEConfig, rng):
    """Random target and components of the stated shapes (the step's synthetic setup).
    V scales by its per-block fan-in and each block's U by the site's C = E*c
    (`BLOCKED_U_INIT_FAN_IN = "site"`, `pd/core/components.py:639-677`)."""
    d, f, E, c = cfg.d, cfg.f, cfg.E, cfg.c

    def rn(*shape, scale=1.0):
        return rng.standard_normal(size=shape, dtype=np.float32).astype(np.float64) * scale

    params = []
    for _ in range(cfg.L):
        P = dict(ln=rn(d, scale=0.1), router=rn(E, d, scale=d**-0.5),
                 Wg=rn(E, d, f, scale=d**-0.5), Wu=rn(E, d, f, scale=d**-0.5), Wd=rn(E, f, d, scale=f**-0.5),
                 Vg=rn(E, d, c, scale=d**-0.5), Ug=rn(E, c, f, scale=(E * c)**-0.5),
                 Vu=rn(E, d, c, scale=d**-0.5), Uu=rn(E, c, f, scale=(E * c)**-0.5),
                 Vd=rn(E, f, c, scale=f**-0.5), Ud=rn(E, c, d, scale=(E * c)**-0.5))
        params.append(P)
    x0 = rn(cfg.T, d)
    ci = [{s: rng.uniform(-0.3, 1.3, size=(cfg.T, cfg.k, c)) for s in SITES} for _ in range(cfg.L)]
    return params, x0, ci


def moe_stack_step_torch(cfg: MoEConfig, params, x0, ci_pre, draw_key, *, p=2.0, imp_coeff=1.0, recon_coeff=1.0,
                         use_delta=True, partitionable=True, dtype=None, threads=None, imp_min=None,
                         sources=None, freq_ema=None, ema_count=0.0, routes=None):
    """The same step as `moe_stack_step` (no bf16 storage model) written as a torch
    forward whose backward is torch autograd: in float64 it pins `moe_stack_step`'s
    hand-written backward (tests/test_moe_oracle.py). The expert selection and Threefry
    draws are computed as in `moe_stack_step` (integer and bit-level work, outside
    autograd). The smooth-L0 imp-min (`imp_min`) is written as the reference writes it, a
    scatter-add of psi into the [E, c] component frequencies, so autograd differentiates
    the frequency penalty through the scatter; with `freq_ema` ([L, 3, E * c]) the
    penalty is the reference's EMA surrogate `Phi(f_hat) + Phi'(f_hat) (f - sg(f))`
    (`pd/core/losses.py:449-456`). Returns dict(loss, recon, imp, freq, grads, d_ci_pre,
    top_idx)."""
    import torch

    spec = imp_min if imp_min is not None else po.ImpMin("pnorm", p=p, coeff=imp_coeff)

    if threads:
        torch.set_num_threads(threads)
    dt = dtype or torch.float64
    T, k, c, E = cfg.T, cfg.k, cfg.c, cfg.E
    t = lambda a, g=False: torch.tensor(np.asarray(a, np.float64), dtype=dt, requires_grad=g)  # noqa: E731

    def norm(x, w):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + cfg.eps) * (1.0 + w)

    def gmm(lhs, rhs, offs):
        return torch.cat([lhs[offs[e]:offs[e + 1]] @ rhs[e] for e in range(E)], 0)

    P = [{n: t(v, n[0] in "VU") for n, v in layer.items()} for layer in params]
    pre = [{s: t(ci_pre[l][s], True) for s in SITES} for l in range(cfg.L)]
    if sources is not None:  # persistent source tables as autograd leaves
        src = [{s: t(sources[0][l][s], True) for s in SITES} for l in range(cfg.L)]
        srcd = [{s: t(sources[1][l][s], True) for s in SITES} for l in range(cfg.L)]
        rps = sources[2]
        doc = torch.as_tensor(np.arange(T) // rps, dtype=torch.long)
    # clean pass: the expert selection (no gradient)
    with torch.no_grad():
        rc = t(x0)
        tops = []
        for l in range(cfg.L):
            h2 = norm(rc, P[l]["ln"])
            probs = torch.softmax(h2 @ P[l]["router"].T, -1)
            idx = po.select_experts(probs.double().numpy(), k)
            tops.append(idx)
            jobs = po.routed_jobs(idx, E)
            offs = np.concatenate([[0], np.cumsum(jobs.group_sizes)]).tolist()
            xj = h2[torch.as_tensor(jobs.sort_idx // k, dtype=torch.long)]
            din = torch.nn.functional.silu(gmm(xj, P[l]["Wg"], offs)) * gmm(xj, P[l]["Wu"], offs)
            down = gmm(din, P[l]["Wd"], offs)
            w = torch.gather(probs, 1, torch.as_tensor(idx, dtype=torch.long))
            w = w / w.sum(-1, keepdim=True)
            inv = torch.as_tensor(jobs.inv_sort_idx, dtype=torch.long)
            rc = rc + (down[inv].reshape(T, k, -1) * w[..., None]).sum(1)
    r = t(x0)
    imp = 0.0
    freq = 0.0
    for l in range(cfg.L):
        h2 = norm(r, P[l]["ln"])
        probs = torch.softmax(h2 @ P[l]["router"].T, -1)
        idx = torch.as_tensor(tops[l], dtype=torch.long)
        w = torch.gather(probs, 1, idx)
        w = w / w.sum(-1, keepdim=True)
        jobs = po.routed_jobs(tops[l], E)
        offs = np.concatenate([[0], np.cumsum(jobs.group_sizes)]).tolist()
        sidx = torch.as_tensor(jobs.sort_idx, dtype=torch.long)
        tok = sidx // k
        xj = h2[tok]
        keys, dkeys = site_mask_keys(draw_key, l, partitionable), site_delta_keys(draw_key, l, partitionable)
        coef = {}
        for s in SITES:
            lo = pre[l][s].clamp(0.0, 1.0)  # forward of the lower leaky hard sigmoid
            up = torch.where(pre[l][s] > 1.0, 1.0 + 0.01 * (pre[l][s] - 1.0), pre[l][s].clamp(0.0, 1.0))
            if spec.kind == "pnorm":
                imp = imp + (up**spec.p).sum() / T
            else:
                g2 = spec.gamma**2
                psi = up**2 / (up**2 + g2) * ((1.0 + g2) if spec.normalize_at_one else 1.0)
                F = torch.zeros(E, c, dtype=dt).index_add(0, idx.reshape(-1), psi.reshape(-1, c))
                fr = F / T
                imp = imp + fr.sum()
                if spec.ref_count > 0 and freq_ema is None:
                    freq = freq + (fr * torch.log2(1.0 + spec.ref_count * fr)).sum()
                elif spec.ref_count > 0:
                    alpha, debias = po.ema_decay_terms(ema_count, spec.ema_halflife)
                    f_sg = fr.detach().reshape(-1)
                    prev = t(np.asarray(freq_ema)[l, SITES.index(s)])
                    f_hat = (prev + alpha * (f_sg - prev)) / debias
                    a_ = spec.ref_count
                    slope = torch.log2(1.0 + a_ * f_hat) + a_ * f_hat / ((1.0 + a_ * f_hat) * math.log(2.0))
                    freq = freq + (f_hat * torch.log2(1.0 + a_ * f_hat) + slope * (fr.reshape(-1) - f_sg)).sum()
            if sources is not None:
                u = src[l][s][doc[:, None], idx]
                dlt = srcd[l][s][doc]
            else:
                u = t(tf.uniform(keys[s], (T, k * c), "bfloat16", partitionable=partitionable).reshape(T, k, c))
                dlt = (t(tf.uniform(dkeys[s], (T,), "bfloat16", partitionable=partitionable)) if use_delta
                       else torch.zeros(T, dtype=dt))
            m = (lo + (1.0 - lo) * u).reshape(T * k, c)[sidx]
            if routes is None:
                coef[s] = (m - dlt[tok][:, None], dlt[tok][:, None])
            else:  # unrouted tokens: the frozen output alone
                rj = torch.as_tensor(np.asarray(routes[l][s], bool))[tok][:, None]
                coef[s] = ((m - dlt[tok][:, None]) * rj, torch.where(rj, dlt[tok][:, None], torch.ones((), dtype=dt)))
        wj = w.reshape(-1)[sidx]
        out = {}
        for s in ("gate", "up"):
            acts = gmm(xj, P[l]["V" + s[0]], offs) * coef[s][0]
            out[s] = gmm(acts, P[l]["U" + s[0]], offs) + coef[s][1] * gmm(xj, P[l]["W" + s[0]], offs)
        din = torch.nn.functional.silu(out["gate"]) * out["up"] * wj[:, None]
        acts = gmm(din, P[l]["Vd"], offs) * coef["down"][0]
        dout = gmm(acts, P[l]["Ud"], offs) + coef["down"][1] * gmm(din, P[l]["Wd"], offs)
        inv = torch.as_tensor(jobs.inv_sort_idx, dtype=torch.long)
        r = r + dout[inv].reshape(T, k, -1).sum(1)
    recon = ((r - rc) ** 2).mean()
    loss = recon_coeff * recon + spec.coeff * imp + (spec.freq_coeff * freq if spec.kind == "smooth_l0" else 0.0)
    names = [(l, n) for l in range(cfg.L) for n in ("Vg", "Ug", "Vu", "Uu", "Vd", "Ud")]
    wrt = [P[l][n] for l, n in names] + [pre[l][s] for l in range(cfg.L) for s in SITES]
    if sources is not None:
        wrt += [src[l][s] for l in range(cfg.L) for s in SITES] + [srcd[l][s] for l in range(cfg.L) for s in SITES]
    g = torch.autograd.grad(loss, wrt)
    grads = [dict() for _ in range(cfg.L)]
    for (l, n), v in zip(names, g[:len(names)]):
        grads[l][n] = v.double().numpy()
    d_ci = [dict() for _ in range(cfg.L)]
    d_src = [dict() for _ in range(cfg.L)]
    d_srcd = [dict() for _ in range(cfg.L)]
    nls = cfg.L * len(SITES)
    for i, (l, s) in enumerate((l, s) for l in range(cfg.L) for s in SITES):
        d_ci[l][s] = g[len(names) + i].double().numpy()
        if sources is not None:
            d_src[l][s] = g[len(names) + nls + i].double().numpy()
            d_srcd[l][s] = g[len(names) + 2 * nls + i].double().numpy()
    return dict(loss=float(loss.detach()), recon=float(recon.detach()), imp=float(imp.detach()),
                freq=float(freq.detach()) if torch.is_tensor(freq) else freq, grads=grads, d_ci_pre=d_ci, top_idx=tops,
                d_src=d_src, d_src_delta=d_srcd)
