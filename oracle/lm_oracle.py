"""Torch-float64 (CPU) restatement of the decomposed Llama-style LM step (oracle only:
test infrastructure and the CPU baseline's checker, never the product path).

Paths are relative to the reference root; `pd/` = `param_decomp/param_decomp/`.

The target is the pre-RMSNorm transformer of `pd/targets/transformer.py:1031-1140`
(`_run_transformer_block`): per layer
    h = rms_norm(r, ln1); q, k, v = site(h); a = causal_attention(rope(q), rope(k), v)
    r = r + site_o(a); h2 = rms_norm(r, ln2)
    plain MLP (LlamaSimpleMLP, `pd/targets/llama_simple_mlp.py`): r = r + site_down(gelu_tanh(site_fc(h2)))
    GLU MLP (Llama/Qwen):                                         r = r + site_down(silu(site_gate(h2)) * site_up(h2))
then `rms_norm(r, norm)` and the (tied) head. Pieces:
- `rms_norm`: `pd/target_ports/llama.py:90-97` (weight * (x * rsqrt(mean x^2 + eps)));
- RoPE: rotate-half with `inv_freq = base^(-2i/hd)` (`pd/targets/llama_simple_mlp.py:127-132`,
  `pd/target_ports/llama.py:100-117`), positions 0..T-1;
- attention: causal SDPA with GQA head repeat and scale hd^-1/2
  (`pd/targets/transformer.py:701-747`, `pd/target_ports/llama.py:120-125`);
- GELU: tanh approximation (`pd/targets/transformer.py:802-805`);
- a decomposed site: `((x@V) * (m - d)) @ U + d * (x @ W^T)` (`pd/core/decomposed_linear.py:142-175`);
- stochastic masks drawn in-block: `m = ci + (1 - ci) * uniform(k_m, ci)`,
  `d = uniform(k_d, ci[..., 0])` with `k_m = fold_in(fold_in(split(draw_key)[0], kind), layer)`
  and `k_d` the same over `split(draw_key)[1]` (`pd/targets/transformer.py:1048-1058, 1424-1451`),
  drawn in bf16 over each site's `[B*T, C]` CI;
- KL(clean || masked) per position, averaged (`pd/targets/losses.py:50-60`, streamed form
  `:102-163` equal to it), clean side held fixed;
- imp-min: the L_p form over the upper-leaky CI, `sum_sites sum_c mean_tokens upper^p`.

Gradients come from torch autograd in float64. With `bf16_storage=True` every tensor the
GPU step stores in bf16 is rounded to bf16 in the forward, and its cotangent is rounded to
bf16 in the backward (a bf16 value's cotangent is bf16 in the reference's arithmetic); all
else is float64.

Pinned by (tests/test_lm_oracle.py): the reference's frozen LlamaSimpleMLP logits fixture
(`pd/tests/targets/simple_mlp_equivalence/tiny_fixture.npz`: RoPE, GQA, causal attention,
GELU-tanh, norms, tied head; fp32 max-abs 1e-5), the reference's frozen PPGD loss golden
(`pd/tests/targets/equivalence/fixtures.npz` with `torch_reference.json`: masked GLU sites
with the weight-delta channel, source masks, final norm, head and KL; RTOL 2e-4 / ATOL
1e-5), attention against torch's `scaled_dot_product_attention`, RoPE's relative-position
invariance, and finite differences of the float64 step.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from oracle import pd_oracle as po
from oracle import threefry as tf

F64 = torch.float64
PLAIN_KINDS = ("q_proj", "k_proj", "v_proj", "o_proj", "c_fc", "down_proj")  # llama_simple_mlp KIND_ORDER
GLU_KINDS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass
class LMConfig:
    n_layers: int
    d: int
    n_head: int
    n_kv_head: int
    d_mlp: int
    vocab: int
    C: dict = field(default_factory=dict)  # kind -> components (decomposed kinds only)
    mlp: str = "plain"  # "plain" (fc -> gelu_tanh -> down) or "glu" (silu(gate) * up -> down)
    eps: float = 1e-6
    rope_base: float = 10000.0
    # Llama-3 RoPE scaling (factor, low_freq_factor, high_freq_factor, original context);
    # None: the plain inverse frequencies
    rope_scaling: tuple | None = None

    @property
    def head_dim(self) -> int:
        return self.d // self.n_head

    @property
    def kinds(self) -> tuple[str, ...]:
        return PLAIN_KINDS if self.mlp == "plain" else GLU_KINDS

    def site_dims(self, kind: str) -> tuple[int, int]:
        """(d_in, d_out) of one layer's matrix of this kind (right-multiplication)."""
        hd = self.head_dim
        return {"q_proj": (self.d, self.n_head * hd), "k_proj": (self.d, self.n_kv_head * hd),
                "v_proj": (self.d, self.n_kv_head * hd), "o_proj": (self.n_head * hd, self.d),
                "c_fc": (self.d, self.d_mlp), "gate_proj": (self.d, self.d_mlp), "up_proj": (self.d, self.d_mlp),
                "down_proj": (self.d_mlp, self.d)}[kind]


# ---------------------------------------------------------------- bf16 storage model
def _round_t(x: torch.Tensor) -> torch.Tensor:
    return torch.from_numpy(po.round_bf16(x.detach().cpu().numpy())).to(x.dtype)


class _RoundBF16(torch.autograd.Function):
    """bf16 rounding of a stored value, and of its cotangent on the way back."""

    @staticmethod
    def forward(ctx, x):
        return _round_t(x)

    @staticmethod
    def backward(ctx, g):
        return _round_t(g)


class _Rounder:
    """The storage model: bf16 rounding (value and cotangent) or the identity."""

    def __init__(self, bf16: bool):
        self.bf16 = bf16

    def __call__(self, t):
        return _RoundBF16.apply(t) if self.bf16 else t


def _rounder(bf16_storage: bool):
    return _Rounder(bf16_storage)


# ---------------------------------------------------------------- squashing with the reference VJPs
class _LowerLeaky(torch.autograd.Function):
    """`lower_leaky_hard_sigmoid` (`pd/core/ci_fn/squashing.py:8-22`) with its custom VJP."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return x.clamp(0.0, 1.0)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return torch.from_numpy(np.asarray(po.lower_leaky_vjp(x.numpy(), g.numpy()))).to(x.dtype)


class _UpperLeaky(torch.autograd.Function):
    """`upper_leaky_hard_sigmoid` (`pd/core/ci_fn/squashing.py:41-45`)."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return torch.from_numpy(np.asarray(po.upper_leaky(x.numpy()))).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return torch.from_numpy(np.asarray(po.upper_leaky_vjp(x.numpy(), g.numpy()))).to(x.dtype)


# ---------------------------------------------------------------- target pieces
def rms_norm(x, w, eps, rb=lambda t: t):
    """`pd/target_ports/llama.py:90-97`: `w * (x * rsqrt(mean(x^2) + eps))`, the normalized
    value cast to the activation dtype before the weight multiply (`rb`)."""
    return w * rb(x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps))


def rope_inv_freq(head_dim: int, base: float, scaling=None):
    """`inv_freq = base^(-2i/head_dim)`, with Llama-3 scaling when `scaling = (factor, low,
    high, old_ctx)` (`pd/target_ports/llama.py:71-87`): wavelengths above old_ctx / low
    divide by factor, below old_ctx / high stay, and the band between interpolates with
    `smooth = (old_ctx / wavelen - low) / (high - low)`."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=F64) / head_dim))
    if scaling is None:
        return inv_freq
    factor, low, high, old_ctx = scaling
    wavelen = 2.0 * math.pi / inv_freq
    scaled = torch.where(wavelen > old_ctx / low, inv_freq / factor, inv_freq)
    smooth = (old_ctx / wavelen - low) / (high - low)
    smoothed = (1.0 - smooth) * scaled / factor + smooth * scaled
    medium = ~(wavelen < old_ctx / high) & ~(wavelen > old_ctx / low)
    return torch.where(medium, smoothed, scaled)


def rope_cos_sin(T: int, head_dim: int, base: float, scaling=None):
    """Rotate-half RoPE tables at positions 0..T-1 (`pd/target_ports/llama.py:100-105`)
    over `rope_inv_freq`."""
    inv_freq = rope_inv_freq(head_dim, base, scaling)
    freqs = torch.arange(T, dtype=F64)[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def apply_rope(x, cos, sin):
    """x [b, heads, t, hd]."""
    return x * cos + rotate_half(x) * sin


class _CausalCore(torch.autograd.Function):
    """softmax(q k^T * scale, causal) v on head-major [b, H, t, hd] operands, with the
    backward spelled out: dP = dO V^T, dS = P (dP - rowsum(P dP)) scale, dQ = dS K,
    dK = dS^T Q, dV = P^T dO. `bf16` rounds P, dS, dQ, dK and dV (the tensors a fused bf16
    attention stores) and nothing else."""

    @staticmethod
    def forward(ctx, q, k, v, bf16):
        t, hd = q.shape[-2], q.shape[-1]
        rb = _round_t if bf16 else (lambda x: x)
        s = (q @ k.transpose(-1, -2)) * hd**-0.5
        causal = torch.ones(t, t, dtype=torch.bool).tril()
        p = rb(torch.softmax(s.masked_fill(~causal, float("-inf")), dim=-1))
        ctx.save_for_backward(q, k, v, p)
        ctx.bf16 = bf16
        return p @ v

    @staticmethod
    def backward(ctx, do):
        q, k, v, p = ctx.saved_tensors
        rb = _round_t if ctx.bf16 else (lambda x: x)
        dp = do @ v.transpose(-1, -2)
        ds = rb(p * (dp - (p * dp).sum(-1, keepdim=True)) * q.shape[-1] ** -0.5)
        return rb(ds @ k), rb(ds.transpose(-1, -2) @ q), rb(p.transpose(-1, -2) @ do), None


def causal_attention(q, k, v, n_head: int, n_kv_head: int, base: float, rb=lambda t: t, scaling=None):
    """q [b, t, H*hd], k/v [b, t, KV*hd] -> [b, t, H*hd]: RoPE on q and k, then causal
    softmax(q k^T / sqrt(hd)) v with each kv head serving H/KV query heads."""
    b, t, qd = q.shape
    hd = qd // n_head
    rep = n_head // n_kv_head
    qh = q.reshape(b, t, n_head, hd).transpose(1, 2)
    kh = k.reshape(b, t, n_kv_head, hd).transpose(1, 2)
    vh = v.reshape(b, t, n_kv_head, hd).transpose(1, 2)
    cos, sin = rope_cos_sin(t, hd, base, scaling)
    cos, sin = rb(cos.to(q.dtype)), rb(sin.to(q.dtype))  # the tables are cast to the activation dtype
    qh, kh = rb(apply_rope(qh, cos, sin)), rb(apply_rope(kh, cos, sin))
    kh = kh.repeat_interleave(rep, dim=1)
    vh = vh.repeat_interleave(rep, dim=1)
    o = _CausalCore.apply(qh, kh, vh, bool(getattr(rb, "bf16", False)))
    return o.transpose(1, 2).reshape(b, t, qd)


def gelu_tanh(x):
    """`jax.nn.gelu(approximate=True)` (`pd/targets/transformer.py:802-805`)."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x**3)))


def site(x, W, V=None, U=None, mask=None, delta=None, rb=lambda t: t, route=None):
    """`((x@V) * (m - d)) @ U + d * (x @ W^T)` (`pd/core/decomposed_linear.py:142-175`);
    the frozen `x @ W^T` when V is None; with `route` ([..., bool]) the unrouted rows take
    the frozen `x @ W^T` (`blend_target_output`, `:72-85`)."""
    if V is None:
        return rb(x @ W.T)
    xV = rb(x @ V)
    coef = mask if delta is None else mask - delta[..., None]
    acts = rb(xV * coef)
    if delta is None:
        out = rb(acts @ U)
    else:
        # d * (x @ W^T) scales its own fp32 accumulation before acts @ U joins it: one
        # rounding of the sum, and neither d * x nor its cotangent d * g is stored
        out = rb(acts @ U + delta[..., None] * (x @ W.T))
    if route is None:
        return out
    return torch.where(torch.as_tensor(route, dtype=torch.bool)[..., None], out, rb(x @ W.T))


def block(cfg: LMConfig, P: dict, r, masks=None, deltas=None, rb=lambda t: t, layer=0, routes=None):
    """One transformer block (`pd/targets/transformer.py:1085-1140`). P holds ln1, ln2
    and W_<kind> [d_out, d_in] for every kind, plus V_<kind>/U_<kind> for decomposed
    kinds; masks/deltas/routes map kind -> [b, t, C] / [b, t] / [b, t] bool (absent kind:
    frozen; absent route: every position routed)."""
    masks = masks or {}
    deltas = deltas or {}
    routes = routes or {}

    def run(kind, x):
        if kind in masks:
            return site(x, P["W_" + kind], P["V_" + kind], P["U_" + kind], masks[kind], deltas.get(kind), rb=rb,
                        route=routes.get(kind))
        return site(x, P["W_" + kind], rb=rb)

    h = rb(rms_norm(r, P["ln1"], cfg.eps, rb))
    q, k, v = run("q_proj", h), run("k_proj", h), run("v_proj", h)
    a = rb(causal_attention(q, k, v, cfg.n_head, cfg.n_kv_head, cfg.rope_base, rb=rb, scaling=cfg.rope_scaling))
    r = rb(r + run("o_proj", a))
    h2 = rb(rms_norm(r, P["ln2"], cfg.eps, rb))
    if cfg.mlp == "plain":
        down_in = rb(gelu_tanh(run("c_fc", h2)))
    else:
        down_in = rb(torch.nn.functional.silu(run("gate_proj", h2)) * run("up_proj", h2))
    return rb(r + run("down_proj", down_in))


def final_act(cfg: LMConfig, params: dict, r, rb=lambda t: t):
    return rb(rms_norm(r, params["norm"], cfg.eps, rb))


def forward(cfg: LMConfig, params: dict, r0, masks=None, deltas=None, rb=lambda t: t, routes=None):
    """Residual stream r0 [b, t, d] through every layer; masks[l] / deltas[l] / routes[l]
    per layer (None: the frozen target). Returns the final normed activations [b, t, d]."""
    r = r0
    for l, P in enumerate(params["layers"]):
        r = block(cfg, P, r, None if masks is None else masks[l], None if deltas is None else deltas[l], rb=rb,
                  layer=l, routes=None if routes is None else routes[l])
    return final_act(cfg, params, r, rb=rb)


def logits(params, act):
    return act @ params["head"].T


def kl_per_position(masked_logits, clean_logits):
    """`pd/targets/losses.py:50-60`: mean over positions of KL(softmax(clean) || softmax(masked))."""
    log_q = torch.log_softmax(masked_logits, -1)
    log_p = torch.log_softmax(clean_logits, -1)
    n = math.prod(masked_logits.shape[:-1])
    return (log_p.exp() * (log_p - log_q)).sum() / n


# ---------------------------------------------------------------- the step
def site_keys(draw_key, cfg: LMConfig, kind: str, layer: int, partitionable=True):
    """(mask key, delta key) of one site (`pd/targets/transformer.py:1424-1451`)."""
    src_base, delta_base = tf.split(draw_key, partitionable=partitionable)
    ki = cfg.kinds.index(kind)
    return (tf.fold_in(tf.fold_in(src_base, ki), layer), tf.fold_in(tf.fold_in(delta_base, ki), layer))


def lm_stack_step(cfg: LMConfig, params: dict, tokens, ci_pre, draw_key, *, p=2.0, imp_coeff=1.0, recon_coeff=1.0,
                  bf16_storage=False, partitionable=True, use_delta=True, uniforms=None, dtype=F64, imp_min=None,
                  freq_ema=None, ema_count=0.0, routes=None, sources=None):
    """One stochastic-recon KL + imp-min step, forward and backward. The imp-min term is
    L_p (p, imp_coeff) or `imp_min` (a `pd_oracle.ImpMin`; smooth-L0 with the frequency
    penalty as the reference writes it, `pd/core/losses.py:340-394`: per-site means of
    psi over the tokens, differentiated by autograd). `freq_ema[l][kind]` ([C_kind], with
    `imp_min.ema_halflife`) is the EMA frequency estimate before this step after
    `ema_count` observations: the frequency term is then the reference's surrogate
    `Phi(f_hat) + Phi'(f_hat) (f - sg(f))` (`pd/core/losses.py:425-458`), and the result
    also holds the new estimates (`freq_ema`) and the batch penalty (`freq_batch`).

    params: wte [V, d] (the embedding and the tied head), norm [d], layers: list of
    dicts (ln1, ln2, W_<kind> [d_out, d_in], V_<kind> [d_in, C], U_<kind> [C, d_out])
    as float64 numpy arrays; tokens [b, t] int; ci_pre[l][kind] [b*t, C_kind].
    `uniforms[l][kind] = (u [b*t, C], d [b*t])` replaces the Threefry draws when given.
    `routes[l][kind]` ([b*t] bool) routes the recon term per token: an unrouted token's
    site output is the target's (`site`'s route arm).
    `dtype` torch.float32 runs the same arithmetic in fp32 (the CPU baseline's timing
    form; the float64 default is the checker).
    `sources = (src, src_delta, rows_per_source)` replaces the draws by persistent
    (adversarial) source tables (`pd/core/source_mask.py:56-63`, `pd/core/masking.py:
    260-272`): src[l][kind] [S, C_kind], src_delta[l][kind] [S] (or src_delta None: no
    delta channel), every source row covering rows_per_source consecutive tokens of the
    flattened [b*t] order (S = b*t / rows_per_source: the `c`, `bc` and `bsc` shapes). The
    tables are cast to the CI dtype before use (bf16 with `bf16_storage`), m = lower +
    (1 - lower) src[n // rps] and d = src_delta[n // rps]; the result then also holds the
    tables' gradients d_src[l][kind] and d_src_delta[l][kind].
    Returns dict(loss, recon, imp, freq, dV[l][kind], dU[l][kind], d_ci_pre[l][kind], u, delta)."""
    rb = _rounder(bf16_storage)
    spec = imp_min if imp_min is not None else po.ImpMin("pnorm", p=p, coeff=imp_coeff)
    b, t = tokens.shape
    N = b * t
    T = lambda a, g=False: torch.tensor(np.asarray(a, np.float64), dtype=dtype, requires_grad=g)  # noqa: E731
    prm = {"head": T(params["wte"]), "norm": T(params["norm"]), "layers": []}
    leaves = []
    for l, L_ in enumerate(params["layers"]):
        P = {"ln1": T(L_["ln1"]), "ln2": T(L_["ln2"])}
        for kind in cfg.kinds:
            P["W_" + kind] = T(L_["W_" + kind])
            if kind in cfg.C:
                P["V_" + kind], P["U_" + kind] = T(L_["V_" + kind], True), T(L_["U_" + kind], True)
                leaves.append((l, kind))
        prm["layers"].append(P)
    r0 = rb(prm["head"][torch.as_tensor(np.asarray(tokens, np.int64))])
    with torch.no_grad():
        act_c = forward(cfg, prm, r0, rb=rb)
        clean_logits = logits(prm, act_c)
    masks, deltas, pres, us, ds = [], [], {}, {}, {}
    src_leaf, srcd_leaf = {}, {}
    if sources is not None:
        use_delta = sources[1] is not None
        doc = torch.as_tensor(np.arange(N) // sources[2], dtype=torch.long)
    imp = torch.zeros((), dtype=dtype)
    freq = torch.zeros((), dtype=dtype)
    freq_batch = 0.0
    new_ema = None if freq_ema is None else [{} for _ in range(cfg.n_layers)]
    for l in range(cfg.n_layers):
        masks.append({})
        deltas.append({})
        for kind in cfg.kinds:
            if kind not in cfg.C:
                continue
            C = cfg.C[kind]
            pre = T(ci_pre[l][kind], True)
            pres[(l, kind)] = pre
            if sources is not None:  # the tables as autograd leaves, cast to the CI dtype
                src_leaf[(l, kind)] = T(sources[0][l][kind], True)
                u_t = rb(src_leaf[(l, kind)])[doc]
                if use_delta:
                    srcd_leaf[(l, kind)] = T(sources[1][l][kind], True)
                    d_t = rb(srcd_leaf[(l, kind)])[doc]
                u, dl = u_t.detach().numpy(), (d_t.detach().numpy() if use_delta else np.zeros(N))
            elif uniforms is not None:
                u, dl = uniforms[l][kind]
                u = np.asarray(u, np.float64)
                dl = np.asarray(dl, np.float64)
            else:
                mk, dk = site_keys(draw_key, cfg, kind, l, partitionable)
                u = tf.uniform(mk, (N, C), "bfloat16", partitionable=partitionable)
                dl = tf.uniform(dk, (N,), "bfloat16", partitionable=partitionable) if use_delta else np.zeros(N)
            us[(l, kind)], ds[(l, kind)] = u, dl
            lo = _LowerLeaky.apply(pre)
            up = _UpperLeaky.apply(pre)
            if spec.kind == "pnorm":
                imp = imp + (up**spec.p).sum() / N
            else:
                g2 = spec.gamma**2
                psi = up**2 / (up**2 + g2) * ((1.0 + g2) if spec.normalize_at_one else 1.0)
                fr = psi.mean(0)
                imp = imp + fr.sum()
                if spec.ref_count > 0:
                    f_sg = fr.detach()
                    freq_batch += float((f_sg * torch.log2(1.0 + spec.ref_count * f_sg)).sum())
                    if freq_ema is None:
                        freq = freq + (fr * torch.log2(1.0 + spec.ref_count * fr)).sum()
                    else:
                        alpha, debias = po.ema_decay_terms(ema_count, spec.ema_halflife)
                        prev = torch.tensor(np.asarray(freq_ema[l][kind], np.float64), dtype=dtype)
                        nxt = prev + alpha * (f_sg - prev)
                        new_ema[l][kind] = nxt.numpy()
                        f_hat = nxt / debias
                        a_ = spec.ref_count
                        slope = torch.log2(1.0 + a_ * f_hat) + a_ * f_hat / ((1.0 + a_ * f_hat) * math.log(2.0))
                        freq = freq + (f_hat * torch.log2(1.0 + a_ * f_hat) + slope * (fr - f_sg)).sum()
            if sources is not None:
                masks[l][kind] = (lo + (1.0 - lo) * u_t).reshape(b, t, C)
                deltas[l][kind] = d_t.reshape(b, t) if use_delta else None
            else:
                masks[l][kind] = (lo + (1.0 - lo) * T(u)).reshape(b, t, C)
                deltas[l][kind] = T(dl).reshape(b, t) if use_delta else None
    rts = None if routes is None else [{k: np.asarray(v, bool).reshape(b, t) for k, v in layer.items()}
                                       for layer in routes]
    act_m = forward(cfg, prm, r0, masks, deltas, rb=rb, routes=rts)
    recon = kl_per_position(logits(prm, act_m), clean_logits)
    loss = recon_coeff * recon + spec.coeff * imp + (spec.freq_coeff * freq if spec.kind == "smooth_l0" else 0.0)
    wrt = [prm["layers"][l]["V_" + k] for l, k in leaves] + [prm["layers"][l]["U_" + k] for l, k in leaves] + [
        pres[key] for key in pres] + [src_leaf[key] for key in src_leaf] + [srcd_leaf[key] for key in srcd_leaf]
    grads = torch.autograd.grad(loss, wrt)
    n = len(leaves)
    out = dict(loss=float(loss.detach()), recon=float(recon.detach()), imp=float(imp.detach()),
               freq=float(freq.detach()), freq_ema=new_ema, freq_batch=freq_batch,
               dV=[{} for _ in range(cfg.n_layers)],
               dU=[{} for _ in range(cfg.n_layers)], d_ci_pre=[{} for _ in range(cfg.n_layers)], u=us, delta=ds)
    for i, (l, k) in enumerate(leaves):
        out["dV"][l][k] = grads[i].numpy()
        out["dU"][l][k] = grads[n + i].numpy()
    for i, key in enumerate(pres):
        out["d_ci_pre"][key[0]][key[1]] = grads[2 * n + i].numpy()
    if sources is not None:
        out["d_src"] = [{} for _ in range(cfg.n_layers)]
        out["d_src_delta"] = [{} for _ in range(cfg.n_layers)]
        base = 2 * n + len(pres)
        for i, key in enumerate(src_leaf):
            out["d_src"][key[0]][key[1]] = grads[base + i].numpy()
        for i, key in enumerate(srcd_leaf):
            out["d_src_delta"][key[0]][key[1]] = grads[base + len(src_leaf) + i].numpy()
    return out


def init_lm(cfg: LMConfig, rng, *, ci_range=(-0.3, 1.3)):
    """Random target (N(0, d_in^-1/2) weights, N(0, 1) tied embedding/head scaled by
    d^-1/2, unit norms) and components (`pd/core/components.py:650-677`: V by d_in^-1/2,
    U by C^-1/2), with CI preactivations uniform on `ci_range`."""

    def rn(*shape, scale=1.0):
        return rng.standard_normal(size=shape, dtype=np.float32).astype(np.float64) * scale

    params = {"wte": rn(cfg.vocab, cfg.d, scale=cfg.d**-0.5), "norm": np.ones(cfg.d), "layers": []}
    for _ in range(cfg.n_layers):
        L_ = {"ln1": 1.0 + rn(cfg.d, scale=0.1), "ln2": 1.0 + rn(cfg.d, scale=0.1)}
        for kind in cfg.kinds:
            din, dout = cfg.site_dims(kind)
            L_["W_" + kind] = rn(dout, din, scale=din**-0.5)
            if kind in cfg.C:
                C = cfg.C[kind]
                L_["V_" + kind] = rn(din, C, scale=din**-0.5)
                L_["U_" + kind] = rn(C, dout, scale=C**-0.5)
        params["layers"].append(L_)
    return params


def init_ci(cfg: LMConfig, n_tokens: int, rng, lo=-0.3, hi=1.3):
    return [{k: rng.uniform(lo, hi, size=(n_tokens, cfg.C[k])) for k in cfg.kinds if k in cfg.C}
            for _ in range(cfg.n_layers)]
