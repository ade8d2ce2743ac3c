"""fp32 PyTorch-CPU restatement of the llm.cu LoRA training step.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product path.

Each function cites the reference file:line (visheshnarayan/llm.cu) whose
math it restates.  The reference is fp32 CUDA; this module is fp32 torch on
the CPU, with exact math where the reference deviates from it (the quirk
switches ``quirks={'lora_dx','silu_alias','final_norm'}`` reproduce the
reference's deviations for characterisation only):

  Q1 ``lora_dx``    src/kernels/lora_backward.cu:87 reads A[r, d_in] as if it
                    were [d_in, r] when forming the LoRA input gradient.
  Q2 ``silu_alias`` src/kernels/lora_backward.cu:287 calls silu_backward with
                    d_swiglu aliasing d_gate, so d_up picks up the freshly
                    written d_gate (src/kernels/activation.cu:36-37).
  Q3 ``final_norm`` src/kernels/lora_backward.cu:266 back-propagates the
                    final RMSNorm with x = post_attn of the last layer.
Q4 (the uninitialised last dlogits row, src/kernels/loss.cu:18-21) is always
resolved to zeros here; Q5 (loss averaged over the S-1 rows that have a
target inside the window, src/kernels/loss.cu:86-90) is kept.

Parity pinning: every closed form here is checked in tests/ against
torch.autograd and (float64, tiny shapes) central finite differences.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence

import torch
import torch.nn.functional as F

PROJS = ("wq", "wk", "wv", "wo")


@dataclass(frozen=True)
class Dims:
    """Model constants (reference include/config.h:5-21, include/lora.h:6-8)."""
    hidden: int = 2048
    n_layers: int = 28
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    vocab: int = 151936
    rank: int = 16
    alpha: float = 32.0
    eps: float = 1e-6
    theta: float = 1e6

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def group(self) -> int:
        # config.h:15 KV_HEAD_GROUPS; Q head h reads KV head h // group
        return self.n_heads // self.n_kv_heads

    @property
    def lora_scale(self) -> float:
        # lora.h:8 LORA_SCALE = LORA_ALPHA / LORA_RANK = 2.0
        return self.alpha / self.rank

    def adapter_dims(self, proj: str):
        """(d_out, d_in) per adapter (reference lora.cu:70-77)."""
        return {"wq": (self.q_dim, self.hidden), "wk": (self.kv_dim, self.hidden),
                "wv": (self.kv_dim, self.hidden), "wo": (self.hidden, self.q_dim)}[proj]


QWEN3_1_7B = Dims()
TINY = Dims(hidden=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16,
            intermediate=96, vocab=512)


@dataclass
class LayerW:
    """Frozen per-layer weights, [out, in] row-major like the reference ``LW``
    (src/train.cu:10-17)."""
    attn_norm: torch.Tensor
    ffn_norm: torch.Tensor
    wq: torch.Tensor
    wk: torch.Tensor
    wv: torch.Tensor
    wo: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    w_gate: torch.Tensor
    w_up: torch.Tensor
    w_down: torch.Tensor


@dataclass
class ModelW:
    """Frozen model (reference ``MW``, src/train.cu:18-24)."""
    embed: torch.Tensor
    layers: List[LayerW]
    final_norm: torch.Tensor
    lm_head: torch.Tensor


@dataclass
class Adapter:
    """One LoRA adapter: A [r, d_in], B [d_out, r] (include/lora.h:13-20)."""
    A: torch.Tensor
    B: torch.Tensor
    mA: Optional[torch.Tensor] = None
    vA: Optional[torch.Tensor] = None
    mB: Optional[torch.Tensor] = None
    vB: Optional[torch.Tensor] = None


Adapters = List[Dict[str, Adapter]]
Identity: Callable[[torch.Tensor], torch.Tensor] = lambda t: t


# ---------------------------------------------------------------- primitives

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w  (src/kernels/rmsnorm.cu:6-29)."""
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return x * r * w


def rmsnorm_bwd(dy: torch.Tensor, x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """dx = r*(dy*w - (r^2/n)*sum(dy*w*x)*x), r recomputed from x
    (src/kernels/rmsnorm.cu:53-89).  The norm weight is frozen: no dw."""
    n = x.shape[-1]
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    c = (r * r / n) * (dy * w * x).sum(-1, keepdim=True)
    return r * (dy * w - c * x)


def rope_tables(seq_len: int, head_dim: int, theta: float):
    """cos/sin [S, head_dim/2] for the half-split rotation.

    The reference evaluates freq = 1/powf(theta, 2d/head_dim), angle =
    pos*freq and cosf/sinf in fp32 (src/kernels/rope.cu:15-18); the angles are
    formed here in float64 and rounded once to fp32, which is what the HIP
    library uploads as its table (fp32 angle rounding at pos ~2047 alone is
    ~1e-4 rad, the only difference)."""
    d = torch.arange(head_dim // 2, dtype=torch.float64)
    freq = 1.0 / (theta ** (2.0 * d / head_dim))
    pos = torch.arange(seq_len, dtype=torch.float64)
    ang = pos[:, None] * freq[None, :]
    return torch.cos(ang).float(), torch.sin(ang).float()


def rope_fwd(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate pairs (d, d+hd/2) by angle pos*freq_d (src/kernels/rope.cu:7-27).
    x: [B, S, heads, hd]; cos/sin: [S, hd/2]."""
    half = x.shape[-1] // 2
    x0, x1 = x[..., :half], x[..., half:]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return torch.cat([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1)


def rope_bwd(dy: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Transpose (= inverse) rotation (src/kernels/rope.cu:57-82)."""
    half = dy.shape[-1] // 2
    d0, d1 = dy[..., :half], dy[..., half:]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return torch.cat([d0 * c + d1 * s, d1 * c - d0 * s], dim=-1)


def attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """Causal GQA attention, scale 1/sqrt(hd), Q head h reads KV head h//group
    (src/kernels/lora_forward.cu:48-120, 138-147).
    q: [B, S, nq, hd]; k, v: [B, S, nkv, hd].  Returns O [B, S, nq, hd] and the
    log-sum-exp of the scaled scores [B, nq, S] (what a flash backward keeps
    instead of P)."""
    Bn, S, nq, hd = q.shape
    group = nq // k.shape[2]
    kx = k.repeat_interleave(group, dim=2)
    vx = v.repeat_interleave(group, dim=2)
    qh, kh, vh = (t.permute(0, 2, 1, 3) for t in (q, kx, vx))
    s = torch.matmul(qh, kh.transpose(-1, -2)) * (1.0 / math.sqrt(hd))
    mask = torch.ones(S, S, dtype=torch.bool).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    o = torch.matmul(p, vh).permute(0, 2, 1, 3)
    return o, lse


def attention_bwd(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  o: torch.Tensor, lse: torch.Tensor):
    """Closed-form causal GQA attention backward with P recomputed from the LSE
    (the math of src/kernels/lora_backward.cu:104-199 without atomics):
    dP = dO V^T; delta_i = sum_d dO_id O_id; dS = P*(dP - delta);
    dQ = dS K/sqrt(d); dK = dS^T Q/sqrt(d); dV = P^T dO; GQA heads summed."""
    Bn, S, nq, hd = q.shape
    nkv = k.shape[2]
    group = nq // nkv
    scale = 1.0 / math.sqrt(hd)
    kx = k.repeat_interleave(group, dim=2)
    vx = v.repeat_interleave(group, dim=2)
    qh, kh, vh, oh, doh = (t.permute(0, 2, 1, 3) for t in (q, kx, vx, o, do))
    s = torch.matmul(qh, kh.transpose(-1, -2)) * scale
    mask = torch.ones(S, S, dtype=torch.bool).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    p = torch.exp(s - lse[..., None])
    dp = torch.matmul(doh, vh.transpose(-1, -2))
    delta = (doh * oh).sum(-1, keepdim=True)
    ds = p * (dp - delta)
    dq = torch.matmul(ds, kh) * scale
    dkx = torch.matmul(ds.transpose(-1, -2), qh) * scale
    dvx = torch.matmul(p.transpose(-1, -2), doh)
    dq = dq.permute(0, 2, 1, 3)
    dk = dkx.permute(0, 2, 1, 3).reshape(Bn, S, nkv, group, hd).sum(3)
    dv = dvx.permute(0, 2, 1, 3).reshape(Bn, S, nkv, group, hd).sum(3)
    return dq, dk, dv


def silu_mul(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """silu(g)*u (src/kernels/activation.cu:5-11)."""
    return g * torch.sigmoid(g) * u


def silu_mul_bwd(dy: torch.Tensor, g: torch.Tensor, u: torch.Tensor, alias_quirk: bool = False):
    """d_g = dy*u*sig*(1+g*(1-sig)); d_u = dy*silu(g)
    (src/kernels/activation.cu:26-38).  ``alias_quirk`` reproduces Q2."""
    sig = torch.sigmoid(g)
    dg = dy * u * (sig * (1.0 + g * (1.0 - sig)))
    du = (dg if alias_quirk else dy) * (g * sig)
    return dg, du


def lora_fwd(x: torch.Tensor, A: torch.Tensor, B: torch.Tensor, scale: float):
    """h = x A^T [T, r]; delta_y = scale * h B^T (src/kernels/lora.cu:181-202)."""
    h = x @ A.t()
    return h, scale * (h @ B.t())


def lora_bwd(x: torch.Tensor, h: torch.Tensor, dy: torch.Tensor, A: torch.Tensor,
             B: torch.Tensor, scale: float, dx_quirk: bool = False):
    """dB = s dy^T h; dh = dy B; dA = s dh^T x; dx = s dh A
    (src/kernels/lora_backward.cu:50-90 + the caller's scale_add, :319).
    ``dx_quirk`` reproduces Q1 (A[r, d_in] read as [d_in, r], :87)."""
    dB = scale * (dy.t() @ h)
    dh = dy @ B
    dA = scale * (dh.t() @ x)
    if dx_quirk:
        dx = scale * (dh @ A.reshape(A.shape[1], A.shape[0]).t())
    else:
        dx = scale * (dh @ A)
    return dA, dB, dx, dh


def valid_rows(batch: int, seq_len: int) -> torch.Tensor:
    """Rows with a next-token target inside the window: i < S-1 per sequence
    (src/kernels/loss.cu:18-21, Q5)."""
    m = torch.ones(batch, seq_len, dtype=torch.bool)
    m[:, -1] = False
    return m.reshape(-1)


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor, valid: torch.Tensor):
    """Per row: m = max; Z = sum exp(x-m); loss_i = -(x_t - m - ln Z);
    dlogits = (exp(x-m)/Z - 1[j=t]) / n_valid; mean over valid rows
    (src/kernels/loss.cu:13-91).  Invalid rows get dlogits = 0 (Q4)."""
    n_valid = int(valid.sum())
    m = logits.max(-1, keepdim=True).values
    z = torch.exp(logits - m).sum(-1, keepdim=True)
    lse = m + torch.log(z)
    tgt = targets.long().clamp(0, logits.shape[-1] - 1)
    x_t = logits.gather(-1, tgt[:, None])
    loss_rows = (lse - x_t).squeeze(-1)
    loss = (loss_rows * valid).sum() / n_valid
    p = torch.exp(logits - lse)
    onehot = torch.zeros_like(logits).scatter_(-1, tgt[:, None], 1.0)
    dlogits = (p - onehot) / n_valid * valid[:, None]
    return loss, dlogits, loss_rows


def adamw(p, g, m, v, lr, beta1, beta2, eps, wd, step):
    """Decoupled-decay AdamW, decay applied to A and B alike
    (src/kernels/lora.cu:206-246): bc = 1 - beta^t in fp32 (powf, :238-239);
    m = b1 m + (1-b1) g; v = b2 v + (1-b2) g^2;
    p = p (1 - lr wd) - lr (m/bc1) / (sqrt(v/bc2) + eps).  Returns new p, m, v."""
    f32 = torch.float32
    bc1 = torch.tensor(1.0, dtype=f32) - torch.tensor(beta1, dtype=f32) ** step
    bc2 = torch.tensor(1.0, dtype=f32) - torch.tensor(beta2, dtype=f32) ** step
    m2 = beta1 * m + (1.0 - beta1) * g
    v2 = beta2 * v + (1.0 - beta2) * g * g
    p2 = p * (1.0 - lr * wd) - lr * (m2 / bc1) / (torch.sqrt(v2 / bc2) + eps)
    return p2, m2, v2


# ---------------------------------------------------------------- one layer

def layer_forward(x: torch.Tensor, lw: LayerW, lad: Dict[str, Adapter], dims: Dims,
                  batch: int, seq_len: int, cos, sin, rnd: Callable = Identity):
    """One decoder layer with LoRA on Q/K/V/O, in the reference op order
    (src/kernels/lora_forward.cu:198-298): LoRA enters before the QK-norm.
    x: [T, H] with T = batch*seq_len.  ``rnd`` rounds GEMM operands (identity
    for the exact oracle; fp16 rounding to emulate the device precision)."""
    s = dims.lora_scale
    T = x.shape[0]
    st = {"x_in": x}
    xn = rmsnorm(x, lw.attn_norm, dims.eps)
    st["xn"] = xn
    xr = rnd(xn)
    out = {}
    for proj, w in (("wq", lw.wq), ("wk", lw.wk), ("wv", lw.wv)):
        h, dy = lora_fwd(xr, rnd(lad[proj].A), lad[proj].B, s)
        st["h_" + proj] = h
        out[proj] = xr @ rnd(w).t() + dy
    st["q_raw"], st["k_raw"], st["v"] = out["wq"], out["wk"], out["wv"]
    q = rmsnorm(out["wq"].reshape(T, dims.n_heads, dims.head_dim), lw.q_norm, dims.eps)
    k = rmsnorm(out["wk"].reshape(T, dims.n_kv_heads, dims.head_dim), lw.k_norm, dims.eps)
    q = rope_fwd(q.reshape(batch, seq_len, dims.n_heads, dims.head_dim), cos, sin)
    k = rope_fwd(k.reshape(batch, seq_len, dims.n_kv_heads, dims.head_dim), cos, sin)
    v = out["wv"].reshape(batch, seq_len, dims.n_kv_heads, dims.head_dim)
    q, k, v = rnd(q), rnd(k), rnd(v)
    st["q"], st["k"], st["vh"] = q, k, v
    o, lse = attention_fwd(q, k, v)
    st["lse"] = lse
    o = rnd(o.reshape(T, dims.q_dim))
    st["o"] = o
    h_o, dy_o = lora_fwd(o, rnd(lad["wo"].A), lad["wo"].B, s)
    st["h_wo"] = h_o
    x_mid = x + (o @ rnd(lw.wo).t() + dy_o)
    st["x_mid"] = x_mid
    xn2 = rnd(rmsnorm(x_mid, lw.ffn_norm, dims.eps))
    st["xn2"] = xn2
    g = xn2 @ rnd(lw.w_gate).t()
    u = xn2 @ rnd(lw.w_up).t()
    st["g"], st["u"] = g, u
    a = rnd(silu_mul(g, u))
    x_out = x_mid + a @ rnd(lw.w_down).t()
    return x_out, st


def layer_backward(dx_out: torch.Tensor, st: dict, lw: LayerW, lad: Dict[str, Adapter],
                   dims: Dims, batch: int, seq_len: int, cos, sin,
                   quirks: Sequence[str] = (), rnd: Callable = Identity, rnd_g: Callable = Identity):
    """Closed-form backward of ``layer_forward`` in the reference order
    (src/kernels/lora_backward.cu:271-406).  Returns (dx_in, grads) where
    grads[proj] = (dA, dB).  ``rnd_g`` rounds gradient GEMM operands."""
    s = dims.lora_scale
    T = dx_out.shape[0]
    grads = {}
    # MLP (:284-300)
    da = rnd_g(dx_out) @ rnd(lw.w_down)
    dg, du = silu_mul_bwd(da, st["g"], st["u"], alias_quirk="silu_alias" in quirks)
    d_xn2 = rnd_g(dg) @ rnd(lw.w_gate) + rnd_g(du) @ rnd(lw.w_up)
    dx_mid = dx_out + rmsnorm_bwd(d_xn2, st["x_mid"], lw.ffn_norm, dims.eps)
    # O projection + LoRA (:312-319)
    dxm = rnd_g(dx_mid)
    d_o = dxm @ rnd(lw.wo)
    dA, dB, dx_l, _ = lora_bwd(st["o"], st["h_wo"], dx_mid, lad["wo"].A, lad["wo"].B, s,
                               dx_quirk="lora_dx" in quirks)
    grads["wo"] = (dA, dB)
    d_o = d_o + dx_l
    # attention (:321-356)
    dq, dk, dv = attention_bwd(rnd_g(d_o).reshape(batch, seq_len, dims.n_heads, dims.head_dim),
                               st["q"], st["k"], st["vh"],
                               st["o"].reshape(batch, seq_len, dims.n_heads, dims.head_dim),
                               st["lse"])
    # RoPE + QK-norm (:359-367)
    dq = rope_bwd(dq, cos, sin).reshape(T, dims.n_heads, dims.head_dim)
    dk = rope_bwd(dk, cos, sin).reshape(T, dims.n_kv_heads, dims.head_dim)
    dq = rmsnorm_bwd(dq, st["q_raw"].reshape(T, dims.n_heads, dims.head_dim), lw.q_norm, dims.eps)
    dk = rmsnorm_bwd(dk, st["k_raw"].reshape(T, dims.n_kv_heads, dims.head_dim), lw.k_norm, dims.eps)
    dproj = {"wq": dq.reshape(T, dims.q_dim), "wk": dk.reshape(T, dims.kv_dim),
             "wv": dv.reshape(T, dims.kv_dim)}
    # Q/K/V projections + LoRA (:376-397)
    d_xn = None
    for proj, w in (("wq", lw.wq), ("wk", lw.wk), ("wv", lw.wv)):
        dy = dproj[proj]
        t = rnd_g(dy) @ rnd(w)
        dA, dB, dx_l, _ = lora_bwd(st["xn"], st["h_" + proj], dy, lad[proj].A, lad[proj].B, s,
                                   dx_quirk="lora_dx" in quirks)
        grads[proj] = (dA, dB)
        t = t + dx_l
        d_xn = t if d_xn is None else d_xn + t
    # attention RMSNorm + residual (:400-403)
    dx_in = dx_mid + rmsnorm_bwd(d_xn, st["x_in"], lw.attn_norm, dims.eps)
    return dx_in, grads


# ---------------------------------------------------------------- full model

def model_forward(W: ModelW, ad: Adapters, tokens: torch.Tensor, dims: Dims,
                  rnd: Callable = Identity):
    """Embedding gather -> L layers -> final RMSNorm -> lm_head logits
    (src/kernels/lora_forward.cu:169-305, src/kernels/embed.cu:6-20).
    tokens: int [B, S].  Returns logits [T, V] and the stash (a list of
    per-layer dicts plus 'x_final' and 'xf')."""
    batch, seq_len = tokens.shape
    cos, sin = rope_tables(seq_len, dims.head_dim, dims.theta)
    x = W.embed[tokens.reshape(-1).long()]
    stash = {"layers": []}
    for l in range(dims.n_layers):
        x, st = layer_forward(x, W.layers[l], ad[l], dims, batch, seq_len, cos, sin, rnd)
        stash["layers"].append(st)
    stash["x_final"] = x
    xf = rnd(rmsnorm(x, W.final_norm, dims.eps))
    stash["xf"] = xf
    logits = xf @ rnd(W.lm_head).t()
    return logits, stash


def model_backward(dlogits: torch.Tensor, stash: dict, W: ModelW, ad: Adapters, dims: Dims,
                   batch: int, seq_len: int, quirks: Sequence[str] = (),
                   rnd: Callable = Identity, rnd_g: Callable = Identity):
    """Closed-form backward (src/kernels/lora_backward.cu:212-408).
    Returns grads[l][proj] = (dA, dB) and the gradient at the embedding output."""
    cos, sin = rope_tables(seq_len, dims.head_dim, dims.theta)
    dxf = rnd_g(dlogits) @ rnd(W.lm_head)                      # :243
    if "final_norm" in quirks:                                  # Q3, :266
        x_fin = stash["layers"][-1]["x_mid"]
    else:
        x_fin = stash["x_final"]
    dx = rmsnorm_bwd(dxf, x_fin, W.final_norm, dims.eps)
    grads: List[Dict[str, tuple]] = [None] * dims.n_layers
    for l in range(dims.n_layers - 1, -1, -1):
        dx, grads[l] = layer_backward(dx, stash["layers"][l], W.layers[l], ad[l], dims,
                                      batch, seq_len, cos, sin, quirks, rnd, rnd_g)
    return grads, dx


def step_autograd(W: ModelW, ad: Adapters, tokens: torch.Tensor, targets: torch.Tensor, dims: Dims):
    """Loss and adapter gradients through torch.autograd (ground truth for the
    closed-form backward).  targets: int [B, S]."""
    batch, seq_len = tokens.shape
    leaves = []
    ad2 = []
    for l in range(dims.n_layers):
        d = {}
        for p in PROJS:
            A = ad[l][p].A.detach().clone().requires_grad_(True)
            B = ad[l][p].B.detach().clone().requires_grad_(True)
            leaves += [A, B]
            d[p] = Adapter(A, B)
        ad2.append(d)
    logits, _ = model_forward(W, ad2, tokens, dims)
    valid = valid_rows(batch, seq_len)
    loss = F.cross_entropy(logits[valid], targets.reshape(-1)[valid].long())
    loss.backward()
    grads = [{p: (ad2[l][p].A.grad, ad2[l][p].B.grad) for p in PROJS} for l in range(dims.n_layers)]
    return loss.detach(), grads


def train_step(W: ModelW, ad: Adapters, tokens: torch.Tensor, targets: torch.Tensor, dims: Dims,
               step: int, lr: float = 3e-4, beta1: float = 0.9, beta2: float = 0.999,
               eps: float = 1e-8, wd: float = 0.01, quirks: Sequence[str] = (),
               rnd: Callable = Identity, rnd_g: Callable = Identity):
    """One llm_train step (src/train.cu:251-288): forward, CE, closed-form
    backward, AdamW.  Updates ``ad`` in place (A, B, m, v) and returns
    (loss, grads, dlogits)."""
    batch, seq_len = tokens.shape
    logits, stash = model_forward(W, ad, tokens, dims, rnd)
    loss, dlogits, _ = cross_entropy(logits, targets.reshape(-1), valid_rows(batch, seq_len))
    grads, _ = model_backward(dlogits, stash, W, ad, dims, batch, seq_len, quirks, rnd, rnd_g)
    adamw_all(ad, grads, lr, beta1, beta2, eps, wd, step)
    return loss, grads, dlogits


def adamw_all(ad: Adapters, grads, lr, beta1, beta2, eps, wd, step):
    """adamw_step_lora over every A and B (src/kernels/lora.cu:235-246)."""
    for l, d in enumerate(ad):
        for p in PROJS:
            a = d[p]
            for name in ("A", "B"):
                g = grads[l][p][0 if name == "A" else 1]
                prm = getattr(a, name)
                m = getattr(a, "m" + name)
                v = getattr(a, "v" + name)
                if m is None:
                    m = torch.zeros_like(prm)
                    v = torch.zeros_like(prm)
                p2, m2, v2 = adamw(prm, g, m, v, lr, beta1, beta2, eps, wd, step)
                setattr(a, name, p2)
                setattr(a, "m" + name, m2)
                setattr(a, "v" + name, v2)


def round_fp16(t: torch.Tensor) -> torch.Tensor:
    """Emulate an fp16 GEMM operand (round to nearest even, back to fp32)."""
    return t.half().float()


def round_fp16_rowscaled(t: torch.Tensor) -> torch.Tensor:
    """Emulate a gradient operand stored as fp16 with a power-of-two scale per
    row chosen so the row's max magnitude lands in [2^13, 2^14)."""
    amax = t.abs().amax(-1, keepdim=True).clamp_min(1e-30)
    e = torch.floor(torch.log2(amax))
    sc = torch.pow(2.0, 13.0 - e)
    return (t * sc).half().float() / sc
