"""CPU tests that pin the oracle (oracle/lora_step.py, oracle/quant.py).

Each check is independent of the formula it checks: torch.autograd, central
finite differences, textbook identities (complex rotation for RoPE, explicit
softmax loops for attention), known answers (ln V for uniform logits,
torch.optim.AdamW), invariants (rows of P sum to 1, dS rows sum to 0,
round trips) and element-wise brute force in float32 scalars for the int8
quantizer.  Planted reference quirks (Q1-Q3) must be caught by the same
checks, which shows the checks can fail.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import lora_step as ref
from oracle.configs import config1, make_adapters, make_layer, make_model
from oracle.quant import dequant, quantize_rows

D64 = torch.float64
TINY = ref.TINY


def g(seed):
    return torch.Generator().manual_seed(seed)


def rel(a, b):
    a, b = a.detach(), b.detach()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


# ------------------------------------------------------------------ RMSNorm

def test_rmsnorm_unit_rms_with_unit_weight():
    x = torch.randn(7, 64, generator=g(1), dtype=D64) * 3.0
    y = ref.rmsnorm(x, torch.ones(64, dtype=D64), 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(7, dtype=D64), atol=1e-12)


def test_rmsnorm_bwd_matches_autograd():
    x = torch.randn(5, 48, generator=g(2), dtype=D64, requires_grad=True)
    w = torch.randn(48, generator=g(3), dtype=D64)
    dy = torch.randn(5, 48, generator=g(4), dtype=D64)
    ref.rmsnorm(x, w, 1e-6).backward(dy)
    dx = ref.rmsnorm_bwd(dy, x.detach(), w, 1e-6)
    assert rel(dx, x.grad) < 1e-12


# ------------------------------------------------------------------ RoPE

def test_rope_is_complex_rotation():
    S, hd = 9, 16
    cos, sin = ref.rope_tables(S, hd, 1e6)
    x = torch.randn(1, S, 3, hd, generator=g(5), dtype=D64)
    y = ref.rope_fwd(x, cos.double(), sin.double())
    # pair (d, d + hd/2) as a complex number rotated by pos * theta^(-2d/hd)
    d = torch.arange(hd // 2, dtype=D64)
    ang = torch.arange(S, dtype=D64)[:, None] * (1e6 ** (-2.0 * d / hd))[None, :]
    z = torch.complex(x[..., : hd // 2], x[..., hd // 2:]) * torch.polar(
        torch.ones_like(ang), ang)[None, :, None, :]
    assert torch.allclose(y[..., : hd // 2], z.real, atol=1e-6)
    assert torch.allclose(y[..., hd // 2:], z.imag, atol=1e-6)


def test_rope_invariants():
    S, hd = 33, 128
    cos, sin = ref.rope_tables(S, hd, 1e6)
    assert torch.equal(cos[0], torch.ones(hd // 2)) and torch.equal(sin[0], torch.zeros(hd // 2))
    assert abs(float(cos[5, 0]) - math.cos(5.0)) < 1e-7  # d = 0: frequency 1
    x = torch.randn(2, S, 4, hd, generator=g(6))
    y = ref.rope_fwd(x, cos, sin)
    assert torch.equal(y[:, 0], x[:, 0])                   # position 0 is the identity
    n_in = x[..., :64] ** 2 + x[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-6)  # pair norms preserved
    assert torch.allclose(ref.rope_bwd(y, cos, sin), x, atol=1e-5)  # inverse round trip


def test_rope_bwd_matches_autograd():
    S, hd = 6, 16
    cos, sin = (t.double() for t in ref.rope_tables(S, hd, 1e4))
    x = torch.randn(1, S, 2, hd, generator=g(7), dtype=D64, requires_grad=True)
    dy = torch.randn(1, S, 2, hd, generator=g(8), dtype=D64)
    ref.rope_fwd(x, cos, sin).backward(dy)
    assert rel(ref.rope_bwd(dy, cos, sin), x.grad) < 1e-12


# ------------------------------------------------------------------ attention

def _attn_loops(q, k, v):
    """Explicit per-(b, head, query) softmax over keys <= query (GQA h -> h//group)."""
    B, S, nq, hd = q.shape
    group = nq // k.shape[2]
    o = torch.zeros_like(q)
    for b in range(B):
        for h in range(nq):
            for i in range(S):
                s = [float(q[b, i, h] @ k[b, j, h // group]) / math.sqrt(hd) for j in range(i + 1)]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                o[b, i, h] = sum(e[j] / z * v[b, j, h // group] for j in range(i + 1))
    return o


def test_attention_fwd_matches_loops_and_lse():
    q = torch.randn(2, 5, 4, 8, generator=g(9), dtype=D64)
    k = torch.randn(2, 5, 2, 8, generator=g(10), dtype=D64)
    v = torch.randn(2, 5, 2, 8, generator=g(11), dtype=D64)
    o, lse = ref.attention_fwd(q, k, v)
    assert rel(o, _attn_loops(q, k, v)) < 1e-12
    # row 0 attends to key 0 only: lse = s_00
    s00 = (q[:, 0] * k[:, 0].repeat_interleave(2, dim=1)).sum(-1) / math.sqrt(8)
    assert torch.allclose(lse[:, :, 0], s00, atol=1e-12)


def test_attention_causality_and_probabilities():
    q = torch.randn(1, 6, 2, 8, generator=g(12), dtype=D64)
    k = torch.randn(1, 6, 1, 8, generator=g(13), dtype=D64)
    v = torch.randn(1, 6, 1, 8, generator=g(14), dtype=D64)
    o, lse = ref.attention_fwd(q, k, v)
    k2, v2 = k.clone(), v.clone()
    k2[:, 4:] += 5.0
    v2[:, 4:] -= 3.0
    o2, _ = ref.attention_fwd(q, k2, v2)
    assert torch.equal(o[:, :4], o2[:, :4])       # queries < 4 never see keys >= 4
    s = torch.einsum("bqhd,bkhd->bhqk", q, k.repeat_interleave(2, dim=2)) / math.sqrt(8)
    s = s.masked_fill(torch.ones(6, 6, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.exp(s - lse[..., None])
    assert torch.allclose(p.sum(-1), torch.ones_like(lse), atol=1e-12)


def test_attention_bwd_matches_autograd_and_invariants():
    q = torch.randn(2, 7, 4, 8, generator=g(15), dtype=D64, requires_grad=True)
    k = torch.randn(2, 7, 2, 8, generator=g(16), dtype=D64, requires_grad=True)
    v = torch.randn(2, 7, 2, 8, generator=g(17), dtype=D64, requires_grad=True)
    do = torch.randn(2, 7, 4, 8, generator=g(18), dtype=D64)
    o, lse = ref.attention_fwd(q, k, v)
    o.backward(do)
    dq, dk, dv = ref.attention_bwd(do, q.detach(), k.detach(), v.detach(), o.detach(), lse)
    assert rel(dq, q.grad) < 1e-10 and rel(dk, k.grad) < 1e-10 and rel(dv, v.grad) < 1e-10
    # shifting every score of a query row leaves P unchanged: sum_j dS_ij = 0,
    # hence sum_j dS_ij k_j-independent -> dq of a constant key shift is 0
    kc = k.detach() + 0.0
    kc[:] = kc[:, :1]  # all keys equal -> P uniform over the causal prefix, dq = 0
    o1, l1 = ref.attention_fwd(q.detach(), kc, v.detach())
    dq1, _, _ = ref.attention_bwd(do, q.detach(), kc, v.detach(), o1, l1)
    assert dq1.abs().max() < 1e-12


def test_attention_bwd_finite_differences():
    q = torch.randn(1, 4, 2, 4, generator=g(19), dtype=D64)
    k = torch.randn(1, 4, 1, 4, generator=g(20), dtype=D64)
    v = torch.randn(1, 4, 1, 4, generator=g(21), dtype=D64)
    do = torch.randn(1, 4, 2, 4, generator=g(22), dtype=D64)
    o, lse = ref.attention_fwd(q, k, v)
    dq, dk, dv = ref.attention_bwd(do, q, k, v, o, lse)
    f = lambda qq, kk, vv: float((ref.attention_fwd(qq, kk, vv)[0] * do).sum())
    h = 1e-6
    for t, grad, idx in ((q, dq, (0, 2, 1, 3)), (k, dk, (0, 1, 0, 2)), (v, dv, (0, 3, 0, 0))):
        tp, tm = t.clone(), t.clone()
        tp[idx] += h
        tm[idx] -= h
        args_p = [tp if x is t else x for x in (q, k, v)]
        args_m = [tm if x is t else x for x in (q, k, v)]
        num = (f(*args_p) - f(*args_m)) / (2 * h)
        assert abs(num - float(grad[idx])) < 1e-7


# ------------------------------------------------------------------ SwiGLU, LoRA

def test_silu_mul_bwd_matches_autograd_and_catches_alias_quirk():
    gg = torch.randn(6, 10, generator=g(23), dtype=D64, requires_grad=True)
    u = torch.randn(6, 10, generator=g(24), dtype=D64, requires_grad=True)
    dy = torch.randn(6, 10, generator=g(25), dtype=D64)
    assert torch.allclose(ref.silu_mul(gg, u), F.silu(gg) * u)
    (F.silu(gg) * u).backward(dy)
    dg, du = ref.silu_mul_bwd(dy, gg.detach(), u.detach())
    assert rel(dg, gg.grad) < 1e-12 and rel(du, u.grad) < 1e-12
    _, du_q = ref.silu_mul_bwd(dy, gg.detach(), u.detach(), alias_quirk=True)
    assert rel(du_q, u.grad) > 0.1  # Q2 (src/kernels/lora_backward.cu:287) is caught


def test_lora_bwd_matches_autograd_and_catches_layout_quirk():
    x = torch.randn(9, 32, generator=g(26), dtype=D64)
    A = torch.randn(16, 32, generator=g(27), dtype=D64, requires_grad=True)
    B = torch.randn(24, 16, generator=g(28), dtype=D64, requires_grad=True)
    xg = x.clone().requires_grad_(True)
    dy = torch.randn(9, 24, generator=g(29), dtype=D64)
    h, y = ref.lora_fwd(xg, A, B, 2.0)
    assert torch.allclose(y, 2.0 * xg @ A.t() @ B.t())
    y.backward(dy)
    dA, dB, dx, _ = ref.lora_bwd(x, h.detach(), dy, A.detach(), B.detach(), 2.0)
    assert rel(dA, A.grad) < 1e-12 and rel(dB, B.grad) < 1e-12 and rel(dx, xg.grad) < 1e-12
    _, _, dx_q, _ = ref.lora_bwd(x, h.detach(), dy, A.detach(), B.detach(), 2.0, dx_quirk=True)
    assert rel(dx_q, xg.grad) > 0.1  # Q1 (src/kernels/lora_backward.cu:87) is caught


# ------------------------------------------------------------------ cross-entropy

def test_cross_entropy_matches_torch():
    S, V = 6, 50
    logits = torch.randn(2 * S, V, generator=g(30), dtype=D64, requires_grad=True)
    tgt = torch.randint(0, V, (2 * S,), generator=g(31))
    valid = ref.valid_rows(2, S)
    assert valid.tolist() == [True] * (S - 1) + [False] + [True] * (S - 1) + [False]
    loss, dl, rows = ref.cross_entropy(logits.detach(), tgt, valid)
    want = F.cross_entropy(logits[valid], tgt[valid])
    assert abs(float(loss) - float(want)) < 1e-12
    want.backward()
    assert rel(dl, logits.grad) < 1e-12
    assert dl[~valid].abs().max() == 0                       # Q4 rows written as zeros
    assert dl[valid].sum(-1).abs().max() < 1e-15             # softmax minus one-hot
    assert torch.allclose(rows, F.cross_entropy(logits.detach(), tgt, reduction="none"))


def test_cross_entropy_known_answer_full_vocab():
    V, S = 151936, 4
    loss, dl, _ = ref.cross_entropy(torch.zeros(S, V), torch.tensor([0, 5, 151935, 7]),
                                    ref.valid_rows(1, S))
    assert abs(float(loss) - 11.93122) < 1e-5               # ln 151936
    assert abs(float(dl[1, 5]) - (1 / V - 1) / 3) < 1e-7      # fp32: one ulp at 1/3


# ------------------------------------------------------------------ AdamW

@pytest.mark.parametrize("steps", [1, 3])
def test_adamw_matches_torch_optim(steps):
    p0 = torch.randn(40, generator=g(32), dtype=D64)
    p = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([p], lr=3e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    q, m, v = p0.clone(), torch.zeros(40, dtype=D64), torch.zeros(40, dtype=D64)
    for t in range(1, steps + 1):
        grad = torch.randn(40, generator=g(100 + t), dtype=D64)
        p.grad = grad.clone()
        opt.step()
        q, m, v = ref.adamw(q, grad, m, v, 3e-4, 0.9, 0.999, 1e-8, 0.01, t)
    # The oracle forms the bias corrections in fp32 like the reference (powf,
    # src/kernels/lora.cu:238-239): 1 - 0.999f = 1.0000467e-3, a 5e-5 relative
    # change of v_hat.  Compare the updates with a tolerance above that.
    du, dt = q - p0, p.detach() - p0
    assert float((du - dt).norm() / dt.norm()) < 1e-4


def test_adamw_first_step_is_signed_lr():
    p = torch.randn(30, generator=g(33))
    grad = torch.randn(30, generator=g(34))
    q, _, _ = ref.adamw(p, grad, torch.zeros(30), torch.zeros(30), 3e-4, 0.9, 0.999, 1e-8, 0.01, 1)
    assert torch.allclose(q, p * (1 - 3e-6) - 3e-4 * torch.sign(grad), atol=1e-8)


# ------------------------------------------------------------------ layer / model

def _adapters64(ad):
    return [{p: ref.Adapter(a.A.double(), a.B.double()) for p, a in d.items()} for d in ad]


def _model64(W):
    f = lambda t: t.double()
    layers = [ref.LayerW(**{k: f(getattr(l, k)) for k in l.__dataclass_fields__}) for l in W.layers]
    return ref.ModelW(embed=f(W.embed), layers=layers, final_norm=f(W.final_norm),
                      lm_head=f(W.lm_head))


def test_layer_backward_matches_autograd():
    gen = g(35)
    lw = make_layer(gen, TINY, wdtype=torch.float32)
    lw = ref.LayerW(**{k: getattr(lw, k).double() for k in lw.__dataclass_fields__})
    ad = _adapters64(make_adapters(gen, TINY))[0]
    B, S = 2, 5
    cos, sin = (t.double() for t in ref.rope_tables(S, TINY.head_dim, TINY.theta))
    x = torch.randn(B * S, TINY.hidden, generator=gen, dtype=D64, requires_grad=True)
    leaves = {p: (ad[p].A.clone().requires_grad_(True), ad[p].B.clone().requires_grad_(True))
              for p in ref.PROJS}
    adg = {p: ref.Adapter(*leaves[p]) for p in ref.PROJS}
    y, _ = ref.layer_forward(x, lw, adg, TINY, B, S, cos, sin)
    dy = torch.randn(B * S, TINY.hidden, generator=gen, dtype=D64)
    y.backward(dy)
    _, st = ref.layer_forward(x.detach(), lw, ad, TINY, B, S, cos, sin)
    dx, grads = ref.layer_backward(dy, st, lw, ad, TINY, B, S, cos, sin)
    assert rel(dx, x.grad) < 1e-10
    for p in ref.PROJS:
        assert rel(grads[p][0], leaves[p][0].grad) < 1e-10
        assert rel(grads[p][1], leaves[p][1].grad) < 1e-10


@pytest.fixture(scope="module")
def tiny_step():
    gen = g(36)
    W = _model64(make_model(gen, TINY))
    ad = _adapters64(make_adapters(gen, TINY))
    win = torch.randint(0, TINY.vocab, (2, 9), generator=gen)
    return W, ad, win[:, :-1], win[:, 1:]


def test_model_backward_matches_autograd(tiny_step):
    W, ad, tok, tgt = tiny_step
    loss_a, grads_a = ref.step_autograd(W, ad, tok, tgt, TINY)
    logits, stash = ref.model_forward(W, ad, tok, TINY)
    loss, dl, _ = ref.cross_entropy(logits, tgt.reshape(-1), ref.valid_rows(2, 8))
    grads, _ = ref.model_backward(dl, stash, W, ad, TINY, 2, 8)
    assert abs(float(loss) - float(loss_a)) < 1e-12
    for l in range(TINY.n_layers):
        for p in ref.PROJS:
            assert rel(grads[l][p][0], grads_a[l][p][0]) < 1e-9
            assert rel(grads[l][p][1], grads_a[l][p][1]) < 1e-9


def test_model_backward_finite_differences(tiny_step):
    W, ad, tok, tgt = tiny_step
    valid = ref.valid_rows(2, 8)

    def loss_of(adp):
        logits, _ = ref.model_forward(W, adp, tok, TINY)
        return float(ref.cross_entropy(logits, tgt.reshape(-1), valid)[0])

    logits, stash = ref.model_forward(W, ad, tok, TINY)
    _, dl, _ = ref.cross_entropy(logits, tgt.reshape(-1), valid)
    grads, _ = ref.model_backward(dl, stash, W, ad, TINY, 2, 8)
    h = 1e-6
    for l, p, which, idx in ((0, "wq", 0, (3, 7)), (1, "wo", 1, (11, 2)), (0, "wv", 1, (5, 0))):
        a2 = [{q: ref.Adapter(x.A.clone(), x.B.clone()) for q, x in d.items()} for d in ad]
        a3 = [{q: ref.Adapter(x.A.clone(), x.B.clone()) for q, x in d.items()} for d in ad]
        t2 = a2[l][p].A if which == 0 else a2[l][p].B
        t3 = a3[l][p].A if which == 0 else a3[l][p].B
        t2[idx] += h
        t3[idx] -= h
        num = (loss_of(a2) - loss_of(a3)) / (2 * h)
        assert abs(num - float(grads[l][p][which][idx])) < 1e-7 * max(1.0, abs(num)) + 1e-9


def test_final_norm_quirk_is_caught(tiny_step):
    W, ad, tok, tgt = tiny_step
    _, grads_a = ref.step_autograd(W, ad, tok, tgt, TINY)
    logits, stash = ref.model_forward(W, ad, tok, TINY)
    _, dl, _ = ref.cross_entropy(logits, tgt.reshape(-1), ref.valid_rows(2, 8))
    grads_q, _ = ref.model_backward(dl, stash, W, ad, TINY, 2, 8, quirks=("final_norm",))
    assert rel(grads_q[1]["wq"][1], grads_a[1]["wq"][1]) > 1e-3  # Q3 is caught


def test_train_step_updates_adapters(tiny_step):
    W, ad, tok, tgt = tiny_step
    ad2 = [{q: ref.Adapter(x.A.clone(), x.B.clone()) for q, x in d.items()} for d in ad]
    loss, grads, _ = ref.train_step(W, ad2, tok, tgt, TINY, step=1)
    for l in range(TINY.n_layers):
        for p in ref.PROJS:
            want, _, _ = ref.adamw(ad[l][p].A, grads[l][p][0], 0 * ad[l][p].A, 0 * ad[l][p].A,
                                   3e-4, 0.9, 0.999, 1e-8, 0.01, 1)
            assert torch.allclose(ad2[l][p].A, want)


# ------------------------------------------------------------------ int8 quantizer

def _quantize_scalar(row):
    """Element-wise float32 scalar arithmetic (src/kernels/quantize.cu:30-40)."""
    f32 = np.float32
    amax = f32(0)
    for w in row:
        amax = max(amax, abs(f32(w)))
    scale = f32(amax / f32(127))
    inv = f32(f32(1) / scale) if scale > 0 else f32(0)
    out = []
    for w in row:
        v = f32(f32(w) * inv)
        v = min(max(v, f32(-127)), f32(127))
        out.append(int(np.rint(v)))
    return np.array(out, dtype=np.int8), scale


def test_quantize_bit_exact_brute_force():
    rng = np.random.default_rng(37)
    w = (rng.standard_normal((6, 96)) * 0.02).astype(np.float32)
    w[1] = 0.0
    w[2, :5] = [127.0, 0.5, 1.5, -2.5, 2.5]   # w*inv = 127, .5, 1.5, -2.5, 2.5 exactly
    q, s = quantize_rows(w)
    for r in range(6):
        qr, sr = _quantize_scalar(w[r])
        assert np.array_equal(q[r], qr) and s[r].view(np.uint32) == np.float32(sr).view(np.uint32)
    assert q[2, :5].tolist() == [127, 0, 2, -2, 2]  # round half to even
    assert (q[1] == 0).all() and s[1] == 0
    assert np.abs(dequant(q, s) - w).max() <= s.max() / 2 + 1e-9


# ------------------------------------------------------------------ configs

def test_configs_are_seeded_and_shaped():
    x1, W1, t1 = config1(vocab=1024, hidden=64, rows=8)
    x2, W2, t2 = config1(vocab=1024, hidden=64, rows=8)
    assert torch.equal(W1, W2) and torch.equal(t1, t2) and x1.dtype == torch.float16
    ad = make_adapters(g(38), ref.Dims(hidden=2048, n_layers=1, n_heads=16, n_kv_heads=8,
                                       head_dim=128, intermediate=64, vocab=64))
    A = ad[0]["wq"].A
    assert abs(float(A.std()) - 2048 ** -0.5) < 2e-3  # N(0, 1/2048) read as variance
