"""GPU parity of the benchmark configurations C0-C4 against the
exact fp32 CPU oracle, through the C ABI.

Tolerances (north star): loss within 1e-3 absolute; every gradient tensor
within 1e-2 relative L2; integer work bit-exact.  C2 is checked at full size
(28 layers, vocabulary 151936, batch 1 x seq 128); C4 at full width with
2 layers and B2 x S256 against the oracle, and at full size through
size-independent properties (finite, loss near ln V, bit-identical reruns)."""
import math

import numpy as np
import pytest
import torch

import llmt
from helpers import grad_errors, oracle_grads, rel_l2, upload_model
from oracle import lora_step as ref
from oracle.configs import config0, config1, config3, config_model

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-3
GRAD_TOL = 1e-2
Q3 = ref.QWEN3_1_7B


@pytest.fixture(scope="module")
def c2(dev):
    torch.set_num_threads(16)
    print("case: C2 full model, seed 1002, B1 x S128", flush=True)
    W, ad, tok, tgt, _ = config_model(Q3, 1, 128, 1002)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, Q3)
    return dict(W=W, ad=ad, tok=tok, tgt=tgt, loss_ref=float(loss_ref), grads_ref=grads_ref)


def test_c2_full_step_parity(c2, dev):
    ctx = llmt.Context(llmt.make_dims(Q3), 1, 128)
    try:
        upload_model(ctx, c2["W"], dev)
        ctx.lora_set("param", llmt.flatten_adapters(c2["ad"]).to(dev))
        loss = ctx.forward_backward(c2["tok"].to(dev), c2["tgt"].to(dev))
        print(f"C2 loss {loss:.6f} oracle {c2['loss_ref']:.6f}", flush=True)
        assert abs(loss - c2["loss_ref"]) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), c2["grads_ref"], Q3)
        worst = max(errs.items(), key=lambda kv: kv[1])
        print("C2 worst grad rel-L2", worst, flush=True)
        assert worst[1] < GRAD_TOL
        # the step through a captured graph: same loss, then AdamW
        ctx.set_graph(True)
        loss_g = ctx.step(c2["tok"].to(dev), c2["tgt"].to(dev), llmt.hparams(), 1)
        assert loss_g == loss
    finally:
        ctx.close()


# ------------------------------------------------------------------ compat layer

import ctypes as C


class LoraAdapterC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("A", "B", "mA", "vA", "mB", "vB")] + \
               [("d_in", C.c_int), ("d_out", C.c_int)]


class LoraWeightsC(C.Structure):
    _fields_ = [(p, LoraAdapterC * 28) for p in ("wq", "wk", "wv", "wo")]


class LoraGradC(C.Structure):
    _fields_ = [("dA", C.c_void_p), ("dB", C.c_void_p)]


class LoraGradsC(C.Structure):
    _fields_ = [(p, LoraGradC * 28) for p in ("wq", "wk", "wv", "wo")]


class LoraActsC(C.Structure):
    _fields_ = [(n, C.c_void_p * 28) for n in (
        "layer_in", "attn_norm_out", "q_raw", "k_raw", "q_rope", "k_rope", "v_raw", "attn_w",
        "pre_o", "post_attn", "ffn_norm_out", "gate_raw", "up_raw", "hq", "hk", "hv", "ho")]


class LWC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "q_norm",
                                          "k_norm", "w_gate", "w_up", "w_down")] + \
               [("_pad", C.c_void_p * 21)]


class MWC(C.Structure):
    _fields_ = [("embed_table", C.c_void_p), ("layers", LWC * 28), ("final_norm", C.c_void_p),
                ("lm_head", C.c_void_p), ("_pad", C.c_void_p * 3)]


def test_compat_struct_sizes():
    assert C.sizeof(LWC) == 32 * 8 and C.sizeof(LoraAdapterC) == 56
    assert C.sizeof(MWC) == 8 * (1 + 32 * 28 + 5)


def _compat_bind():
    L = llmt.lib()
    L.lora_weights_init.argtypes = [C.POINTER(LoraWeightsC)]
    L.lora_grads_alloc.argtypes = [C.POINTER(LoraGradsC), C.POINTER(LoraWeightsC)]
    L.lora_grads_zero.argtypes = [C.POINTER(LoraGradsC)]
    L.lora_acts_alloc.argtypes = [C.POINTER(LoraActsC), C.c_int]
    L.transformer_forward_lora.argtypes = [C.c_void_p, C.POINTER(MWC), C.POINTER(LoraWeightsC)] + \
        [C.c_void_p] * 12 + [C.POINTER(LoraActsC), C.c_int]
    L.cross_entropy_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
    L.cross_entropy_forward.restype = C.c_float
    L.transformer_backward_lora.argtypes = [C.c_void_p, C.POINTER(MWC), C.POINTER(LoraWeightsC),
                                            C.POINTER(LoraActsC), C.POINTER(LoraGradsC)] + \
        [C.c_void_p] * 14 + [C.c_int]
    L.adamw_step_lora.argtypes = [C.POINTER(LoraWeightsC), C.POINTER(LoraGradsC)] + \
        [C.c_float] * 5 + [C.c_int]
    L.lora_weights_free.argtypes = [C.POINTER(LoraWeightsC)]
    L.lora_grads_free.argtypes = [C.POINTER(LoraGradsC)]
    return L


def _compat_step(L, mw, ad, tok, tgt, S, dev):
    """One forward / CE / backward through the reference's call sequence
    (src/train.cu:261-287) with library-allocated adapters holding `ad`.
    Returns (loss, dlogits, grads[l][proj] = (dA, dB) on the CPU, lora, grads)."""
    lora = LoraWeightsC()
    L.lora_weights_init(C.byref(lora))
    for l in range(len(ad)):
        for p in ref.PROJS:
            a = getattr(lora, p)[l]
            for addr, t in ((a.A, ad[l][p].A), (a.B, ad[l][p].B)):
                _ptr_tensor(addr, t.numel(), dev).copy_(t.reshape(-1).float().to(dev))
    grads = LoraGradsC()
    L.lora_grads_alloc(C.byref(grads), C.byref(lora))
    acts = LoraActsC()
    L.lora_acts_alloc(C.byref(acts), S)
    tokd = tok.reshape(-1).to(dev)
    tgtd = tgt.reshape(-1).to(dev)
    logits = torch.full((S, Q3.vocab), float("nan"), device=dev)
    dlogits = torch.full((S, Q3.vocab), float("nan"), device=dev)
    ws = [torch.empty(1, device=dev) for _ in range(15)]
    torch.cuda.synchronize()
    L.transformer_forward_lora(tokd.data_ptr(), C.byref(mw), C.byref(lora),
                               *[w.data_ptr() for w in ws[:11]], logits.data_ptr(), C.byref(acts), S)
    loss = L.cross_entropy_forward(logits.data_ptr(), tgtd.data_ptr(), dlogits.data_ptr(), S)
    L.lora_grads_zero(C.byref(grads))
    L.transformer_backward_lora(dlogits.data_ptr(), C.byref(mw), C.byref(lora), C.byref(acts),
                                C.byref(grads), *[w.data_ptr() for w in ws[:14]], S)
    torch.cuda.synchronize()
    out = []
    for l in range(len(ad)):
        d = {}
        for p in ref.PROJS:
            gg = getattr(grads, p)[l]
            nA, nB = ad[l][p].A.numel(), ad[l][p].B.numel()
            d[p] = (_ptr_tensor(gg.dA, nA, dev).cpu().view_as(ad[l][p].A),
                    _ptr_tensor(gg.dB, nB, dev).cpu().view_as(ad[l][p].B))
        out.append(d)
    return loss, dlogits, out, lora, grads


def _worst(got, want):
    return max(max(rel_l2(got[l][p][0], want[l][p][0]), rel_l2(got[l][p][1], want[l][p][1]))
               for l in range(len(want)) for p in ref.PROJS)


def test_compat_reference_api_matches_oracle(c2, dev):
    """The reference's own step API (src/train.cu:261-287 call sequence) with
    fp16 weights in the MW pad slots (src/main.cu:40-55 map)."""
    L = _compat_bind()
    W, S = c2["W"], 128
    keep = []

    def dev16(t):
        x = t.to(torch.float16).to(dev).contiguous()
        keep.append(x)
        return x.data_ptr()

    def dev32(t):
        x = t.to(torch.float32).to(dev).contiguous()
        keep.append(x)
        return x.data_ptr()

    mw = MWC()
    for l, lw in enumerate(W.layers):
        d = mw.layers[l]
        d.attn_norm, d.ffn_norm = dev32(lw.attn_norm), dev32(lw.ffn_norm)
        d.q_norm, d.k_norm = dev32(lw.q_norm), dev32(lw.k_norm)
        for i, name in enumerate(("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")):
            d._pad[i] = dev16(getattr(lw, name))
    mw._pad[0] = dev16(W.embed)
    mw.final_norm = dev32(W.final_norm)
    loss, dlogits, got, lora, grads = _compat_step(L, mw, c2["ad"], c2["tok"], c2["tgt"], S, dev)
    assert abs(loss - c2["loss_ref"]) < LOSS_TOL
    assert float(dlogits[-1].abs().max()) == 0.0       # Q4: last row written as zeros
    worst = _worst(got, c2["grads_ref"])
    print("compat worst grad rel-L2", worst, flush=True)
    assert worst < GRAD_TOL
    L.adamw_step_lora(C.byref(lora), C.byref(grads), 3e-4, 0.9, 0.999, 1e-8, 0.01, 1)
    torch.cuda.synchronize()
    a0 = lora.wq[0]
    got = _ptr_tensor(a0.A, 16 * 2048, dev).cpu().view(16, 2048)
    want, _, _ = ref.adamw(c2["ad"][0]["wq"].A, c2["grads_ref"][0]["wq"][0], torch.zeros(16, 2048),
                           torch.zeros(16, 2048), 3e-4, 0.9, 0.999, 1e-8, 0.01, 1)
    assert rel_l2(got, want) < GRAD_TOL
    L.lora_grads_free(C.byref(grads))
    L.lora_weights_free(C.byref(lora))


def test_compat_int8_pads_ragged_seq_matches_oracle(dev):
    """The reference API with int8 frozen weights in the LW pad slots
    _pad[7..20] (int8 values, float* row scales: src/main.cu:49-55), the
    embedding as the fp32 embed_table and the lm_head as the MW int8 pair
    _pad[1..2] (src/main.cu:64), at a sequence length that is not a multiple
    of 16 (seq 100, src/train.cu:176,187).  Against the oracle on the
    dequantised weights (fp16 scales of the C4 recipe; the head as fp16
    q * scale)."""
    import numpy as np
    from oracle.quant import dequant, quantize_rows
    torch.set_num_threads(16)
    S = 100
    print("case: compat API, int8 pads, full model, B1 x S100", flush=True)
    W, ad, tok, tgt, qs = config_model(Q3, 1, S, 1005, int8=True)
    hq, hs = quantize_rows(W.embed.numpy())
    W.lm_head = torch.from_numpy(dequant(hq, hs)).half().float()
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, Q3)
    L = _compat_bind()
    keep = []

    def put(a):
        x = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        keep.append(x)
        return x.data_ptr()

    def dev32(t):
        x = t.to(torch.float32).to(dev).contiguous()
        keep.append(x)
        return x.data_ptr()

    mw = MWC()
    for l, lw in enumerate(W.layers):
        d = mw.layers[l]
        d.attn_norm, d.ffn_norm = dev32(lw.attn_norm), dev32(lw.ffn_norm)
        d.q_norm, d.k_norm = dev32(lw.q_norm), dev32(lw.k_norm)
        for i, name in enumerate(("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")):
            q, s16 = qs[(l, name)]
            d._pad[7 + 2 * i] = put(q)
            d._pad[8 + 2 * i] = put(s16.astype(np.float32))
    mw.embed_table = dev32(W.embed)
    mw._pad[1] = put(hq)
    mw._pad[2] = put(hs.astype(np.float32))
    mw.final_norm = dev32(W.final_norm)
    loss, dlogits, got, lora, grads = _compat_step(L, mw, ad, tok, tgt, S, dev)
    print(f"compat int8 S{S}: loss {loss:.6f} oracle {float(loss_ref):.6f}", flush=True)
    assert abs(loss - float(loss_ref)) < LOSS_TOL
    assert float(dlogits[-1].abs().max()) == 0.0
    assert torch.isfinite(dlogits).all()
    worst = _worst(got, grads_ref)
    print("compat int8 worst grad rel-L2", worst, flush=True)
    assert worst < GRAD_TOL
    L.lora_grads_free(C.byref(grads))
    L.lora_weights_free(C.byref(lora))


def _ptr_tensor(addr, n, dev):
    """A float32 torch view of n floats at device address addr."""
    class _Holder:
        __cuda_array_interface__ = {"shape": (n,), "typestr": "<f4", "data": (addr, False),
                                    "version": 3, "strides": None}
    return torch.as_tensor(_Holder(), device=dev)


# ------------------------------------------------------------------ C0

def test_c0_single_layer(dev):
    print("case: C0 one layer fp32 weights, B1 x S128", flush=True)
    d1, lw, ad, x, dy = config0()
    cos, sin = ref.rope_tables(128, d1.head_dim, d1.theta)
    y_ref, st = ref.layer_forward(x, lw, ad, d1, 1, 128, cos, sin)
    dx_ref, grads_ref = ref.layer_backward(dy, st, lw, ad, d1, 1, 128, cos, sin)
    ctx = llmt.Context(llmt.make_dims(d1), 1, 128)
    try:
        h = lambda t: t.to(torch.float16).to(dev).contiguous()
        f = lambda t: t.to(torch.float32).to(dev).contiguous()
        ctx.set_layer_f16(0, h(lw.wq), h(lw.wk), h(lw.wv), h(lw.wo), h(lw.w_gate), h(lw.w_up),
                          h(lw.w_down), f(lw.attn_norm), f(lw.ffn_norm), f(lw.q_norm), f(lw.k_norm))
        ctx.lora_set("param", llmt.flatten_adapters([ad]).to(dev))
        y = ctx.layer_forward(0, x.to(dev), 1)
        assert rel_l2(y.cpu(), y_ref) < GRAD_TOL
        dx = ctx.layer_backward(0, dy.to(dev), 1)
        assert rel_l2(dx.cpu(), dx_ref) < GRAD_TOL
        errs = grad_errors(ctx.lora_get("grad"), [grads_ref], d1)
        print("C0 worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


def test_c0_single_layer_int8(dev):
    """C0's layer on int8 weights through llmt_layer_forward /
    llmt_layer_backward: the layer API's input-gradient rows (grad_rows) carry
    the down projection's per-k weight scale into the down dX operand; output,
    input gradient and adapter gradients against the oracle on the
    dequantised weights."""
    from oracle.quant import quantize_rows
    print("case: C0 one layer int8 weights, B1 x S128 (layer API)", flush=True)
    d1, lw, ad, x, dy = config0()
    names = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
    qs = {}
    for n in names:
        q, sc = quantize_rows(getattr(lw, n).float().numpy())
        sc16 = sc.astype(np.float16)
        qs[n] = (q, sc16)
        setattr(lw, n, torch.from_numpy(q.astype(np.float32) * sc16.astype(np.float32)[:, None]))
    cos, sin = ref.rope_tables(128, d1.head_dim, d1.theta)
    y_ref, st = ref.layer_forward(x, lw, ad, d1, 1, 128, cos, sin)
    dx_ref, grads_ref = ref.layer_backward(dy, st, lw, ad, d1, 1, 128, cos, sin)
    ctx = llmt.Context(llmt.make_dims(d1), 1, 128, int8=True)
    try:
        f = lambda t: t.to(torch.float32).to(dev).contiguous()
        ctx.set_layer_i8(0, [torch.from_numpy(qs[n][0]).to(dev) for n in names],
                         [torch.from_numpy(qs[n][1]).to(dev) for n in names],
                         f(lw.attn_norm), f(lw.ffn_norm), f(lw.q_norm), f(lw.k_norm))
        ctx.lora_set("param", llmt.flatten_adapters([ad]).to(dev))
        y = ctx.layer_forward(0, x.to(dev), 1)
        assert rel_l2(y.cpu(), y_ref) < GRAD_TOL
        dx = ctx.layer_backward(0, dy.to(dev), 1)
        assert rel_l2(dx.cpu(), dx_ref) < GRAD_TOL
        errs = grad_errors(ctx.lora_get("grad"), [grads_ref], d1)
        print("C0 int8 worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


# ------------------------------------------------------------------ C1

@pytest.mark.parametrize("via_ctx", [False, True])
def test_c1_head_ce(dev, via_ctx):
    print(f"case: C1 lm_head + CE, ctx={via_ctx}", flush=True)
    x, W, tgt = config1()
    S = 128
    logits = x.float() @ W.float().t()
    valid = ref.valid_rows(1, S)
    loss_ref, dl_ref, _ = ref.cross_entropy(logits, tgt, valid)
    dh_ref = dl_ref @ W.float()
    if via_ctx:
        d = ref.Dims(n_layers=1)
        ctx = llmt.Context(llmt.make_dims(d), 1, S)
        try:
            ctx.set_embed_f16(W.to(dev), torch.ones(2048, device=dev))
            loss, dl, dh = ctx.head_ce(x.to(dev), tgt.to(dev), want_dlogits=True)
        finally:
            ctx.close()
    else:
        lm, dl, dh = llmt.lm_head_ce(x.to(dev), W.to(dev), tgt.to(dev), S)
        loss = float(lm)
    assert abs(loss - float(loss_ref)) < LOSS_TOL
    assert rel_l2(dl.cpu(), dl_ref) < GRAD_TOL
    assert float(dl[-1].abs().max()) == 0.0
    assert rel_l2(dh.cpu(), dh_ref) < GRAD_TOL


# ------------------------------------------------------------------ C3

def _attn_block_ref(q_raw, k_raw, v, do, eps=1e-6, theta=1e6):
    """Oracle: QK-RMSNorm (weights 1) + RoPE + causal GQA attention fwd/bwd,
    returning gradients w.r.t. q_raw, k_raw, v (fp32 on the CPU)."""
    B, S, nq, hd = q_raw.shape
    cos, sin = ref.rope_tables(S, hd, theta)
    w = torch.ones(hd)
    qr, kr, vv, dd = (t.float() for t in (q_raw, k_raw, v, do))
    qn = ref.rope_fwd(ref.rmsnorm(qr, w, eps), cos, sin)
    kn = ref.rope_fwd(ref.rmsnorm(kr, w, eps), cos, sin)
    o, lse = ref.attention_fwd(qn, kn, vv)
    dq, dk, dv = ref.attention_bwd(dd, qn, kn, vv, o, lse)
    dq = ref.rmsnorm_bwd(ref.rope_bwd(dq, cos, sin), qr, w, eps)
    dk = ref.rmsnorm_bwd(ref.rope_bwd(dk, cos, sin), kr, w, eps)
    return dq, dk, dv


@pytest.mark.parametrize("B,S", [(4, 2048), (1, 200)])
def test_c3_attention_block(dev, B, S):
    print(f"case: C3 attention block B{B} S{S}", flush=True)
    q, k, v, do = config3(batch=B, seq_len=S)
    dq_ref, dk_ref, dv_ref = _attn_block_ref(q, k, v, do)
    one = torch.ones(128, device=dev)
    dq, dk, dv = llmt.attention_block_bwd(q.to(dev), k.to(dev), v.to(dev), one, one, do.to(dev))
    for got, want in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        assert torch.isfinite(got).all()
        assert rel_l2(got.cpu(), want) < GRAD_TOL


@pytest.mark.parametrize("B,S,nq,nkv", [(2, 256, 16, 8), (1, 77, 4, 1), (3, 64, 2, 2)])
def test_attention_fwd_bwd(dev, B, S, nq, nkv):
    g = torch.Generator().manual_seed(S + nq)
    q = torch.randn(B, S, nq, 128, generator=g).half()
    k = torch.randn(B, S, nkv, 128, generator=g).half()
    v = torch.randn(B, S, nkv, 128, generator=g).half()
    do = torch.randn(B, S, nq, 128, generator=g) * 1e-3   # small dO: exercises the dO scale
    o_ref, lse_ref = ref.attention_fwd(q.float(), k.float(), v.float())
    o, lse = llmt.attention_fwd(q.to(dev), k.to(dev), v.to(dev))
    assert rel_l2(o.float().cpu(), o_ref) < 2e-3
    assert (lse.cpu() - lse_ref).abs().max() < 1e-3
    dq_ref, dk_ref, dv_ref = ref.attention_bwd(do, q.float(), k.float(), v.float(),
                                               o.float().cpu(), lse.cpu())
    dq, dk, dv = llmt.attention_bwd(q.to(dev), k.to(dev), v.to(dev), o, lse, do.to(dev))
    for got, want in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        assert rel_l2(got.cpu(), want) < GRAD_TOL


@pytest.mark.parametrize("mode", ["pow2_rows", "zero_rows", "zero_batch"])
def test_attention_bwd_row_scales(dev, mode):
    """dO reaches the backward as fp16 rows each scaled by its own power of
    two.  dQ row i depends on dO row i only and is computed in that row's
    scale: rows multiplied by 2^e (e from -30 to 2) give dQ rows exactly 2^e
    times those of the unscaled dO (bit-exact).  dK and dV mix rows at the
    batch's common scale (checked against the oracle).  All-zero rows and an
    all-zero batch stay finite and give exact zeros where the mathematics
    does."""
    B, S, nq, nkv = 2, 96, 4, 2
    g = torch.Generator().manual_seed(31)
    q = torch.randn(B, S, nq, 128, generator=g).half()
    k = torch.randn(B, S, nkv, 128, generator=g).half()
    v = torch.randn(B, S, nkv, 128, generator=g).half()
    do = torch.randn(B, S, nq, 128, generator=g)
    mag = 2.0 ** (torch.arange(S) % 33 - 30).float()
    if mode == "pow2_rows":
        do_run = do * mag[None, :, None, None]
    elif mode == "zero_rows":
        do_run = do.clone()
        do_run[:, ::3] = 0.0
    else:
        do_run = do.clone()
        do_run[1] = 0.0
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o, lse = llmt.attention_fwd(qd, kd, vd)
    dq_ref, dk_ref, dv_ref = ref.attention_bwd(do_run, q.float(), k.float(), v.float(),
                                               o.float().cpu(), lse.cpu())
    dq, dk, dv = (t.cpu() for t in llmt.attention_bwd(qd, kd, vd, o, lse, do_run.to(dev)))
    for got, want in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        assert torch.isfinite(got).all()
        assert rel_l2(got, want) < GRAD_TOL
    if mode == "pow2_rows":
        dq1 = llmt.attention_bwd(qd, kd, vd, o, lse, do.to(dev))[0].cpu()
        assert torch.equal(dq, dq1 * mag[None, :, None, None])
    elif mode == "zero_rows":
        assert (dq[:, ::3] == 0).all()
    else:
        assert (dq[1] == 0).all() and (dk[1] == 0).all() and (dv[1] == 0).all()


@pytest.mark.parametrize("cfg,dkdv", [("2,1", "2"), ("2,2", "4"), ("4,1", "4"), ("4,2", "2")])
@pytest.mark.parametrize("B,S,nq,nkv", [(1, 200, 4, 2), (2, 128, 2, 1)])
def test_attention_launch_shapes(dev, monkeypatch, cfg, dkdv, B, S, nq, nkv):
    """Every workgroup shape of the attention kernels (waves x 16-row tiles
    per wave for the forward and dQ, waves for dK/dV) against the oracle."""
    monkeypatch.setenv("LLMT_ATTN_CFG", cfg)
    monkeypatch.setenv("LLMT_ATTN_DKDV_WAVES", dkdv)
    print(f"case: attention shape {cfg}/{dkdv} B{B} S{S} nq{nq} nkv{nkv}", flush=True)
    g = torch.Generator().manual_seed(7 * S + nq)
    q = torch.randn(B, S, nq, 128, generator=g).half()
    k = torch.randn(B, S, nkv, 128, generator=g).half()
    v = torch.randn(B, S, nkv, 128, generator=g).half()
    do = torch.randn(B, S, nq, 128, generator=g)
    o_ref, lse_ref = ref.attention_fwd(q.float(), k.float(), v.float())
    o, lse = llmt.attention_fwd(q.to(dev), k.to(dev), v.to(dev))
    assert rel_l2(o.float().cpu(), o_ref) < 2e-3
    assert (lse.cpu() - lse_ref).abs().max() < 1e-3
    dq_ref, dk_ref, dv_ref = ref.attention_bwd(do, q.float(), k.float(), v.float(),
                                               o.float().cpu(), lse.cpu())
    dq, dk, dv = llmt.attention_bwd(q.to(dev), k.to(dev), v.to(dev), o, lse, do.to(dev))
    for got, want in ((dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        assert rel_l2(got.cpu(), want) < GRAD_TOL


# ------------------------------------------------------------------ C4 (int8 weights)

def _upload_i8(ctx, W, qs, dev):
    f = lambda t: t.to(torch.float32).to(dev).contiguous()
    for l, lw in enumerate(W.layers):
        names = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
        q8 = [torch.from_numpy(qs[(l, n)][0]).to(dev) for n in names]
        s16 = [torch.from_numpy(qs[(l, n)][1]).to(dev) for n in names]
        ctx.set_layer_i8(l, q8, s16, f(lw.attn_norm), f(lw.ffn_norm), f(lw.q_norm), f(lw.k_norm))
    ctx.set_embed_f16(W.embed.half().to(dev), f(W.final_norm))


def test_c4_int8_reduced_matches_oracle(dev):
    """C4's int8 path (fused dequant in every frozen GEMM) at full width,
    2 layers, B2 x S256, against the oracle on the dequantised weights."""
    print("case: C4 reduced (2 layers, B2 S256, int8)", flush=True)
    d = ref.Dims(n_layers=2)
    W, ad, tok, tgt, qs = config_model(d, batch=2, seq_len=256, seed=1004, int8=True)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, d)
    ctx = llmt.Context(llmt.make_dims(d), 2, 256, int8=True)
    try:
        _upload_i8(ctx, W, qs, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, d)
        print("C4-reduced worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


def test_gqa_8_4_heads_t128_matches_oracle(dev):
    """Full width with 8 query / 4 KV heads at B1 x S128: the Q/K/V GEMM
    (N = 2096) takes four split partials, so qkv_post's four-split form runs
    (C2's own shapes give it two); loss and every adapter gradient against
    the oracle (vocabulary 8192 keeps the CPU oracle to seconds)."""
    print("case: H 2048, 8/4 heads, 2 layers, B1 S128, V 8192", flush=True)
    d = ref.Dims(n_layers=2, n_heads=8, n_kv_heads=4, vocab=8192)
    W, ad, tok, tgt, _ = config_model(d, batch=1, seq_len=128, seed=1021)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, d)
    ctx = llmt.Context(llmt.make_dims(d), 1, 128)
    try:
        upload_model(ctx, W, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, d)
        print("8/4 heads worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


def test_c4_int8_large_tile_full_width_matches_oracle(dev):
    """C4's token count (B8 x S512 = 4096 rows) on the large-tile path
    (gemm_dma_kernel with per-row and per-k int8 scales, the fused SwiGLU
    epilogue at N = 2 x 6144, LoRA tail columns, the fp16 logits GEMM) at full
    width with 2 layers; vocabulary 8192 keeps the CPU oracle to seconds."""
    print("case: C4 T=4096 full width, 2 layers, V 8192, int8", flush=True)
    torch.set_num_threads(16)
    d = ref.Dims(n_layers=2, vocab=8192)
    W, ad, tok, tgt, qs = config_model(d, batch=8, seq_len=512, seed=1014, int8=True)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, d)
    ctx = llmt.Context(llmt.make_dims(d), 8, 512, int8=True)
    try:
        _upload_i8(ctx, W, qs, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        print(f"C4 T=4096: loss {loss:.6f} oracle {float(loss_ref):.6f}", flush=True)
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, d)
        print("C4 T=4096 worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


def test_logits_gemm_full_size(dev):
    """The C4 logits GEMM shape, M = 4096 x N = 151936 x K = 2048 (fp16, fp32
    accumulation), against fp32 torch on column slices at both ends and a
    random sample of columns."""
    print("case: GEMM 4096 x 151936 x 2048", flush=True)
    M, N, K = 4096, 151936, 2048
    g = torch.Generator(device=dev).manual_seed(1024)
    A = torch.randn(M, K, generator=g, device=dev).half()
    B = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
    C = llmt.gemm_f16(A, B)
    torch.cuda.synchronize()
    cols = torch.cat([torch.arange(0, 256), torch.arange(N - 256, N),
                      torch.randperm(N, generator=torch.Generator().manual_seed(3))[:512]])
    want = A.float().cpu() @ B[cols.to(dev)].float().cpu().t()
    got = C[:, cols.to(dev)].cpu()
    assert rel_l2(got, want) < 1e-5
    del C


def test_device_quantizer_matches_oracle_on_c4_weights(dev):
    g = torch.Generator().manual_seed(1004)
    w = torch.randn(2048, 2048, generator=g) * 0.02
    from oracle.quant import quantize_rows
    q_ref, s_ref = quantize_rows(w.numpy())
    q, s = llmt.quantize_rows_i8(w.to(dev))
    assert np.array_equal(q.cpu().numpy(), q_ref)                 # bit-exact
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_c4_full_size_properties(dev):
    """Full C4 (28 layers, int8 weights, B8 x S512): finite loss near ln V,
    finite gradients, bit-identical reruns (fixed reduction order)."""
    print("case: C4 full size (B8 S512 int8)", flush=True)
    import bench
    ctx = llmt.Context(llmt.make_dims(Q3), 8, 512, int8=True)
    try:
        bench.build_model(ctx, Q3, 1004, dev, int8=True)
        ctx.lora_init(1004, 2048 ** -0.5, 0.01)
        g = torch.Generator(device=dev).manual_seed(1005)
        win = torch.randint(0, Q3.vocab, (8, 513), generator=g, device=dev, dtype=torch.int32)
        tok, tgt = win[:, :-1].contiguous(), win[:, 1:].contiguous()
        l1 = ctx.forward_backward(tok, tgt)
        g1 = ctx.lora_get("grad").clone()
        # the loss is the mean over the 8 x 511 rows with a target of
        # logsumexp(row) - row[target], from the library's own fp32 logits
        logits = _ptr_tensor(llmt.lib().llmt_logits(ctx.h), 4096 * Q3.vocab, dev).view(4096, -1)
        t = tgt.reshape(-1).long()
        lse = torch.logsumexp(logits.double(), 1)
        rows = lse - logits.gather(1, t[:, None]).squeeze(1).double()
        valid = ref.valid_rows(8, 512).to(dev)
        want = float(rows[valid].mean())
        print(f"C4 full: loss {l1:.6f} from logits {want:.6f}", flush=True)
        assert abs(l1 - want) < 1e-4
        l2 = ctx.forward_backward(tok, tgt)
        g2 = ctx.lora_get("grad")
        assert math.isfinite(l1) and abs(l1 - math.log(Q3.vocab)) < 2.0
        assert torch.isfinite(g1).all() and g1.abs().max() > 0
        assert l1 == l2 and torch.equal(g1, g2)
    finally:
        ctx.close()


# ------------------------------------------------------------------ large-T path
# T = B x S >= 1024 runs every frozen-weight GEMM on the 256 x 256 tile kernel
# (fp16 and int8 B operands, LoRA rows in the column tiles, per-row int8
# scales, the dX GEMMs' per-k scales carried by their operands); checked
# against the oracle on the small model.

def _small_dims():
    from helpers import SMALL
    return SMALL


@pytest.mark.parametrize("batch,seq", [(2, 64), (4, 256)])
def test_int8_zero_scale_channels_match_oracle(dev, batch, seq):
    """int8 weights with output channels whose fp16 scale is 0, in every
    projection: an all-zero row, and (q, k, v, o) a row below 4e-6 whose scale
    rounds to 0 in fp16 while its int8 values do not.  The forward applies the
    scale per output row, the Q/K/V and O dX GEMMs per k, and the down and
    gate/up dX operands carry it per column; the step matches the oracle on
    the dequantised weights at T = 128 (small-M GEMMs) and T = 1024 (large
    tiles)."""
    from oracle.configs import quantize_model_int8
    d = _small_dims()
    print(f"case: int8 zero-scale channels, B{batch} S{seq}", flush=True)
    W, ad, tok, tgt, _ = config_model(d, batch=batch, seq_len=seq, seed=1013)
    chans = {"wq": (5, 130), "wk": (3, 70), "wv": (7, 100), "wo": (11, 200),
             "w_gate": (2,), "w_up": (9,), "w_down": (4,)}
    for lw in W.layers:
        for name, rows in chans.items():
            w = getattr(lw, name).float().clone()
            w[rows[0]] = 0.0
            if len(rows) > 1:
                w[rows[1]] *= 1e-5  # |w| < 1e-6: the fp16 scale underflows to 0
            setattr(lw, name, w)
    W, qs = quantize_model_int8(W)
    for l in range(d.n_layers):
        for name, rows in chans.items():
            q, sc16 = qs[(l, name)]
            assert sc16[rows[0]] == 0 and not q[rows[0]].any()
            if len(rows) > 1:  # the case is exercised: scale 0, int8 values not
                assert sc16[rows[1]] == 0 and q[rows[1]].any()
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, d)
    ctx = llmt.Context(llmt.make_dims(d), batch, seq, int8=True)
    try:
        _upload_i8(ctx, W, qs, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert math.isfinite(loss) and abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, d)
        print("zero-scale worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


def test_int8_wide_qkv_rows_match_oracle(dev):
    """int8 weights with 32 query / 8 KV heads: the Q/K/V operand rows are
    6144 wide, past the 4096 the QK-norm backward writes eight columns a
    thread, so it takes its column-a-pass form."""
    d = ref.Dims(hidden=256, n_layers=1, n_heads=32, n_kv_heads=8, head_dim=128,
                 intermediate=512, vocab=2048)
    print("case: int8, 32/8 heads (Q + 2 KV = 6144), B2 S64", flush=True)
    W, ad, tok, tgt, qs = config_model(d, batch=2, seq_len=64, seed=1014, int8=True)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, d)
    ctx = llmt.Context(llmt.make_dims(d), 2, 64, int8=True)
    try:
        _upload_i8(ctx, W, qs, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, d)
        print("wide-qkv worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


@pytest.mark.parametrize("int8", [False, True])
def test_large_tile_step_matches_oracle(dev, int8):
    d = _small_dims()
    print(f"case: small model, B4 S256 (T=1024), int8={int8}", flush=True)
    W, ad, tok, tgt, qs = config_model(d, batch=4, seq_len=256, seed=1011, int8=int8)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, d)
    ctx = llmt.Context(llmt.make_dims(d), 4, 256, int8=int8)
    try:
        if int8:
            _upload_i8(ctx, W, qs, dev)
        else:
            upload_model(ctx, W, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, d)
        print("large-T worst", max(errs.items(), key=lambda kv: kv[1]), flush=True)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()
