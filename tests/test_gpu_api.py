"""GPU: tight pins of the optimizer step and of API contracts around the step.

- AdamW (src/kernels/lora.cu:206-220, bias corrections in fp32 with powf,
  :238-239) inside llmt_step, fed with the GPU's own gradients of that step:
  the update p' - p, m' and v' against the formula evaluated in float64 on
  the same inputs, within 1e-5 relative L2, at t = 1 (zero moments) and t = 3
  (non-zero moments), and with weight decay 0.1.  A planted mistake in the
  reference computation (the decoupled decay dropped, or the bias
  corrections of step t - 1) fails the same bar, so the pin can see each term.
- llmt_profile_kernels: a step run through the profiler leaves the adapters,
  m and v exactly where a plain step leaves them, and its launch counts per
  kind are those of the step's structure.
- Re-tying the lm_head: an untied head set, then a tied embedding set again,
  gives the tied model's loss (in the API and through the weight files).
- int8 frozen weights from the reference's fp32 weight files
  (llmt_load_weights_dir on an int8 context, the src/kernels/quantize.cu
  recipe on the device) against the oracle on the dequantised weights."""
import copy

import numpy as np
import pytest
import torch

import llmt
from helpers import (SMALL, grad_errors, oracle_grads, rel_l2, small_problem, upload_model,
                     write_weights_dir)
from oracle import lora_step as ref
from oracle.configs import quantize_model_int8

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-3
GRAD_TOL = 1e-2
ADAM_TOL = 1e-5


@pytest.fixture(scope="module")
def prob(dev):
    W, ad, tok, tgt = small_problem(SMALL, batch=2, seq_len=64, seed=21)
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=2, seq_len=64)
    upload_model(ctx, W, dev)
    yield dict(W=W, ad=ad, tok=tok.to(dev), tgt=tgt.to(dev), ctx=ctx)
    ctx.close()


def _adamw64(p, g, m, v, lr, b1, b2, eps, wd, t, decay=True, t_bc=None):
    """The reference update in float64 from fp32 inputs; the bias corrections
    1 - beta^t rounded to fp32 as the reference computes them (powf)."""
    t_bc = t if t_bc is None else t_bc
    bc1 = float(np.float32(1.0) - np.power(np.float32(b1), np.float32(t_bc)))
    bc2 = float(np.float32(1.0) - np.power(np.float32(b2), np.float32(t_bc)))
    p, g, m, v = (x.double() for x in (p, g, m, v))
    m2 = b1 * m + (1.0 - b1) * g
    v2 = b2 * v + (1.0 - b2) * g * g
    upd = lr * (m2 / bc1) / (torch.sqrt(v2 / bc2) + eps)
    dp = (-lr * wd * p if decay else 0.0) - upd
    return dp, m2, v2


@pytest.mark.parametrize("t,wd", [(1, 0.01), (3, 0.01), (3, 0.1)])
def test_adamw_in_step_tight(prob, dev, t, wd):
    print(f"case: AdamW in llmt_step, t={t}, wd={wd}", flush=True)
    ctx = prob["ctx"]
    n = ctx.lora_numel
    g = torch.Generator().manual_seed(500 + t)
    p0 = llmt.flatten_adapters(prob["ad"]).float()
    if t == 1:
        m0 = torch.zeros(n)
        v0 = torch.zeros(n)
    else:  # moments of the size a few earlier steps leave
        m0 = torch.randn(n, generator=g) * 2e-4
        v0 = (torch.randn(n, generator=g) * 2e-4) ** 2
    ctx.lora_set("param", p0.to(dev))
    ctx.lora_set("m", m0.to(dev))
    ctx.lora_set("v", v0.to(dev))
    hp = llmt.hparams(wd=wd)
    ctx.step(prob["tok"], prob["tgt"], hp, t)
    grad = ctx.lora_get("grad").cpu()          # this step's own gradients
    p1, m1, v1 = (ctx.lora_get(k).cpu() for k in ("param", "m", "v"))
    assert torch.isfinite(grad).all() and float(grad.abs().max()) > 0
    dp, m2, v2 = _adamw64(p0, grad, m0, v0, hp.lr, hp.beta1, hp.beta2, hp.eps, wd, t)
    errs = dict(dp=rel_l2(p1.double() - p0.double(), dp), m=rel_l2(m1, m2), v=rel_l2(v1, v2))
    print(f"t={t} wd={wd}: rel-L2 {errs}", flush=True)
    assert max(errs.values()) < ADAM_TOL, errs
    # the pin sees each term: planted mistakes in the reference fail the bar
    dp_nodecay, _, _ = _adamw64(p0, grad, m0, v0, hp.lr, hp.beta1, hp.beta2, hp.eps, wd, t,
                                decay=False)
    assert rel_l2(p1.double() - p0.double(), dp_nodecay) > 5 * ADAM_TOL
    if t > 1:
        dp_bc, _, _ = _adamw64(p0, grad, m0, v0, hp.lr, hp.beta1, hp.beta2, hp.eps, wd, t,
                               t_bc=t - 1)
        assert rel_l2(p1.double() - p0.double(), dp_bc) > 5 * ADAM_TOL


def test_adamw_standalone_matches_step_kernel(prob, dev):
    """llmt_adamw over the arena with a given gradient: the same update."""
    ctx = prob["ctx"]
    n = ctx.lora_numel
    g = torch.Generator().manual_seed(77)
    p0 = torch.randn(n, generator=g) * 0.02
    gr = torch.randn(n, generator=g) * 1e-3
    m0 = torch.randn(n, generator=g) * 1e-4
    v0 = (torch.randn(n, generator=g) * 1e-4) ** 2
    for kind, x in (("param", p0), ("grad", gr), ("m", m0), ("v", v0)):
        ctx.lora_set(kind, x.to(dev))
    hp = llmt.hparams(wd=0.1)
    llmt.check(llmt.lib().llmt_adamw(ctx.h, llmt.C.byref(hp), 5))
    p1, m1, v1 = (ctx.lora_get(k).cpu() for k in ("param", "m", "v"))
    dp, m2, v2 = _adamw64(p0, gr, m0, v0, hp.lr, hp.beta1, hp.beta2, hp.eps, 0.1, 5)
    assert rel_l2(p1.double() - p0.double(), dp) < ADAM_TOL
    assert rel_l2(m1, m2) < ADAM_TOL and rel_l2(v1, v2) < ADAM_TOL


def test_profile_kernels_contract(prob, dev):
    """A profiled step then a plain step equals two plain steps, bit for bit
    (the profiler restores p, m and v after its AdamW replays); its launch
    counts follow the step's structure."""
    ctx = prob["ctx"]
    p0 = llmt.flatten_adapters(prob["ad"]).float().to(dev)
    zeros = torch.zeros(ctx.lora_numel, device=dev)
    hp = llmt.hparams()

    def reset():
        ctx.lora_set("param", p0)
        ctx.lora_set("m", zeros)
        ctx.lora_set("v", zeros)

    reset()
    ctx.step(prob["tok"], prob["tgt"], hp, 1)
    l2 = ctx.step(prob["tok"], prob["tgt"], hp, 2)
    want = [ctx.lora_get(k).clone() for k in ("param", "m", "v")]
    reset()
    kinds = ctx.profile_kernels(prob["tok"], prob["tgt"], hp, 1, reps=2)
    got_l2 = ctx.step(prob["tok"], prob["tgt"], hp, 2)
    assert got_l2 == l2
    for k, w in zip(("param", "m", "v"), want):
        assert torch.equal(ctx.lora_get(k), w), k
    count = {}
    for k in kinds:
        base = k["name"].split()[0]
        count[base] = count.get(base, 0) + k["launches"]
        assert k["us"] > 0
    L = SMALL.n_layers
    print("profile kinds", {k["name"]: k["launches"] for k in kinds}, flush=True)
    assert count["embed_norm"] == 1 and count["adamw"] == 1 and count["lora_grad"] == 1
    assert count["cross_entropy"] == 1
    assert count["attn_fwd"] == L and count["attn_bwd"] == L
    assert count["qkv_post"] == L and count["qk_bwd"] == L
    gemms = sum(k["launches"] for k in kinds if k["category"].startswith("gemm"))
    for k in kinds:   # every kind carries its algorithmic work
        assert k["flops"] > 0 or k["bytes"] > 0, k["name"]
    assert gemms == 8 * L + 2       # 4 forward + 4 backward GEMMs a layer, logits, head dX
    per_cat = {}
    for k in kinds:
        per_cat[k["category"]] = per_cat.get(k["category"], 0) + k["launches"]
    assert per_cat["gemm_fwd"] == 4 * L and per_cat["gemm_bwd"] == 4 * L
    assert sum(k["launches"] for k in kinds if k["name"].endswith(" dX")) == 4 * L + 1


def test_lm_head_retied_by_set_embed(prob, dev, tmp_path):
    """Untied head set, then the tied embedding set again: the head is the
    embedding once more (API and weight-file loaders)."""
    W, ad = prob["W"], prob["ad"]
    tok, tgt = prob["tok"], prob["tgt"]
    loss_tied, _, _ = oracle_grads(W, ad, tok.cpu(), tgt.cpu(), SMALL)
    g = torch.Generator().manual_seed(3)
    head = (torch.randn(SMALL.vocab, SMALL.hidden, generator=g) * 0.02).half().float()
    Wu = copy.deepcopy(W)
    Wu.lm_head = head
    loss_untied, _, _ = oracle_grads(Wu, ad, tok.cpu(), tgt.cpu(), SMALL)
    assert abs(float(loss_tied) - float(loss_untied)) > 10 * LOSS_TOL
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=2, seq_len=64)
    try:
        upload_model(ctx, W, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        ctx.set_graph(True)
        ctx.set_lm_head_f16(head.half().to(dev))
        assert abs(ctx.forward_backward(tok, tgt) - float(loss_untied)) < LOSS_TOL
        ctx.set_embed_f16(W.embed.half().to(dev), W.final_norm.to(dev))
        assert abs(ctx.forward_backward(tok, tgt) - float(loss_tied)) < LOSS_TOL
        # weight files: an untied directory, then a tied one, into one context
        write_weights_dir(W, tmp_path / "untied", lm_head=head)
        write_weights_dir(W, tmp_path / "tied")
        ctx.load_weights_dir(tmp_path / "untied")
        assert abs(ctx.forward_backward(tok, tgt) - float(loss_untied)) < LOSS_TOL
        ctx.load_weights_dir(tmp_path / "tied")
        assert abs(ctx.forward_backward(tok, tgt) - float(loss_tied)) < LOSS_TOL
    finally:
        ctx.close()


def test_int8_weight_files_match_oracle(prob, dev, tmp_path):
    """llmt_load_weights_dir into an int8 context: the fp32 weight files are
    quantised on the device (bit-exact recipe, scales rounded to fp16) and the
    step matches the oracle on the dequantised weights."""
    W, ad = prob["W"], prob["ad"]
    tok, tgt = prob["tok"], prob["tgt"]
    write_weights_dir(W, tmp_path / "w")
    Wq, _ = quantize_model_int8(copy.deepcopy(W))
    loss_ref, grads_ref, _ = oracle_grads(Wq, ad, tok.cpu(), tgt.cpu(), SMALL)
    loss_f16, _, _ = oracle_grads(W, ad, tok.cpu(), tgt.cpu(), SMALL)
    print(f"int8 files: oracle loss {float(loss_ref):.6f} (fp16 weights {float(loss_f16):.6f})",
          flush=True)
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=2, seq_len=64, int8=True)
    try:
        ctx.load_weights_dir(tmp_path / "w")
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok, tgt)
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, SMALL)
        worst = max(errs.items(), key=lambda kv: kv[1])
        print("int8 files worst grad", worst, flush=True)
        assert worst[1] < GRAD_TOL
    finally:
        ctx.close()
