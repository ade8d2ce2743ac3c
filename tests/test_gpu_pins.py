"""GPU: the integer and distribution work of the step, pinned exactly.

  * adapter init (src/kernels/lora.cu:32-62: A ~ 0.02 N(0,1), B = 0, m = v = 0):
    moments and normal quantiles of A over the full Qwen3-1.7B arena, B, m and
    v exactly zero when b_std = 0, one seed -> bit-identical arenas;
  * the embedding gather (src/kernels/embed.cu:6-20): the residual stream at
    the input of layer 0 equals E[token] in fp32, bit for bit;
  * the CE target index (src/kernels/loss.cu:13-71): in every valid dlogits
    row the one negative entry sits at the target (integer, bit-exact), with
    value (p_t - 1) / n_valid, and rows without a target are exactly zero;
  * an untied lm_head (src/train.cu:87-88), through the API and through the
    weight-file loader, against the oracle with its own head;
  * the compat lora_forward_add (src/kernels/lora.cu:181-202) against the
    oracle's lora_fwd.
"""
import ctypes as C
import math

import pytest
import torch

import llmt
from helpers import SMALL, oracle_grads, rel_l2, small_problem, upload_model, write_weights_dir
from oracle import lora_step as ref

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-3
GRAD_TOL = 1e-2


def _arena_parts(flat, dims):
    """(all A values, all B values) of a flat arena, float64 on the CPU."""
    ad = llmt.unflatten_adapters(flat.cpu(), dims)
    A = torch.cat([d[p][0].reshape(-1) for d in ad for p in ref.PROJS]).double()
    B = torch.cat([d[p][1].reshape(-1) for d in ad for p in ref.PROJS]).double()
    return A, B


def test_lora_init_distribution_and_determinism(dev):
    print("case: llmt_lora_init, full Qwen3-1.7B arena", flush=True)
    d = ref.QWEN3_1_7B
    ctx = llmt.Context(llmt.make_dims(d), 1, 16)
    try:
        a_std = 0.02
        ctx.lora_init(1234, a_std, 0.0)
        p1 = ctx.lora_get("param")
        A, B = _arena_parts(p1, d)
        n = A.numel()
        assert n == d.n_layers * 16 * (3 * d.hidden + d.q_dim)
        # moments: the sampling error of the mean is a_std / sqrt(n) ~ 5e-4 a_std
        assert abs(float(A.mean())) < 0.01 * a_std
        assert abs(float(A.std()) / a_std - 1.0) < 0.01
        # normal quantiles (a uniform draw has 57.7% within one sigma)
        for k, want in ((1.0, 0.682689), (2.0, 0.954500)):
            frac = float((A.abs() < k * a_std).double().mean())
            assert abs(frac - want) < 0.003, (k, frac)
        # B = 0 and the moments exactly zero (src/kernels/lora.cu:56-62)
        assert torch.count_nonzero(B) == 0
        assert torch.count_nonzero(ctx.lora_get("m")) == 0
        assert torch.count_nonzero(ctx.lora_get("v")) == 0
        # same seed -> bit-identical; another seed -> different draws
        ctx.lora_init(1234, a_std, 0.0)
        assert torch.equal(ctx.lora_get("param"), p1)
        ctx.lora_init(1235, a_std, 0.0)
        assert not torch.equal(ctx.lora_get("param"), p1)
        # a B std (the configs' N(0, 0.01)) reaches B only
        ctx.lora_init(77, a_std, 0.01)
        A2, B2 = _arena_parts(ctx.lora_get("param"), d)
        assert abs(float(B2.std()) / 0.01 - 1.0) < 0.01
        assert abs(float(A2.std()) / a_std - 1.0) < 0.01
    finally:
        ctx.close()


def test_embedding_gather_bit_exact(dev):
    print("case: embedding gather, SMALL B2 S64", flush=True)
    W, ad, tok, tgt = small_problem()
    T = tok.numel()
    ctx = llmt.Context(llmt.make_dims(SMALL), tok.shape[0], tok.shape[1])
    try:
        upload_model(ctx, W, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        ctx.forward_backward(tok.to(dev), tgt.to(dev))
        x0 = ctx.layer_in(0, T).cpu()
        want = W.embed.to(torch.float16).float()[tok.reshape(-1).long()]
        assert torch.equal(x0, want)
        # the next layer's input against the oracle's residual stream
        _, stash = ref.model_forward(W, ad, tok, SMALL)
        assert rel_l2(ctx.layer_in(1, T).cpu(), stash["layers"][1]["x_in"]) < 1e-3
    finally:
        ctx.close()


def test_ce_target_index_bit_exact(dev):
    print("case: CE target index, 2 x 64 rows x 151936", flush=True)
    S, rows, V = 64, 128, 151936
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(rows, V, generator=g) * 2.0
    tgt = torch.randint(0, V, (rows,), generator=g, dtype=torch.int32)
    lm, lr, dl = llmt.cross_entropy(logits.to(dev), tgt.to(dev), S)
    dl = dl.cpu()
    valid = ref.valid_rows(rows // S, S)
    n_valid = int(valid.sum())
    neg = dl < 0
    t = tgt.long()
    # the target index: the one negative entry of each valid row (bit-exact)
    assert torch.equal(neg[valid].sum(1), torch.ones(n_valid, dtype=torch.long))
    assert torch.equal(dl[valid].argmin(1), t[valid])
    # rows without a target are exactly zero
    assert torch.count_nonzero(dl[~valid]) == 0
    # the value at the target: (p_t - 1) / n_valid
    x = logits.double()
    lse = torch.logsumexp(x, 1)
    p_t = torch.exp(x.gather(1, t[:, None]).squeeze(1) - lse)
    got = dl.double().gather(1, t[:, None]).squeeze(1)[valid]
    assert float((got * n_valid + 1.0 - p_t[valid]).abs().max()) < 1e-6
    # per-row losses lse - x_t, zero for rows without a target
    lr = lr.cpu().double()
    want = (lse - x.gather(1, t[:, None]).squeeze(1)) * valid
    assert float((lr - want).abs().max()) < 1e-4
    assert abs(float(lm) - float(want.sum() / n_valid)) < 1e-5


def _untied_problem():
    W, ad, tok, tgt = small_problem()
    g = torch.Generator().manual_seed(8)
    head = (torch.randn(SMALL.vocab, SMALL.hidden, generator=g) * 0.02).half().float()
    W2 = ref.ModelW(embed=W.embed, layers=W.layers, final_norm=W.final_norm, lm_head=head)
    return W, W2, head, ad, tok, tgt


@pytest.mark.parametrize("via", ["api", "weights_dir"])
def test_untied_lm_head_matches_oracle(dev, via, tmp_path):
    print(f"case: untied lm_head via {via}", flush=True)
    W, W2, head, ad, tok, tgt = _untied_problem()
    loss_ref, grads_ref, _ = oracle_grads(W2, ad, tok, tgt, SMALL)
    loss_tied, _, _ = oracle_grads(W, ad, tok, tgt, SMALL)
    assert abs(float(loss_ref) - float(loss_tied)) > 10 * LOSS_TOL   # the head matters
    ctx = llmt.Context(llmt.make_dims(SMALL), tok.shape[0], tok.shape[1])
    try:
        if via == "api":
            upload_model(ctx, W, dev)
            ctx.set_lm_head_f16(head.half().to(dev))
        else:
            write_weights_dir(W, tmp_path / "w", lm_head=head)
            ctx.load_weights_dir(tmp_path / "w")
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        ctx.set_graph(True)
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        from helpers import grad_errors
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, SMALL)
        assert max(errs.values()) < GRAD_TOL
    finally:
        ctx.close()


def test_weights_dir_tied_head_file(dev, tmp_path):
    """A head file equal to the embedding keeps the tied model."""
    W, ad, tok, tgt = small_problem()
    loss_ref, _, _ = oracle_grads(W, ad, tok, tgt, SMALL)
    write_weights_dir(W, tmp_path / "w")
    ctx = llmt.Context(llmt.make_dims(SMALL), tok.shape[0], tok.shape[1])
    try:
        ctx.load_weights_dir(tmp_path / "w")
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
    finally:
        ctx.close()


def test_hf_checkpoint_export_matches_transformers(dev, tmp_path):
    """A random-init transformers Qwen3ForCausalLM (the SMALL shape, weights
    rounded to fp16 values, norm weights randomised, tied head) saved as a
    safetensors checkpoint, exported by llmt.export, loaded by
    llmt_load_weights_dir: with zero adapters the step's loss equals
    transformers' own fp32 loss on the same tokens (labels = inputs, i.e.
    the mean over the S - 1 next-token rows of each sequence)."""
    transformers = pytest.importorskip("transformers")
    from llmt import export
    print("case: HF checkpoint -> llmt.export -> load_weights_dir", flush=True)
    torch.manual_seed(21)
    cfg = transformers.Qwen3Config(
        vocab_size=SMALL.vocab, hidden_size=SMALL.hidden, intermediate_size=SMALL.intermediate,
        num_hidden_layers=SMALL.n_layers, num_attention_heads=SMALL.n_heads,
        num_key_value_heads=SMALL.n_kv_heads, head_dim=SMALL.head_dim, rms_norm_eps=SMALL.eps,
        rope_theta=SMALL.theta, tie_word_embeddings=True)
    model = transformers.Qwen3ForCausalLM(cfg).float().eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(1.0 + 0.2 * torch.randn_like(p))
            p.copy_(p.half().float())
    model.save_pretrained(tmp_path / "ckpt", safe_serialization=True)
    export.export_checkpoint(tmp_path / "ckpt", tmp_path / "w")
    g = torch.Generator().manual_seed(22)
    win = torch.randint(0, SMALL.vocab, (2, 65), generator=g, dtype=torch.int32)
    tok, tgt = win[:, :-1].contiguous(), win[:, 1:].contiguous()
    with torch.no_grad():
        want = float(model(input_ids=tok.long(), labels=tok.long()).loss)
    ctx = llmt.Context(llmt.make_dims(SMALL), tok.shape[0], tok.shape[1])
    try:
        ctx.load_weights_dir(tmp_path / "w")
        ctx.lora_set("param", torch.zeros(ctx.lora_numel, device=dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - want) < LOSS_TOL, (loss, want)
    finally:
        ctx.close()


class _AdapterC(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("A", "B", "mA", "vA", "mB", "vB")] + \
               [("d_in", C.c_int), ("d_out", C.c_int)]


@pytest.mark.parametrize("d_out,d_in,seq", [(1024, 2048, 128), (2048, 2048, 77)])
def test_compat_lora_forward_add(dev, d_out, d_in, seq):
    print(f"case: lora_forward_add {d_out}x{d_in} seq {seq}", flush=True)
    L = llmt.lib()
    L.lora_forward_add.argtypes = [C.c_void_p, C.POINTER(_AdapterC), C.c_void_p, C.c_void_p,
                                   C.c_int]
    g = torch.Generator().manual_seed(d_out + seq)
    x = torch.randn(seq, d_in, generator=g)
    A = torch.randn(16, d_in, generator=g) / math.sqrt(2048.0)
    B = torch.randn(d_out, 16, generator=g) * 0.01
    y0 = torch.randn(seq, d_out, generator=g)
    h_ref, dy = ref.lora_fwd(x, A, B, 2.0)
    xd, Ad, Bd, yd = x.to(dev), A.to(dev), B.to(dev), y0.clone().to(dev)
    h = torch.empty(seq, 16, device=dev)
    a = _AdapterC(Ad.data_ptr(), Bd.data_ptr(), None, None, None, None, d_in, d_out)
    torch.cuda.synchronize()
    L.lora_forward_add(xd.data_ptr(), C.byref(a), yd.data_ptr(), h.data_ptr(), seq)
    torch.cuda.synchronize()
    assert rel_l2(h.cpu(), h_ref) < 1e-5
    assert rel_l2(yd.cpu() - y0, dy) < 1e-5
    # h_buf may be NULL
    yd2 = y0.clone().to(dev)
    L.lora_forward_add(xd.data_ptr(), C.byref(a), yd2.data_ptr(), None, seq)
    torch.cuda.synchronize()
    assert torch.equal(yd2, yd)
