"""Helpers shared by the test modules, __graft_entry__.smoke() and bench.py:
seeded models in oracle form and their upload into a libllmt context."""
from __future__ import annotations

import torch

from oracle import lora_step as ref
from oracle.configs import make_adapters, make_model

# The smallest model the HIP kernels accept (head_dim must be 128): two
# layers, GQA group 2, every dimension a multiple of the GEMM tile.
SMALL = ref.Dims(hidden=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=128,
                 intermediate=512, vocab=2048)


def rel_l2(a, b):
    """||a - b|| / ||b|| in float64 on the CPU."""
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def small_problem(dims=SMALL, batch=2, seq_len=64, seed=7):
    """Seeded fp16-valued weights, adapters (A var 1/2048, B std 0.01) and an
    (S+1)-token window per sequence (src/train.cu:253-258)."""
    g = torch.Generator().manual_seed(seed)
    W = make_model(g, dims)
    ad = make_adapters(g, dims)
    win = torch.randint(0, dims.vocab, (batch, seq_len + 1), generator=g, dtype=torch.int32)
    return W, ad, win[:, :-1].contiguous(), win[:, 1:].contiguous()


def upload_model(ctx, W, dev):
    """Frozen weights of an oracle ModelW into a context (fp16 matrices, fp32 norms)."""
    h = lambda t: t.to(torch.float16).to(dev).contiguous()
    f = lambda t: t.to(torch.float32).to(dev).contiguous()
    for l, lw in enumerate(W.layers):
        ctx.set_layer_f16(l, h(lw.wq), h(lw.wk), h(lw.wv), h(lw.wo), h(lw.w_gate), h(lw.w_up),
                          h(lw.w_down), f(lw.attn_norm), f(lw.ffn_norm), f(lw.q_norm),
                          f(lw.k_norm))
    ctx.set_embed_f16(h(W.embed), f(W.final_norm))


def oracle_grads(W, ad, tokens, targets, dims, quirks=()):
    """Exact fp32 oracle: loss, grads[l][proj] = (dA, dB), dlogits."""
    batch, seq_len = tokens.shape
    logits, stash = ref.model_forward(W, ad, tokens, dims)
    loss, dlogits, _ = ref.cross_entropy(logits, targets.reshape(-1),
                                         ref.valid_rows(batch, seq_len))
    grads, _ = ref.model_backward(dlogits, stash, W, ad, dims, batch, seq_len, quirks)
    return loss, grads, logits


def grad_errors(flat_gpu, grads_ref, dims):
    """Relative L2 error of every adapter-gradient tensor: {(l, proj, 'A'|'B'): err}."""
    import llmt
    got = llmt.unflatten_adapters(flat_gpu.cpu(), dims)
    errs = {}
    for l in range(dims.n_layers):
        for p in ref.PROJS:
            errs[(l, p, "A")] = rel_l2(got[l][p][0], grads_ref[l][p][0])
            errs[(l, p, "B")] = rel_l2(got[l][p][1], grads_ref[l][p][1])
    return errs


def write_weights_dir(W, d, lm_head=None):
    """A model in the reference's weight-file layout (src/train.cu:56-89,
    python/export_weights.py:19-26): <d>/<hf_param_name>.bin raw fp32.  The
    lm_head file is a copy of the embedding (scripts/run.sh:19) unless
    lm_head is given."""
    from pathlib import Path
    d = Path(d)
    d.mkdir(parents=True, exist_ok=True)

    def put(name, t):
        t.detach().to(torch.float32).contiguous().numpy().astype("<f4").tofile(d / f"{name}.bin")

    put("model.embed_tokens.weight", W.embed)
    put("lm_head.weight", W.embed if lm_head is None else lm_head)
    put("model.norm.weight", W.final_norm)
    for l, lw in enumerate(W.layers):
        p = f"model.layers.{l}."
        for name, t in (("self_attn.q_proj", lw.wq), ("self_attn.k_proj", lw.wk),
                        ("self_attn.v_proj", lw.wv), ("self_attn.o_proj", lw.wo),
                        ("mlp.gate_proj", lw.w_gate), ("mlp.up_proj", lw.w_up),
                        ("mlp.down_proj", lw.w_down), ("input_layernorm", lw.attn_norm),
                        ("post_attention_layernorm", lw.ffn_norm),
                        ("self_attn.q_norm", lw.q_norm), ("self_attn.k_norm", lw.k_norm)):
            put(p + name + ".weight", t)
