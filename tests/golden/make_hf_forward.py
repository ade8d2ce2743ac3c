"""Write hf_qwen3.npz: an independent pin of the oracle's model composition.

The oracle (oracle/lora_step.py) restates the reference's forward op order
(src/kernels/lora_forward.cu:198-304: LoRA enters the Q/K/V/O projections
before the QK-norm, then RoPE, causal GQA attention, O projection, residual,
FFN norm, SwiGLU, down projection, residual; final norm; tied lm_head) and its
closed-form backward.  The reference pins its own forward against Hugging Face
Qwen3 (python/verify.py:7-26, python/reference_forward.py:28-67).  This script
does the same with the local transformers package (models/qwen3), building
random-init Qwen3ForCausalLM models from a Qwen3Config (no download), in
float64 with eager attention.

LoRA is folded into the HF weights as W' = W + s B A (s = alpha / r = 2), which
reduces the LoRA forward to the library's dense projection.  Since
y = x W'^T, the gradient of W' is dY^T x, and the adapter gradients follow
exactly: dA = s B^T dW', dB = s dW' A^T.  So HF's autograd pins both the
forward (logits, loss) and the backward (every adapter gradient).

Weights and adapters come from oracle.configs with the seeds below, so the
CPU test rebuilds the same inputs and only the outputs are stored:
  tiny   TINY dims (hidden 64, 2 layers, 4/2 heads, head_dim 16, I 96, V 512),
         batch 2 x seq 8, seed 2001: logits [16, 512], loss, every adapter
         gradient in full (flat arena order: layer, q/k/v/o, A then B).
  wide   one layer at full Qwen3-1.7B width (hidden 2048, 16/8 heads,
         head_dim 128, I 6144), vocabulary 1024, batch 1 x seq 16, seed 2002:
         logits [16, 1024], loss, and for every adapter gradient G [m, n] the
         sketch R_m^T G R_n (8 x 8, R Gaussian from seed 2003), which moves
         with any error in G (Johnson-Lindenstrauss) at a fraction of the size.
Outputs are float64 except the logits (float32).  The loss is torch's
cross_entropy over the HF logits with labels = the input ids shifted by one:
the mean over the S-1 rows of each sequence that have a next token (the
reference's src/kernels/loss.cu:86-90).

Runs in the build container only (transformers must be importable):
    python tests/golden/make_hf_forward.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import lora_step as ref  # noqa: E402
from oracle.configs import make_adapters, make_model  # noqa: E402

CASES = {
    "tiny": dict(dims=ref.TINY, batch=2, seq=8, seed=2001),
    "wide": dict(dims=ref.Dims(n_layers=1, vocab=1024), batch=1, seq=16, seed=2002),
}
SKETCH_SEED = 2003
SKETCH = 8


def case_inputs(name):
    """Seeded model, adapters (B != 0) and token windows of a case, float32."""
    c = CASES[name]
    d = c["dims"]
    g = torch.Generator().manual_seed(c["seed"])
    W = make_model(g, d)
    ad = make_adapters(g, d)
    tok = torch.randint(0, d.vocab, (c["batch"], c["seq"]), generator=g, dtype=torch.int32)
    return d, W, ad, tok


def sketch_mats(m, n):
    """The fixed Gaussian sketch pair (R_m [m, 8], R_n [n, 8]) for an [m, n] tensor."""
    g = torch.Generator().manual_seed(SKETCH_SEED + 7919 * m + n)
    return (torch.randn(m, SKETCH, generator=g, dtype=torch.float64),
            torch.randn(n, SKETCH, generator=g, dtype=torch.float64))


def sketch(G):
    Rm, Rn = sketch_mats(*G.shape)
    return Rm.t() @ G.double() @ Rn


def hf_run(d, W, ad, tok):
    """Logits, loss and adapter gradients of the HF Qwen3 model with merged
    adapters.  Returns (logits [T, V] float64, loss, grads[l][proj] = (dA, dB))."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=d.vocab, hidden_size=d.hidden, intermediate_size=d.intermediate,
                      num_hidden_layers=d.n_layers, num_attention_heads=d.n_heads,
                      num_key_value_heads=d.n_kv_heads, head_dim=d.head_dim, hidden_act="silu",
                      max_position_embeddings=4096, rms_norm_eps=d.eps,
                      rope_parameters={"rope_type": "default", "rope_theta": d.theta},
                      tie_word_embeddings=True, attention_bias=False, use_sliding_window=False,
                      attention_dropout=0.0, use_cache=False)
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).double().eval()
    s = d.lora_scale
    dd = lambda t: t.double()
    merged = {}
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(dd(W.embed))
        model.model.norm.weight.copy_(dd(W.final_norm))
        for l, lw in enumerate(W.layers):
            hl = model.model.layers[l]
            hl.input_layernorm.weight.copy_(dd(lw.attn_norm))
            hl.post_attention_layernorm.weight.copy_(dd(lw.ffn_norm))
            hl.self_attn.q_norm.weight.copy_(dd(lw.q_norm))
            hl.self_attn.k_norm.weight.copy_(dd(lw.k_norm))
            for proj, mod, w in (("wq", hl.self_attn.q_proj, lw.wq), ("wk", hl.self_attn.k_proj, lw.wk),
                                 ("wv", hl.self_attn.v_proj, lw.wv), ("wo", hl.self_attn.o_proj, lw.wo)):
                a = ad[l][proj]
                mod.weight.copy_(dd(w) + s * dd(a.B) @ dd(a.A))
                merged[(l, proj)] = mod.weight
            hl.mlp.gate_proj.weight.copy_(dd(lw.w_gate))
            hl.mlp.up_proj.weight.copy_(dd(lw.w_up))
            hl.mlp.down_proj.weight.copy_(dd(lw.w_down))
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    ids = tok.long()
    logits = model(input_ids=ids).logits
    assert logits.dtype == torch.float64
    # HF's own loss helper upcasts to float32; the same mean over shifted
    # labels in float64 with torch's cross_entropy.
    loss = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, d.vocab),
                                             ids[:, 1:].reshape(-1))
    loss.backward()
    grads = []
    for l in range(d.n_layers):
        gl = {}
        for proj in ref.PROJS:
            dW = merged[(l, proj)].grad
            a = ad[l][proj]
            gl[proj] = (s * dd(a.B).t() @ dW, s * dW @ dd(a.A).t())
        grads.append(gl)
    return logits.detach().reshape(-1, d.vocab), float(loss.detach()), grads


def flat(grads, f=lambda t: t):
    return np.concatenate([f(t).reshape(-1).numpy() for gl in grads for p in ref.PROJS
                           for t in gl[p]])


def main():
    torch.set_num_threads(8)
    arrays = {}
    for name in CASES:
        d, W, ad, tok = case_inputs(name)
        logits, loss, grads = hf_run(d, W, ad, tok)
        arrays[f"{name}_tokens"] = tok.numpy()
        arrays[f"{name}_logits"] = logits.float().numpy()
        arrays[f"{name}_loss"] = np.float64(loss)
        if name == "tiny":
            arrays[f"{name}_grads"] = flat(grads)
        else:
            arrays[f"{name}_grad_sketch"] = flat(grads, sketch)
        print(name, "loss", loss, flush=True)
    np.savez_compressed(HERE / "hf_qwen3.npz", **arrays)
    print("hf_qwen3.npz", (HERE / "hf_qwen3.npz").stat().st_size)


if __name__ == "__main__":
    main()
