"""CPU: the oracle's model composition against Hugging Face Qwen3.

tests/golden/hf_qwen3.npz holds logits, loss and adapter gradients of
random-init transformers Qwen3ForCausalLM models with the adapters merged
into the projections (W + s B A), written by tests/golden/make_hf_forward.py.
The oracle's model_forward / cross_entropy / model_backward (closed forms, no
autograd) run here in float64 on the same seeded weights and must reproduce
them.  This pins the op order of src/kernels/lora_forward.cu:198-304 (LoRA
before the QK-norm, half-split RoPE, GQA head mapping, residuals, SwiGLU,
tied lm_head) and the backward of src/kernels/lora_backward.cu:212-408
independently of the oracle's own autograd checks.  Planted mistakes in the
oracle (interleaved RoPE pairs, the reference's final-norm quirk Q3, a
dropped q/k LoRA term) must fail the same comparison.
"""
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import lora_step as ref

GOLD = Path(__file__).resolve().parent / "golden"
FIX = np.load(GOLD / "hf_qwen3.npz")


def _maker():
    spec = importlib.util.spec_from_file_location("make_hf_forward", GOLD / "make_hf_forward.py")
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


MK = _maker()


def _double(d, W, ad):
    f = lambda t: t.double()
    W = ref.ModelW(embed=f(W.embed),
                   layers=[ref.LayerW(**{k: f(getattr(l, k)) for k in l.__dataclass_fields__})
                           for l in W.layers],
                   final_norm=f(W.final_norm), lm_head=f(W.embed))
    ad = [{p: ref.Adapter(a.A.double(), a.B.double()) for p, a in dl.items()} for dl in ad]
    return W, ad


def _oracle(name, quirks=()):
    d, W, ad, tok = MK.case_inputs(name)
    assert np.array_equal(tok.numpy(), FIX[f"{name}_tokens"])
    W, ad = _double(d, W, ad)
    B, S = tok.shape
    logits, stash = ref.model_forward(W, ad, tok, d)
    # targets: the next token of each window (the last row has none: Q5)
    tgt = torch.cat([tok[:, 1:], tok[:, :1]], dim=1).reshape(-1)
    loss, dlogits, _ = ref.cross_entropy(logits, tgt, ref.valid_rows(B, S))
    grads, _ = ref.model_backward(dlogits, stash, W, ad, d, B, S, quirks)
    return logits, float(loss), grads


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def _grads_vs_fixture(name, grads):
    if name == "tiny":
        return _rel(MK.flat(grads), FIX["tiny_grads"])
    # per-tensor sketches: the worst tensor
    got = MK.flat(grads, MK.sketch).reshape(-1, MK.SKETCH * MK.SKETCH)
    want = FIX["wide_grad_sketch"].reshape(-1, MK.SKETCH * MK.SKETCH)
    return max(_rel(g, w) for g, w in zip(got, want))


@pytest.mark.parametrize("name", ["tiny", "wide"])
def test_oracle_matches_hf_qwen3(name):
    logits, loss, grads = _oracle(name)
    assert _rel(logits.numpy(), FIX[f"{name}_logits"]) < 1e-5
    # HF computes its RMSNorms and RoPE angles in float32: ~1e-7 relative
    assert abs(loss - float(FIX[f"{name}_loss"])) < 1e-6
    assert _grads_vs_fixture(name, grads) < 1e-5


def test_interleaved_rope_is_caught(monkeypatch):
    """RoPE pairing (d, d+1) instead of the half split (d, d+hd/2)."""
    def rope_interleaved(x, cos, sin):
        x0, x1 = x[..., 0::2], x[..., 1::2]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        return torch.stack([x0 * c - x1 * s, x1 * c + x0 * s], dim=-1).flatten(-2)
    monkeypatch.setattr(ref, "rope_fwd", rope_interleaved)
    logits, _, _ = _oracle("tiny")
    assert _rel(logits.numpy(), FIX["tiny_logits"]) > 1e-3


def test_final_norm_quirk_is_caught():
    """Q3 (final-norm backward with the last layer's post-attention residual)."""
    _, _, grads = _oracle("tiny", quirks=("final_norm",))
    assert _grads_vs_fixture("tiny", grads) > 1e-3


def test_dropped_qk_lora_term_is_caught(monkeypatch):
    """The q/k adapters' up-projection left out of the forward."""
    orig = ref.layer_forward

    def late_lora(x, lw, lad, dims, batch, seq_len, cos, sin, rnd=ref.Identity):
        zero = {p: ref.Adapter(a.A, torch.zeros_like(a.B)) if p in ("wq", "wk") else a
                for p, a in lad.items()}
        y, st = orig(x, lw, zero, dims, batch, seq_len, cos, sin, rnd)
        return y, st
    monkeypatch.setattr(ref, "layer_forward", late_lora)
    logits, _, _ = _oracle("tiny")
    assert _rel(logits.numpy(), FIX["tiny_logits"]) > 1e-4
