"""Seeded synthetic inputs for the five benchmark configurations C0-C4.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Seed 1000 + k for config k, one CPU ``torch.Generator`` per config, drawn in
this fixed order: frozen weights layer by layer (wq, wk, wv, wo, w_gate, w_up,
w_down), then the embedding (tied lm_head, the reference scripts copy
embed -> lm_head: scripts/run.sh:19), then adapters layer by layer
(wq, wk, wv, wo; A then B), then the config's inputs.

N(0, s) means standard deviation s for 0.02 / 0.01 / 1; the fan-in form
N(0, 1/2048) for A is a variance (std 2048^-1/2).  Norm weights are 1.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch

from .lora_step import PROJS, Adapter, Dims, LayerW, ModelW, QWEN3_1_7B
from .quant import quantize_rows


def _randn(g: torch.Generator, shape, std: float) -> torch.Tensor:
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std


def make_layer(g: torch.Generator, dims: Dims, wdtype=torch.float16, std: float = 0.02) -> LayerW:
    H, Q, KV, I, hd = dims.hidden, dims.q_dim, dims.kv_dim, dims.intermediate, dims.head_dim
    one = lambda n: torch.ones(n, dtype=torch.float32)
    w = lambda o, i: _randn(g, (o, i), std).to(wdtype).float()
    wq, wk, wv, wo = w(Q, H), w(KV, H), w(KV, H), w(H, Q)
    wg, wu, wd = w(I, H), w(I, H), w(H, I)
    return LayerW(attn_norm=one(H), ffn_norm=one(H), wq=wq, wk=wk, wv=wv, wo=wo,
                  q_norm=one(hd), k_norm=one(hd), w_gate=wg, w_up=wu, w_down=wd)


def make_model(g: torch.Generator, dims: Dims, wdtype=torch.float16, embed: bool = True) -> ModelW:
    layers = [make_layer(g, dims, wdtype) for _ in range(dims.n_layers)]
    emb = _randn(g, (dims.vocab, dims.hidden), 0.02).to(wdtype).float() if embed else None
    return ModelW(embed=emb, layers=layers, final_norm=torch.ones(dims.hidden), lm_head=emb)


def make_adapters(g: torch.Generator, dims: Dims, b_std: float = 0.01):
    ad = []
    for _ in range(dims.n_layers):
        d = {}
        for p in PROJS:
            d_out, d_in = dims.adapter_dims(p)
            A = _randn(g, (dims.rank, d_in), 1.0 / math.sqrt(2048.0))
            B = _randn(g, (d_out, dims.rank), b_std)
            d[p] = Adapter(A, B, torch.zeros_like(A), torch.zeros_like(A),
                           torch.zeros_like(B), torch.zeros_like(B))
        ad.append(d)
    return ad


def quantize_model_int8(W: ModelW):
    """C4: every frozen GEMM weight -> int8 + fp16 scale via the
    src/kernels/quantize.cu:8-44 recipe; returns the dequantised fp32 model and
    the (q, scale16) pairs keyed by (layer, name)."""
    qs = {}
    for l, lw in enumerate(W.layers):
        for name in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            q, sc = quantize_rows(getattr(lw, name).numpy())
            sc16 = sc.astype(np.float16)
            qs[(l, name)] = (q, sc16)
            setattr(lw, name, torch.from_numpy(q.astype(np.float32) * sc16.astype(np.float32)[:, None]))
    return W, qs


def config0(dims: Dims = QWEN3_1_7B, seq_len: int = 128, seed: int = 1000):
    """C0: one Qwen3 layer, fp32 frozen weights, x and dY ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    d1 = Dims(**{**dims.__dict__, "n_layers": 1})
    lw = make_layer(g, d1, wdtype=torch.float32)
    ad = make_adapters(g, d1)
    x = _randn(g, (seq_len, dims.hidden), 1.0)
    dy = _randn(g, (seq_len, dims.hidden), 1.0)
    return d1, lw, ad[0], x, dy


def config1(vocab: int = 151936, hidden: int = 2048, rows: int = 128, seed: int = 1001):
    """C1: fused CE + lm_head backward in isolation (tied fp16 W)."""
    g = torch.Generator().manual_seed(seed)
    W = _randn(g, (vocab, hidden), 0.02).half()
    x = _randn(g, (rows, hidden), 1.0).half()
    targets = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int32)
    return x, W, targets


def config_model(dims: Dims = QWEN3_1_7B, batch: int = 1, seq_len: int = 128, seed: int = 1002,
                 int8: bool = False):
    """C2 (seed 1002, B1xS128) / C4 (seed 1004, int8, B8xS512): full model,
    tokens uniform in [0, V), next-token targets from an (S+1)-token window
    (src/train.cu:253-258)."""
    g = torch.Generator().manual_seed(seed)
    W = make_model(g, dims)
    ad = make_adapters(g, dims)
    win = torch.randint(0, dims.vocab, (batch, seq_len + 1), generator=g, dtype=torch.int32)
    tokens, targets = win[:, :-1].contiguous(), win[:, 1:].contiguous()
    qs = None
    if int8:
        W, qs = quantize_model_int8(W)
    return W, ad, tokens, targets, qs


def config3(batch: int = 4, seq_len: int = 2048, n_heads: int = 16, n_kv: int = 8,
            head_dim: int = 128, seed: int = 1003):
    """C3: attention backward stress inputs (fp16, N(0,1)), QK-norm weights 1."""
    g = torch.Generator().manual_seed(seed)
    q = _randn(g, (batch, seq_len, n_heads, head_dim), 1.0).half()
    k = _randn(g, (batch, seq_len, n_kv, head_dim), 1.0).half()
    v = _randn(g, (batch, seq_len, n_kv, head_dim), 1.0).half()
    do = _randn(g, (batch, seq_len, n_heads, head_dim), 1.0).half()
    return q, k, v, do
