"""Write the committed golden fixtures of this directory from the CPU oracle.

The reference (visheshnarayan/llm.cu) ships no golden vectors or tests for the
training step, so these fixtures are the oracle's outputs on seeded inputs,
recorded once so that later oracle edits and the GPU path are both checked
against fixed numbers:
  small_step.npz  the SMALL model (head_dim 128, 2 layers) step at B2 x S64,
                  seed 7: loss, every adapter gradient (flat arena order:
                  layer, q/k/v/o, A then B), the layer-0 parameters after one
                  AdamW step (lr 3e-4, betas (0.9, 0.999), eps 1e-8, wd 0.01).
  tiny_step.npz   the TINY model (head_dim 16) step in float64, seed 36.
  quant.npz       int8 per-row quantisation (src/kernels/quantize.cu:8-44)
                  of 64 x 256 fp32 rows with planted ties and a zero row.

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (str(ROOT), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import lora_step as ref  # noqa: E402
from oracle.configs import make_adapters, make_model  # noqa: E402
from oracle.quant import quantize_rows  # noqa: E402


def flat_grads(grads):
    return np.concatenate([t.reshape(-1).numpy() for d in grads for p in ref.PROJS for t in d[p]])


def small_step():
    from helpers import SMALL, oracle_grads, small_problem
    W, ad, tok, tgt = small_problem()
    loss, grads, _ = oracle_grads(W, ad, tok, tgt, SMALL)
    ref.adamw_all(ad, grads, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1)
    p0 = np.concatenate([getattr(ad[0][p], n).reshape(-1).numpy() for p in ref.PROJS
                         for n in ("A", "B")])
    return dict(loss=np.float32(loss), grads=flat_grads(grads).astype(np.float32),
                params_l0_after=p0.astype(np.float32))


def tiny_step():
    g = torch.Generator().manual_seed(36)
    W = make_model(g, ref.TINY)
    ad = make_adapters(g, ref.TINY)
    f = lambda t: t.double()
    W = ref.ModelW(embed=f(W.embed), layers=[ref.LayerW(**{k: f(getattr(l, k)) for k in
                   l.__dataclass_fields__}) for l in W.layers], final_norm=f(W.final_norm),
                   lm_head=f(W.lm_head))
    ad = [{p: ref.Adapter(a.A.double(), a.B.double()) for p, a in d.items()} for d in ad]
    win = torch.randint(0, ref.TINY.vocab, (2, 9), generator=g)
    loss, grads = ref.step_autograd(W, ad, win[:, :-1], win[:, 1:], ref.TINY)
    return dict(loss=np.float64(loss), grads=flat_grads(grads))


def quant():
    rng = np.random.default_rng(1004)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    w[0, :6] = [127.0, 0.5, 1.5, -2.5, 2.5, -0.5]
    w[1] = 0.0
    q, s = quantize_rows(w)
    return dict(w=w, q=q, scale=s)


def main():
    np.savez_compressed(HERE / "small_step.npz", **small_step())
    np.savez_compressed(HERE / "tiny_step.npz", **tiny_step())
    np.savez_compressed(HERE / "quant.npz", **quant())
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
