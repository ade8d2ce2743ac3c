"""CPU oracle for the llm.cu LoRA training step (TEST INFRASTRUCTURE ONLY).

This package restates, on the CPU in fp32 PyTorch / numpy, the math of the
reference's ``llm_train`` step (``src/train.cu:251-302`` in
visheshnarayan/llm.cu).  It is the checker for the HIP implementation in
``llm.cu_amd/``: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path never
calls into it; the HIP library fails loudly when its extension is missing.

Modules:
  ``lora_step``  forward, closed-form backward, autograd step, AdamW, CE
  ``quant``      bit-exact int8 per-row quantizer (numpy float32 IEEE ops)
  ``configs``    seeded synthetic inputs for the five benchmark configs

Parity pinning (what checks each function; tests live in ``tests/``):
  * every closed-form backward is checked against ``torch.autograd`` and, at
    float64 on tiny shapes, against central finite differences;
  * CE: ``F.cross_entropy`` and the known answer ln(V) for all-zero logits;
  * AdamW: ``torch.optim.AdamW`` (the identical decoupled-decay formula);
  * RoPE: inverse round trip, norm preservation, identity at position 0;
  * attention: rows of P sum to 1, sum_j dS_ij = 0, autograd, brute force;
  * int8 quantizer: brute-force per-element float32 recomputation and the
    round-half-even special cases;
  * whole step: the closed-form backward against autograd through the full
    tiny model, and the quirk switches reproduce the reference's deviations.
No function is "parity unpinned".
"""
