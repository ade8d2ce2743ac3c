"""GPU parity of the whole LoRA training step (llmt_forward_backward /
llmt_step through the C ABI) against the exact fp32 CPU oracle.

Bars (north star): loss within 1e-3 absolute; every adapter-gradient tensor
within 1e-2 relative L2 of the fp32 reference; integer work bit-exact."""
import pytest
import torch

import llmt
from helpers import SMALL, grad_errors, oracle_grads, rel_l2, small_problem, upload_model
from oracle import lora_step as ref

pytestmark = pytest.mark.gpu

LOSS_TOL = 1e-3
GRAD_TOL = 1e-2


@pytest.fixture(scope="module")
def small(dev):
    W, ad, tok, tgt = small_problem()
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, SMALL)
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=2, seq_len=64)
    upload_model(ctx, W, dev)
    ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
    yield dict(W=W, ad=ad, tok=tok.to(dev), tgt=tgt.to(dev), loss_ref=float(loss_ref),
               grads_ref=grads_ref, ctx=ctx)
    ctx.close()


def test_small_model_loss_and_grads(small):
    ctx = small["ctx"]
    print(f"case: small model {SMALL}, B=2 S=64", flush=True)
    loss = ctx.forward_backward(small["tok"], small["tgt"])
    assert abs(loss - small["loss_ref"]) < LOSS_TOL
    errs = grad_errors(ctx.lora_get("grad"), small["grads_ref"], SMALL)
    worst = max(errs.items(), key=lambda kv: kv[1])
    print("worst grad rel-L2", worst, flush=True)
    assert worst[1] < GRAD_TOL, worst


def test_deterministic_and_graph_replay(small):
    ctx = small["ctx"]
    ctx.set_graph(False)
    l0 = ctx.forward_backward(small["tok"], small["tgt"])
    g0 = ctx.lora_get("grad").clone()
    ctx.set_graph(True)
    try:
        for _ in range(3):
            l1 = ctx.forward_backward(small["tok"], small["tgt"])
            g1 = ctx.lora_get("grad")
            assert l1 == l0
            assert torch.equal(g1, g0)      # fixed reduction order: bit-identical
            torch.cuda.synchronize()
    finally:
        ctx.set_graph(False)


def test_batch_one_uses_first_rows(small, dev):
    # batch 1 through a batch-2 context = the oracle on the first sequence
    W, ad = small["W"], small["ad"]
    tok, tgt = small["tok"][:1].contiguous(), small["tgt"][:1].contiguous()
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok.cpu(), tgt.cpu(), SMALL)
    loss = small["ctx"].forward_backward(tok, tgt)
    assert abs(loss - float(loss_ref)) < LOSS_TOL
    errs = grad_errors(small["ctx"].lora_get("grad"), grads_ref, SMALL)
    assert max(errs.values()) < GRAD_TOL


def test_adamw_step_matches_oracle(small, dev):
    ctx = small["ctx"]
    hp = llmt.hparams()
    # restart from the same adapters with zero moments
    ad = [{p: ref.Adapter(a.A.clone(), a.B.clone()) for p, a in d.items()} for d in small["ad"]]
    ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
    zeros = torch.zeros(ctx.lora_numel, device=dev)
    ctx.lora_set("m", zeros)
    ctx.lora_set("v", zeros)
    try:
        loss = ctx.step(small["tok"], small["tgt"], hp, 1)
        assert abs(loss - small["loss_ref"]) < LOSS_TOL
        ref.adamw_all(ad, small["grads_ref"], hp.lr, hp.beta1, hp.beta2, hp.eps, hp.wd, 1)
        want = llmt.flatten_adapters(ad)
        got = ctx.lora_get("param").cpu()
        assert rel_l2(got, want) < GRAD_TOL
        want_m = llmt.flatten_adapters(ad, attr=("mA", "mB"))
        assert rel_l2(ctx.lora_get("m").cpu(), want_m) < GRAD_TOL
        # second step: the forward now reads the fp16 shadows AdamW refreshed
        loss2 = ctx.step(small["tok"], small["tgt"], hp, 2)
        ad2 = [{p: ref.Adapter(a.A, a.B) for p, a in d.items()} for d in ad]
        loss2_ref, _, _ = oracle_grads(small["W"], ad2, small["tok"].cpu(), small["tgt"].cpu(),
                                       SMALL)
        assert abs(loss2 - float(loss2_ref)) < LOSS_TOL
    finally:
        # the module's later tests compare against the fixture's adapters
        ctx.lora_set("param", llmt.flatten_adapters(small["ad"]).to(dev))
        ctx.lora_set("m", zeros)
        ctx.lora_set("v", zeros)


def test_lora_save_load_roundtrip(small, tmp_path, dev):
    ctx = small["ctx"]
    before = ctx.lora_get("param").clone()
    ctx.lora_save(tmp_path, 5)
    names = sorted(p.name for p in tmp_path.iterdir())
    assert len(names) == SMALL.n_layers * 8
    assert "lora_step5_layer0_wq_A.bin" in names
    a = torch.from_numpy(__import__("numpy").fromfile(tmp_path / "lora_step5_layer1_wo_B.bin",
                                                      dtype="<f4"))
    off = ctx.lora_offset(1, "wo", 1)
    assert torch.equal(a, before[off:off + a.numel()].cpu())
    ctx.lora_set("param", torch.zeros_like(before))
    ctx.lora_load(tmp_path, 5)
    assert torch.equal(ctx.lora_get("param"), before)


def test_lora_peft_round_trip(small, tmp_path, dev):
    """Adapters saved by the library -> PEFT safetensors -> adapter files ->
    llmt_lora_load: the same parameters bit for bit, and each PEFT tensor is
    the context's slice for that layer and projection."""
    import numpy as np
    from llmt import peft
    ctx = small["ctx"]
    dims = peft.AdapterDims(SMALL.n_layers, SMALL.hidden, SMALL.n_heads, SMALL.n_kv_heads,
                            SMALL.head_dim, SMALL.rank, SMALL.alpha)
    before = ctx.lora_get("param").clone()
    (tmp_path / "a").mkdir()
    ctx.lora_save(tmp_path / "a", 4)
    peft.to_peft(tmp_path / "a", 4, tmp_path / "hf", dims)
    state = peft.load_peft(tmp_path / "hf")
    q_a = state["base_model.model.model.layers.1.self_attn.q_proj.lora_A.weight"]
    off = ctx.lora_offset(1, "wq", 0)
    assert np.array_equal(q_a.ravel(), before[off:off + q_a.size].cpu().numpy())
    peft.from_peft(tmp_path / "hf", tmp_path / "b", 9, dims)
    ctx.lora_set("param", torch.zeros_like(before))
    ctx.lora_load(tmp_path / "b", 9)
    assert torch.equal(ctx.lora_get("param"), before)


def test_small_model_matches_golden_fixture(small, dev):
    """Same step against the committed fixture (tests/golden/small_step.npz)."""
    import numpy as np
    from pathlib import Path
    want = np.load(Path(__file__).resolve().parent / "golden" / "small_step.npz")
    ctx = small["ctx"]
    ad = small["ad"]
    ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
    loss = ctx.forward_backward(small["tok"], small["tgt"])
    assert abs(loss - float(want["loss"])) < LOSS_TOL
    got = ctx.lora_get("grad").cpu().double()
    w = torch.from_numpy(want["grads"]).double()
    assert float((got - w).norm() / w.norm()) < GRAD_TOL


@pytest.mark.parametrize("rows", ["2", "3", "4", "8"])
def test_rows_per_workgroup(small, monkeypatch, rows):
    """The parallel-rows epilogues (o_post, resid_norm, and norm_bwd with and
    without the attention norm's three adapter terms: several token rows a
    workgroup side by side, adapter values loaded once), including a partial
    last group (128 rows / 3), give the same step as the oracle."""
    monkeypatch.setenv("LLMT_ROWS_PER_WG", rows)
    print(f"case: rows a workgroup {rows}", flush=True)
    ctx = small["ctx"]
    ctx.set_graph(False)
    loss = ctx.forward_backward(small["tok"], small["tgt"])
    assert abs(loss - small["loss_ref"]) < LOSS_TOL
    errs = grad_errors(ctx.lora_get("grad"), small["grads_ref"], SMALL)
    assert max(errs.values()) < GRAD_TOL


@pytest.mark.parametrize("nq,nkv,hoist", [(2, 2, "1"), (8, 2, "1"), (8, 2, "0"), (16, 8, "1")])
def test_qk_backward_head_layouts(dev, monkeypatch, nq, nkv, hoist):
    """The QK-norm / RoPE backward for GQA groups 1, 4 and 2 with one, two
    and three heads a wave (every load of a row issued before the math) and
    the one-head-at-a-time form (hoist 0) give the oracle's step."""
    monkeypatch.setenv("LLMT_QK_BWD_HOIST", hoist)
    dims = ref.Dims(hidden=256, n_layers=2, n_heads=nq, n_kv_heads=nkv, head_dim=128,
                    intermediate=512, vocab=2048)
    print(f"case: heads {nq}/{nkv} hoist {hoist}", flush=True)
    W, ad, tok, tgt = small_problem(dims)
    loss_ref, grads_ref, _ = oracle_grads(W, ad, tok, tgt, dims)
    ctx = llmt.Context(llmt.make_dims(dims), max_batch=2, seq_len=64)
    try:
        upload_model(ctx, W, dev)
        ctx.lora_set("param", llmt.flatten_adapters(ad).to(dev))
        loss = ctx.forward_backward(tok.to(dev), tgt.to(dev))
        assert abs(loss - float(loss_ref)) < LOSS_TOL
        errs = grad_errors(ctx.lora_get("grad"), grads_ref, dims)
        assert max(errs.values()) < GRAD_TOL, max(errs.items(), key=lambda kv: kv[1])
    finally:
        ctx.close()


def test_graph_copies_inputs_each_replay(small, dev):
    """With the input copies inside the step graph: new token contents under
    the same pointers, then other buffers, give the eager step's loss and
    gradients on every replay (forward + backward, and the full step whose
    AdamW hyper-parameters are staged for each step)."""
    ctx = small["ctx"]
    g = torch.Generator().manual_seed(99)
    wins = [torch.randint(0, SMALL.vocab, (2, 65), generator=g, dtype=torch.int32) for _ in range(3)]
    ref = []
    ctx.set_graph(False)
    for w in wins:
        ref.append((ctx.forward_backward(w[:, :-1].contiguous().to(dev), w[:, 1:].contiguous().to(dev)),
                    ctx.lora_get("grad").clone()))
    tok = torch.empty(2, 64, dtype=torch.int32, device=dev)
    tgt = torch.empty(2, 64, dtype=torch.int32, device=dev)
    ctx.set_graph(True)
    try:
        for i, w in enumerate(wins):          # same pointers, new contents
            tok.copy_(w[:, :-1])
            tgt.copy_(w[:, 1:])
            loss = ctx.forward_backward(tok, tgt)
            assert loss == ref[i][0]
            assert torch.equal(ctx.lora_get("grad"), ref[i][1])
        w = wins[0]                            # other buffers: the graph is rebuilt
        loss = ctx.forward_backward(w[:, :-1].contiguous().to(dev), w[:, 1:].contiguous().to(dev))
        assert loss == ref[0][0]
        # full steps: AdamW with per-step bias corrections, graph vs eager
        p0 = ctx.lora_get("param").clone()
        m0, v0 = ctx.lora_get("m").clone(), ctx.lora_get("v").clone()
        hp = llmt.hparams()
        tok.copy_(wins[1][:, :-1])
        tgt.copy_(wins[1][:, 1:])
        graph_losses = [ctx.step(tok, tgt, hp, s) for s in (1, 2)]
        p_graph = ctx.lora_get("param").clone()
        ctx.set_graph(False)
        ctx.lora_set("param", p0)
        ctx.lora_set("m", m0)
        ctx.lora_set("v", v0)
        eager_losses = [ctx.step(tok, tgt, hp, s) for s in (1, 2)]
        assert graph_losses == eager_losses
        assert torch.equal(ctx.lora_get("param"), p_graph)
        ctx.lora_set("param", p0)
        ctx.lora_set("m", m0)
        ctx.lora_set("v", v0)
    finally:
        ctx.set_graph(False)
