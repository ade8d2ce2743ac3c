"""The llm_train driver (llm.cu_amd/llm_train.cpp) end to end on a small
Qwen3-shaped model, through the reference's file formats: fp32 weight files
named after the HF parameters (src/train.cu:56-89), the [int32 n][ids] token
file, in-order (S+1)-token windows (src/train.cu:253-258), the step log line
and the lora_step{N}_layer{L}_{wq..wo}_{A|B}.bin adapter files
(src/train.cu:146-170).  Checks: the first logged loss against the fp32
oracle; the final adapters against the library driven step by step from
Python on the same windows (bit-exact); a resumed run (adapters + AdamW state)
against an uninterrupted one (bit-exact)."""
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

import llmt
from helpers import SMALL, small_problem, write_weights_dir
from oracle import lora_step as ref

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent.parent / "llm.cu_amd" / "llm_train"
S = 64
NWIN = 3
SEED = 1234
DIMS = (f"{SMALL.hidden},{SMALL.n_layers},{SMALL.n_heads},{SMALL.n_kv_heads},"
        f"{SMALL.intermediate},{SMALL.vocab}")


def _write_weights(W, d: Path):
    write_weights_dir(W, d)


def _run(args):
    print("case: llm_train", " ".join(args), flush=True)
    r = subprocess.run([str(EXE), "--dims", DIMS, "--seq-len", str(S), "--seed", str(SEED),
                        *args], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def _losses(out):
    return {int(m.group(1)): float(m.group(2))
            for m in re.finditer(r"^step\s+(\d+)\s+loss ([-0-9.]+)", out, re.M)}


def _adapters(d: Path, step):
    return {p.name.split("_", 2)[2]: p.read_bytes()
            for p in sorted(d.glob(f"lora_step{step}_layer*.bin"))}


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (python llm.cu_amd/build.py)")
    W, _, _, _ = small_problem(SMALL, batch=1, seq_len=S)
    root = tmp_path_factory.mktemp("llm_train")
    g = torch.Generator().manual_seed(99)
    ids = torch.randint(0, SMALL.vocab, (NWIN * (S + 1) + 5,), generator=g, dtype=torch.int32)
    tok = root / "tokens.bin"
    with open(tok, "wb") as f:
        np.array([ids.numel()], dtype="<i4").tofile(f)
        ids.numpy().astype("<i4").tofile(f)
    for run in ("a", "b", "c"):
        _write_weights(W, root / run)
    return dict(W=W, ids=ids, root=root, tok=tok)


def test_first_loss_matches_oracle(files, dev):
    d = files["root"] / "c"
    out = _run(["--data", str(files["tok"]), "--weights", str(d), "--steps", "1",
                "--log-every", "1", "--save-every", "1"])
    assert "Training sequences available: %d" % NWIN in out
    loss = _losses(out)[1]
    # the same seeded init, read back through the library
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=1, seq_len=S)
    try:
        ctx.lora_init(SEED, 0.02, 0.0)
        ad = [{p: ref.Adapter(A.clone(), B.clone()) for p, (A, B) in d.items()}
              for d in llmt.unflatten_adapters(ctx.lora_get("param").cpu(), SMALL)]
    finally:
        ctx.close()
    win = files["ids"][: S + 1]
    logits, _ = ref.model_forward(files["W"], ad, win[None, :-1], SMALL)
    loss_ref, _, _ = ref.cross_entropy(logits, win[1:].long(), ref.valid_rows(1, S))
    assert abs(loss - float(loss_ref)) < 1e-3 + 5e-5   # printed with 4 decimals


def test_matches_library_and_resume(files, dev):
    tok, root = str(files["tok"]), files["root"]
    # uninterrupted 4 steps (window 3 wraps to window 0)
    out_a = _run(["--data", tok, "--weights", str(root / "a"), "--steps", "4",
                  "--log-every", "1", "--save-every", "2"])
    # 2 steps, then resume from the step-2 adapters and AdamW state
    out_b1 = _run(["--data", tok, "--weights", str(root / "b"), "--steps", "2",
                   "--log-every", "1", "--save-every", "2"])
    out_b2 = _run(["--data", tok, "--weights", str(root / "b"), "--steps", "2", "--resume", "2",
                   "--log-every", "1", "--save-every", "2"])
    la, lb = _losses(out_a), {**_losses(out_b1), **_losses(out_b2)}
    assert sorted(la) == [1, 2, 3, 4] and la == lb
    fa, fb = _adapters(root / "a", 4), _adapters(root / "b", 4)
    assert len(fa) == SMALL.n_layers * 8 and fa == fb
    assert (root / "b" / "lora_step2_adamw.bin").exists()
    # the library driven from Python over the same in-order windows
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=1, seq_len=S)
    try:
        ctx.load_weights_dir(root / "a")
        ctx.lora_init(SEED, 0.02, 0.0)
        ids = files["ids"]
        for step in range(1, 5):
            w = (step - 1) % NWIN
            win = ids[w * (S + 1):(w + 1) * (S + 1)].to(dev)
            loss = ctx.step(win[None, :-1].contiguous(), win[None, 1:].contiguous(),
                            llmt.hparams(), step)
            assert abs(loss - la[step]) < 5e-5 + 1e-6
        want = ctx.lora_get("param").cpu()
    finally:
        ctx.close()
    got = np.concatenate([np.frombuffer(fa[f"layer{l}_{p}_{m}.bin"], dtype="<f4")
                          for l in range(SMALL.n_layers) for p in ("wq", "wk", "wv", "wo")
                          for m in ("A", "B")])
    assert np.array_equal(got, want.numpy())


def test_int8_ragged_seq_first_loss_matches_oracle(files, dev):
    """llm_train --int8 at --seq-len 60 (not a multiple of 16): the fp32
    weight files quantised on the device (src/kernels/quantize.cu recipe,
    fp16 scales); the first logged loss against the oracle on the
    dequantised weights."""
    import copy
    from oracle.configs import quantize_model_int8
    S60 = 60
    d = files["root"] / "i8"
    _write_weights(files["W"], d)
    print("case: llm_train --int8 --seq-len 60", flush=True)
    r = subprocess.run([str(EXE), "--dims", DIMS, "--seq-len", str(S60), "--seed", str(SEED),
                        "--int8", "--data", str(files["tok"]), "--weights", str(d), "--steps", "1",
                        "--log-every", "1", "--save-every", "1"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "(int8)" in r.stdout
    loss = _losses(r.stdout)[1]
    ctx = llmt.Context(llmt.make_dims(SMALL), max_batch=1, seq_len=S60)
    try:
        ctx.lora_init(SEED, 0.02, 0.0)
        ad = [{p: ref.Adapter(A.clone(), B.clone()) for p, (A, B) in dd.items()}
              for dd in llmt.unflatten_adapters(ctx.lora_get("param").cpu(), SMALL)]
    finally:
        ctx.close()
    Wq, _ = quantize_model_int8(copy.deepcopy(files["W"]))
    win = files["ids"][: S60 + 1]
    logits, _ = ref.model_forward(Wq, ad, win[None, :-1], SMALL)
    loss_ref, _, _ = ref.cross_entropy(logits, win[1:].long(), ref.valid_rows(1, S60))
    assert abs(loss - float(loss_ref)) < 1e-3 + 5e-5
