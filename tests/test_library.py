"""CPU: libllmt.so loads, exports every function include/llmt.h declares, and
its host-side argument checks answer before any GPU work (no GPU needed)."""
import ctypes as C

import pytest

import llmt
from oracle import lora_step as ref


def test_library_exports_every_declared_symbol():
    L = llmt.lib()
    names = llmt.header_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_reference_compat_symbols_present():
    # the reference's step API (include/lora.h:66-90, src/train.cu:26-39)
    L = llmt.lib()
    for n in ("transformer_forward_lora", "cross_entropy_forward", "transformer_backward_lora",
              "adamw_step_lora", "lora_weights_init", "lora_weights_free", "lora_grads_alloc",
              "lora_grads_free", "lora_grads_zero", "lora_acts_alloc", "lora_acts_free",
              "lora_forward_add", "scale_add_inplace", "gpu_zero"):
        assert hasattr(L, n), n


def test_qwen3_dims_preset_matches_oracle():
    d = llmt.qwen3_dims()
    o = ref.QWEN3_1_7B
    assert (d.hidden, d.n_layers, d.n_heads, d.n_kv_heads, d.head_dim, d.intermediate, d.vocab,
            d.rank) == (o.hidden, o.n_layers, o.n_heads, o.n_kv_heads, o.head_dim,
                        o.intermediate, o.vocab, o.rank)
    assert d.alpha == 32.0 and abs(d.eps - 1e-6) < 1e-12 and d.theta == 1e6


@pytest.mark.parametrize("field,value", [("head_dim", 64), ("rank", 8), ("n_kv_heads", 3),
                                         ("hidden", 100)])
def test_ctx_create_rejects_unsupported_dims(field, value):
    d = llmt.qwen3_dims()
    setattr(d, field, value)
    h = C.c_void_p()
    rc = llmt.lib().llmt_ctx_create(C.byref(d), 1, 128, 0, None, C.byref(h))
    assert rc == llmt.LLMT_ERR_ARG
    assert llmt.lib().llmt_last_error().decode()
    assert not h.value


def test_standalone_ops_reject_bad_shapes():
    L = llmt.lib()
    # K not a multiple of 32 / M not a multiple of 16: rejected before launch
    assert L.llmt_gemm_f16(C.c_void_p(16), 40, C.c_void_p(16), 40, C.c_void_p(16), 16, 16, 16, 40,
                           None) == llmt.LLMT_ERR_ARG
    assert L.llmt_gemm_f16(C.c_void_p(16), 64, C.c_void_p(16), 64, C.c_void_p(16), 16, 8, 16, 64,
                           None) == llmt.LLMT_ERR_ARG
    assert L.llmt_cross_entropy(C.c_void_p(16), C.c_void_p(16), 10, 8, 3, None, C.c_void_p(16),
                                None, None) == llmt.LLMT_ERR_ARG
    assert L.llmt_attention_fwd(None, None, None, None, None, 1, 8, 4, 3, None) == llmt.LLMT_ERR_ARG


def test_profile_categories_match_header():
    txt = " ".join(llmt.HEADER.read_text().replace("*", " ").split())
    for i, name in enumerate(("forward GEMMs", "backward GEMMs", "lm_head GEMMs", "attention",
                              "row epilogues", "cross-entropy", "LoRA gradients", "AdamW")):
        assert f"{i} {name}" in txt, name
    assert llmt.PROFILE_CATEGORIES == ("gemm_fwd", "gemm_bwd", "gemm_lm_head", "attention",
                                       "row_epilogues", "cross_entropy", "lora_grad", "adamw")


def test_llm_train_cli_rejects_bad_input(tmp_path):
    """The driver exits with status 1 and a message before touching the GPU on
    bad flags, a missing token file or too few tokens (src/train.cu:194-213)."""
    import subprocess
    from pathlib import Path
    import numpy as np
    exe = Path(__file__).resolve().parent.parent / "llm.cu_amd" / "llm_train"
    assert exe.exists(), "llm_train not built (python llm.cu_amd/build.py)"
    run = lambda *a: subprocess.run([str(exe), *a], capture_output=True, text=True, timeout=60)
    r = run("--bogus")
    assert r.returncode == 1 and "unknown" in r.stderr
    r = run("--data", str(tmp_path / "missing.bin"))
    assert r.returncode == 1 and "not found" in r.stderr
    tok = tmp_path / "few.bin"
    np.array([3, 1, 2, 3], dtype="<i4").tofile(tok)
    r = run("--data", str(tok), "--seq-len", "8")
    assert r.returncode == 1 and "need at least 9 tokens, got 3" in r.stderr
    assert "Training config: lr=3.00e-04 steps=1000 seq_len=8" in r.stdout


def test_noalloc_cross_entropy_rejects_inputs_beyond_the_scratch():
    """llmt_cross_entropy_noalloc refuses, before any device work, inputs whose
    statistics exceed its built-in 2 MiB scratch (the pointers are never
    dereferenced: the host-side size check answers first)."""
    f = llmt.lib().llmt_cross_entropy_noalloc
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                  C.c_void_p, C.c_void_p]
    V = 151936
    rows = 14000   # 14000 x 19 chunks > the 262144 statistics of the scratch
    rc = f(C.c_void_p(256), C.c_void_p(256), rows, V, 2, None, C.c_void_p(256), None, None)
    assert rc == llmt.LLMT_ERR_ARG
    assert "exceed" in llmt.lib().llmt_last_error().decode()
    # the largest input that fits is not refused by the size check
    assert 13797 * 19 <= 262144 < 13798 * 19
