"""ctypes binding of libllmt.so (include/llmt.h) for tests and the bench.

Tensors are torch tensors used only as device-memory plumbing: every
computation happens in libllmt.so's HIP kernels.  ``lib()`` raises if the
shared library has not been built (``python llm.cu_amd/build.py``); there is
no fallback path.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
LIB_PATH = PKG / "libllmt.so"
HEADER = ROOT / "include" / "llmt.h"

vp, i32, f32, sz, u64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64
fp = C.POINTER(C.c_float)

LLMT_OK, LLMT_ERR_ARG, LLMT_ERR_HIP, LLMT_ERR_IO, LLMT_ERR_STATE = 0, -1, -2, -3, -4
PROJ = {"wq": 0, "wk": 1, "wv": 2, "wo": 3}
KIND = {"param": 0, "grad": 1, "m": 2, "v": 3}


class LlmtError(RuntimeError):
    pass


class Dims(C.Structure):
    _fields_ = [(n, i32) for n in ("hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                   "intermediate", "vocab", "rank")] + \
               [(n, f32) for n in ("alpha", "eps", "theta")]


class HParams(C.Structure):
    _fields_ = [(n, f32) for n in ("lr", "beta1", "beta2", "eps", "wd")]


# name -> (restype, argtypes)
_PROTOS = {
    "llmt_last_error": (C.c_char_p, []),
    "llmt_dims_qwen3_1_7b": (None, [C.POINTER(Dims)]),
    "llmt_gemm_f16": (i32, [vp, i32, vp, i32, vp, i32, i32, i32, i32, vp]),
    "llmt_gemm_i8": (i32, [vp, i32, vp, i32, vp, vp, i32, i32, i32, i32, vp]),
    "llmt_quantize_rows_i8": (i32, [vp, i32, i32, vp, vp, vp]),
    "llmt_cross_entropy": (i32, [vp, vp, i32, i32, i32, vp, vp, vp, vp]),
    "llmt_lm_head_ce": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp]),
    "llmt_attention_fwd": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]),
    "llmt_attention_bwd": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]),
    "llmt_attention_block_bwd": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                       f32, f32, vp]),
    "llmt_ctx_create": (i32, [C.POINTER(Dims), i32, i32, i32, vp, C.POINTER(vp)]),
    "llmt_ctx_destroy": (i32, [vp]),
    "llmt_ctx_device_bytes": (sz, [vp]),
    "llmt_set_layer_f16": (i32, [vp, i32] + [vp] * 11),
    "llmt_set_layer_i8": (i32, [vp, i32, C.POINTER(vp), C.POINTER(vp), vp, vp, vp, vp]),
    "llmt_set_embed_f16": (i32, [vp, vp, vp]),
    "llmt_load_weights_dir": (i32, [vp, C.c_char_p]),
    "llmt_lora_numel": (sz, [vp]),
    "llmt_lora_offset": (sz, [vp, i32, i32, i32]),
    "llmt_lora_copy": (i32, [vp, i32, vp, i32]),
    "llmt_lora_save": (i32, [vp, C.c_char_p, i32]),
    "llmt_lora_load": (i32, [vp, C.c_char_p, i32]),
    "llmt_lora_init": (i32, [vp, u64, f32, f32]),
    "llmt_step": (i32, [vp, vp, vp, i32, C.POINTER(HParams), i32, fp]),
    "llmt_forward_backward": (i32, [vp, vp, vp, i32, fp]),
    "llmt_set_graph": (i32, [vp, i32]),
    "llmt_logits": (vp, [vp]),
    "llmt_layer_forward": (i32, [vp, i32, vp, vp, i32]),
    "llmt_layer_backward": (i32, [vp, i32, vp, vp, i32]),
    "llmt_adamw": (i32, [vp, C.POINTER(HParams), i32]),
}

_lib = None


def lib():
    """Load libllmt.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise LlmtError(f"{LIB_PATH} is not built; run python llm.cu_amd/build.py")
        L = C.CDLL(str(LIB_PATH))
        for name, (rt, at) in _PROTOS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = rt
            fn.argtypes = at
        _lib = L
    return _lib


def header_functions():
    """Every function name declared in include/llmt.h."""
    txt = HEADER.read_text()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?[\s\*](\w+)\s*\(", txt, flags=re.M)
    return sorted(set(n for n in names if n not in ("if", "while", "for", "return", "sizeof")))


def check(rc: int):
    if rc != LLMT_OK:
        raise LlmtError(f"llmt error {rc}: {lib().llmt_last_error().decode()}")


def ptr(t):
    """Device (or host) address of a tensor, or None."""
    return None if t is None else C.c_void_p(t.data_ptr())


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def qwen3_dims() -> Dims:
    d = Dims()
    lib().llmt_dims_qwen3_1_7b(C.byref(d))
    return d


def make_dims(o) -> Dims:
    """Dims from an object with the oracle's Dims attribute names."""
    return Dims(o.hidden, o.n_layers, o.n_heads, o.n_kv_heads, o.head_dim, o.intermediate,
                o.vocab, o.rank, float(o.alpha), float(o.eps), float(o.theta))


# ------------------------------------------------------------------ operators

def gemm_f16(A, B, out=None, stream=None):
    """out[M, N] fp32 = A[M, K] @ B[N, K]^T with fp16 inputs."""
    import torch
    M, K = A.shape
    N = B.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.float32, device=A.device)
    check(lib().llmt_gemm_f16(ptr(A), A.stride(0), ptr(B), B.stride(0), ptr(out), out.stride(0),
                              M, N, K, stream_ptr(stream)))
    return out


def gemm_i8(A, q, scale16, out=None, stream=None):
    import torch
    M, K = A.shape
    N = q.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=torch.float32, device=A.device)
    check(lib().llmt_gemm_i8(ptr(A), A.stride(0), ptr(q), q.stride(0), ptr(scale16), ptr(out),
                             out.stride(0), M, N, K, stream_ptr(stream)))
    return out


def quantize_rows_i8(w, stream=None):
    import torch
    rows, cols = w.shape
    q = torch.empty(rows, cols, dtype=torch.int8, device=w.device)
    s = torch.empty(rows, dtype=torch.float32, device=w.device)
    check(lib().llmt_quantize_rows_i8(ptr(w), rows, cols, ptr(q), ptr(s), stream_ptr(stream)))
    return q, s


def cross_entropy(logits, targets, seq_len, want_dlogits=True, stream=None):
    """Returns (loss_mean [1], loss_rows [rows], dlogits or None)."""
    import torch
    rows, V = logits.shape
    dl = torch.empty_like(logits) if want_dlogits else None
    lr = torch.empty(rows, dtype=torch.float32, device=logits.device)
    lm = torch.empty(1, dtype=torch.float32, device=logits.device)
    check(lib().llmt_cross_entropy(ptr(logits), ptr(targets), rows, V, seq_len, ptr(dl), ptr(lr),
                                   ptr(lm), stream_ptr(stream)))
    return lm, lr, dl
