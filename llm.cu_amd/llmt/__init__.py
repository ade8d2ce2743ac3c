"""ctypes binding of libllmt.so (include/llmt.h) for tests and the bench.

Tensors are torch tensors used only as device-memory plumbing: every
computation happens in libllmt.so's HIP kernels.  ``lib()`` raises if the
shared library has not been built (``python llm.cu_amd/build.py``); there is
no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
ROOT = PKG.parent
# Always the in-tree build: tests and the bench must measure the library
# built from this tree, so an override of the path is refused outright.
if os.environ.get("LLMT_LIB"):
    raise ImportError("LLMT_LIB is set; llmt loads only the in-tree llm.cu_amd/libllmt.so "
                      "(unset LLMT_LIB)")
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
    "llmt_set_lm_head_f16": (i32, [vp, vp]),
    "llmt_load_weights_dir": (i32, [vp, C.c_char_p]),
    "llmt_lora_numel": (sz, [vp]),
    "llmt_lora_offset": (sz, [vp, i32, i32, i32]),
    "llmt_lora_copy": (i32, [vp, i32, vp, i32]),
    "llmt_lora_save": (i32, [vp, C.c_char_p, i32]),
    "llmt_lora_load": (i32, [vp, C.c_char_p, i32]),
    "llmt_lora_save_state": (i32, [vp, C.c_char_p, i32]),
    "llmt_lora_load_state": (i32, [vp, C.c_char_p, i32]),
    "llmt_lora_init": (i32, [vp, u64, f32, f32]),
    "llmt_step": (i32, [vp, vp, vp, i32, C.POINTER(HParams), i32, fp]),
    "llmt_forward_backward": (i32, [vp, vp, vp, i32, fp]),
    "llmt_set_graph": (i32, [vp, i32]),
    "llmt_logits": (vp, [vp]),
    "llmt_layer_in": (vp, [vp, i32]),
    "llmt_layer_forward": (i32, [vp, i32, vp, vp, i32]),
    "llmt_layer_backward": (i32, [vp, i32, vp, vp, i32]),
    "llmt_adamw": (i32, [vp, C.POINTER(HParams), i32]),
    "llmt_head_ce": (i32, [vp, vp, vp, i32, fp, vp, vp]),
    "llmt_profile_kernels": (i32, [vp, vp, vp, i32, C.POINTER(HParams), i32, i32, i32,
                                   C.POINTER(C.c_int), C.POINTER(C.c_char_p),
                                   C.POINTER(C.c_int), C.POINTER(C.c_int), fp,
                                   C.POINTER(C.c_double), C.POINTER(C.c_double)]),
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


# ------------------------------------------------------------------ training context

PROFILE_CATEGORIES = ("gemm_fwd", "gemm_bwd", "gemm_lm_head", "attention", "row_epilogues",
                      "cross_entropy", "lora_grad", "adamw")


def hparams(lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, wd=0.01) -> HParams:
    """AdamW hyper-parameters; defaults are src/train.cu:174-182."""
    return HParams(lr, beta1, beta2, eps, wd)


class Context:
    """One llmt_ctx: frozen weights, adapters, stashes and workspaces of the
    LoRA training step for up to ``max_batch`` sequences of ``seq_len``."""

    def __init__(self, dims: Dims, max_batch: int, seq_len: int, int8: bool = False, stream=None):
        self.dims = dims
        self.max_batch = max_batch
        self.seq_len = seq_len
        h = vp()
        sp = None if stream is None else C.c_void_p(stream.cuda_stream)
        check(lib().llmt_ctx_create(C.byref(dims), max_batch, seq_len, 1 if int8 else 0, sp,
                                    C.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().llmt_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def device_bytes(self) -> int:
        return lib().llmt_ctx_device_bytes(self.h)

    # -- weights
    def set_layer_f16(self, layer, wq, wk, wv, wo, w_gate, w_up, w_down, attn_norm, ffn_norm,
                      q_norm, k_norm):
        check(lib().llmt_set_layer_f16(self.h, layer, *(ptr(t) for t in (
            wq, wk, wv, wo, w_gate, w_up, w_down, attn_norm, ffn_norm, q_norm, k_norm))))

    def set_layer_i8(self, layer, qs, scales16, attn_norm, ffn_norm, q_norm, k_norm):
        qa = (vp * 7)(*(t.data_ptr() for t in qs))
        sa = (vp * 7)(*(t.data_ptr() for t in scales16))
        check(lib().llmt_set_layer_i8(self.h, layer, qa, sa, ptr(attn_norm), ptr(ffn_norm),
                                      ptr(q_norm), ptr(k_norm)))

    def set_embed_f16(self, embed, final_norm):
        check(lib().llmt_set_embed_f16(self.h, ptr(embed), ptr(final_norm)))

    def set_lm_head_f16(self, lm_head):
        """An untied lm_head [V, H] fp16 (llmt_set_lm_head_f16)."""
        check(lib().llmt_set_lm_head_f16(self.h, ptr(lm_head)))

    def load_weights_dir(self, path):
        check(lib().llmt_load_weights_dir(self.h, str(path).encode()))

    # -- adapters
    @property
    def lora_numel(self) -> int:
        return lib().llmt_lora_numel(self.h)

    def lora_offset(self, layer, proj, is_b) -> int:
        return lib().llmt_lora_offset(self.h, layer, PROJ[proj] if isinstance(proj, str) else proj,
                                      int(is_b))

    def lora_set(self, kind: str, flat):
        """Copy a flat fp32 tensor (device or host) into an arena."""
        flat = flat.contiguous()
        assert flat.numel() == self.lora_numel and flat.dtype.is_floating_point
        check(lib().llmt_lora_copy(self.h, KIND[kind], ptr(flat), 1))

    def lora_get(self, kind: str, device="cuda"):
        import torch
        out = torch.empty(self.lora_numel, dtype=torch.float32, device=device)
        check(lib().llmt_lora_copy(self.h, KIND[kind], ptr(out), 0))
        return out

    def lora_init(self, seed: int, a_std: float, b_std: float):
        check(lib().llmt_lora_init(self.h, seed, a_std, b_std))

    def lora_save(self, path, step: int):
        check(lib().llmt_lora_save(self.h, str(path).encode(), step))

    def lora_load(self, path, step: int):
        check(lib().llmt_lora_load(self.h, str(path).encode(), step))

    def lora_save_state(self, path, step: int):
        """AdamW moments to <path>/lora_step{step}_adamw.bin (for resuming)."""
        check(lib().llmt_lora_save_state(self.h, str(path).encode(), step))

    def lora_load_state(self, path, step: int):
        check(lib().llmt_lora_load_state(self.h, str(path).encode(), step))

    # -- the step
    def _check_tokens(self, tokens, targets):
        """tokens/targets must be int32 device tensors [B, seq_len] with
        1 <= B <= max_batch, contiguous (the library copies B * seq_len ids
        from each pointer; the step graph repeats that copy on every replay)."""
        import torch
        for name, t in (("tokens", tokens), ("targets", targets)):
            if not isinstance(t, torch.Tensor):
                raise LlmtError(f"{name} must be a torch tensor")
            if t.dtype != torch.int32:
                raise LlmtError(f"{name} must be int32 (got {t.dtype})")
            if not t.is_cuda:
                raise LlmtError(f"{name} must be a device tensor")
            if not t.is_contiguous():
                raise LlmtError(f"{name} must be contiguous")
            if t.dim() != 2 or t.shape[1] != self.seq_len or not 1 <= t.shape[0] <= self.max_batch:
                raise LlmtError(f"{name} must be [B, {self.seq_len}] with 1 <= B <= "
                                f"{self.max_batch} (got {tuple(t.shape)})")
        if tokens.shape != targets.shape:
            raise LlmtError(f"tokens {tuple(tokens.shape)} and targets {tuple(targets.shape)} differ")
        return tokens.shape[0]

    def set_graph(self, enable: bool):
        check(lib().llmt_set_graph(self.h, int(enable)))

    def step(self, tokens, targets, hp: HParams, step: int) -> float:
        B = self._check_tokens(tokens, targets)
        loss = C.c_float()
        check(lib().llmt_step(self.h, ptr(tokens), ptr(targets), B, C.byref(hp), step,
                              C.byref(loss)))
        return loss.value

    def forward_backward(self, tokens, targets) -> float:
        B = self._check_tokens(tokens, targets)
        loss = C.c_float()
        check(lib().llmt_forward_backward(self.h, ptr(tokens), ptr(targets), B, C.byref(loss)))
        return loss.value

    def layer_in(self, layer, rows):
        """A copy of the fp32 residual stream [rows, H] at the input of
        `layer` from the last forward (llmt_layer_in)."""
        import torch
        addr = lib().llmt_layer_in(self.h, layer)
        if not addr:
            raise LlmtError(f"llmt_layer_in: no layer {layer}")
        H = self.dims.hidden

        class _View:
            __cuda_array_interface__ = {"shape": (rows, H), "typestr": "<f4",
                                        "data": (addr, False), "version": 3, "strides": None}
        return torch.as_tensor(_View(), device="cuda").clone()

    def logits(self, rows):
        """A copy of the first `rows` rows of the fp32 logits of the last
        forward (llmt_logits)."""
        import torch
        addr = lib().llmt_logits(self.h)
        V = self.dims.vocab

        class _View:
            __cuda_array_interface__ = {"shape": (rows, V), "typestr": "<f4",
                                        "data": (addr, False), "version": 3, "strides": None}
        return torch.as_tensor(_View(), device="cuda").clone()

    def head_ce(self, hidden16, targets, want_dlogits=False):
        """C1 on the context's tied embedding: (loss, dlogits or None, dhidden)."""
        import torch
        T = hidden16.shape[0]
        loss = C.c_float()
        dl = torch.empty(T, self.dims.vocab, dtype=torch.float32, device=hidden16.device) \
            if want_dlogits else None
        dh = torch.empty(T, self.dims.hidden, dtype=torch.float32, device=hidden16.device)
        check(lib().llmt_head_ce(self.h, ptr(hidden16), ptr(targets), T // self.seq_len,
                                 C.byref(loss), ptr(dl), ptr(dh)))
        return loss.value, dl, dh

    def layer_forward(self, layer, x, batch):
        import torch
        y = torch.empty_like(x)
        check(lib().llmt_layer_forward(self.h, layer, ptr(x), ptr(y), batch))
        return y

    def layer_backward(self, layer, dy, batch):
        import torch
        dx = torch.empty_like(dy)
        check(lib().llmt_layer_backward(self.h, layer, ptr(dy), ptr(dx), batch))
        return dx

    def profile_kernels(self, tokens, targets, hp: HParams, step: int, reps: int = 5):
        """Per kernel kind of one step (llmt_profile_kernels): a list of dicts
        with name, category, launches (per step), us (average launch
        duration), flops and bytes (per launch; GEMMs only).  The adapters
        advance by one AdamW step."""
        mx = 256
        ns = C.c_int()
        names = (C.c_char_p * mx)()
        cats, nl = (C.c_int * mx)(), (C.c_int * mx)()
        us = (C.c_float * mx)()
        fl, by = (C.c_double * mx)(), (C.c_double * mx)()
        check(lib().llmt_profile_kernels(self.h, ptr(tokens), ptr(targets),
                                         self._check_tokens(tokens, targets), C.byref(hp), step,
                                         reps, mx, C.byref(ns), names, cats, nl, us, fl, by))
        return [dict(name=names[k].decode(), category=PROFILE_CATEGORIES[cats[k]],
                     launches=nl[k], us=us[k], flops=fl[k], bytes=by[k])
                for k in range(ns.value)]


def flatten_adapters(adapters, attr=("A", "B")):
    """Adapters as list-of-dicts (layer -> proj -> object with A, B) -> one
    flat fp32 tensor in the arena order: layer by layer, q, k, v, o, A then B."""
    import torch
    parts = []
    for d in adapters:
        for p in ("wq", "wk", "wv", "wo"):
            for a in attr:
                parts.append(getattr(d[p], a).reshape(-1).float())
    return torch.cat(parts)


def unflatten_adapters(flat, dims):
    """Inverse of flatten_adapters: list of {proj: (A, B)} tensors (views)."""
    r = dims.rank
    q, kv, hd = dims.n_heads * dims.head_dim, dims.n_kv_heads * dims.head_dim, dims.hidden
    shapes = {"wq": (q, hd), "wk": (kv, hd), "wv": (kv, hd), "wo": (hd, q)}
    out, off = [], 0
    for _ in range(dims.n_layers):
        d = {}
        for p in ("wq", "wk", "wv", "wo"):
            d_out, d_in = shapes[p]
            A = flat[off:off + r * d_in].view(r, d_in)
            off += r * d_in
            B = flat[off:off + d_out * r].view(d_out, r)
            off += d_out * r
            d[p] = (A, B)
        out.append(d)
    assert off == flat.numel()
    return out


def lm_head_ce(hidden16, W16, targets, seq_len, want_dlogits=True, stream=None):
    """Standalone C1: (loss_mean [1], dlogits or None, dhidden [T, H])."""
    import torch
    T, H = hidden16.shape
    V = W16.shape[0]
    lm = torch.empty(1, dtype=torch.float32, device=hidden16.device)
    dl = torch.empty(T, V, dtype=torch.float32, device=hidden16.device) if want_dlogits else None
    dh = torch.empty(T, H, dtype=torch.float32, device=hidden16.device)
    check(lib().llmt_lm_head_ce(ptr(hidden16), ptr(W16), ptr(targets), T, seq_len, H, V, ptr(lm),
                                ptr(dl), ptr(dh), stream_ptr(stream)))
    return lm, dl, dh


def attention_fwd(q, k, v, stream=None):
    """q [B,S,nq,128], k/v [B,S,nkv,128] fp16 -> (o fp16 like q, lse fp32 [B,nq,S])."""
    import torch
    B, S, nq, _ = q.shape
    nkv = k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty(B, nq, S, dtype=torch.float32, device=q.device)
    check(lib().llmt_attention_fwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), B, S, nq, nkv,
                                   stream_ptr(stream)))
    return o, lse


def attention_bwd(q, k, v, o, lse, dout32, stream=None):
    """Gradients (fp32) w.r.t. q, k, v of the causal GQA attention."""
    import torch
    B, S, nq, _ = q.shape
    nkv = k.shape[2]
    dq = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    dk = torch.empty(k.shape, dtype=torch.float32, device=q.device)
    dv = torch.empty(v.shape, dtype=torch.float32, device=q.device)
    check(lib().llmt_attention_bwd(ptr(q), ptr(k), ptr(v), ptr(o), ptr(lse), ptr(dout32), ptr(dq),
                                   ptr(dk), ptr(dv), B, S, nq, nkv, stream_ptr(stream)))
    return dq, dk, dv


def attention_block_bwd(q_raw, k_raw, v, q_norm, k_norm, dout16, theta=1e6, eps=1e-6, stream=None):
    """Config C3: QK-norm + RoPE + flash attention forward and backward."""
    import torch
    B, S, nq, _ = q_raw.shape
    nkv = k_raw.shape[2]
    dq = torch.empty(q_raw.shape, dtype=torch.float32, device=q_raw.device)
    dk = torch.empty(k_raw.shape, dtype=torch.float32, device=q_raw.device)
    dv = torch.empty(v.shape, dtype=torch.float32, device=q_raw.device)
    check(lib().llmt_attention_block_bwd(ptr(q_raw), ptr(k_raw), ptr(v), ptr(q_norm), ptr(k_norm),
                                         ptr(dout16), ptr(dq), ptr(dk), ptr(dv), B, S, nq, nkv,
                                         theta, eps, stream_ptr(stream)))
    return dq, dk, dv
