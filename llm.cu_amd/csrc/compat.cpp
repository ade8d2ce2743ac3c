// compat.cpp — the reference's own step API (include/lora.h:66-90,
// src/train.cu:26-39), extern "C", so a train.cu-style driver links
// unchanged.  It is a shim over one lazily created native context (Qwen3-1.7B
// dimensions, batch 1, the caller's seq_len) on its own stream, which is
// blocking with respect to the legacy default stream the reference uses.
//
// Behaviour kept from the reference: failures print to stderr and exit
// (include/utils.h:10-28); the caller owns the workspaces and logits /
// dlogits buffers; lora_grads_zero + transformer_backward_lora accumulate;
// cross_entropy_forward returns the loss (one host sync).  Differences
// (exact math): the LoRA input gradient, the SwiGLU backward and the final
// RMSNorm backward follow autograd, and the last dlogits row is written as
// zeros (the reference's Q1-Q4).
//
// Adapters allocated by lora_weights_init / lora_grads_alloc live in one
// arena per kind (A and B of every adapter in the native arena order), so the
// step moves them with single copies; adapter structs filled by the caller
// are gathered and scattered tensor by tensor instead.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ctx.h"

using namespace llmt;

// The reference's struct layouts (include/lora.h:13-62, src/train.cu:10-24).
static_assert(sizeof(LW) == 32 * sizeof(void*), "LW: 11 weights + 21 pad slots");
static_assert(sizeof(MW) == sizeof(void*) * (1 + 32 * LLMT_NUM_LAYERS + 2 + 3), "MW layout");
static_assert(sizeof(LoraAdapter) == 6 * sizeof(float*) + 2 * sizeof(int), "LoraAdapter layout");
static_assert(sizeof(LoraWeights) == 4 * LLMT_NUM_LAYERS * sizeof(LoraAdapter), "LoraWeights");
static_assert(sizeof(LoraGrads) == 4 * LLMT_NUM_LAYERS * 2 * sizeof(float*), "LoraGrads");
static_assert(sizeof(LoraActs) == 17 * LLMT_NUM_LAYERS * sizeof(float*), "LoraActs");

namespace {

[[noreturn]] void die(const char* what) {
  fprintf(stderr, "llmt: %s: %s\n", what, llmt_last_error());
  exit(EXIT_FAILURE);
}

void check_rc(int rc, const char* what) {
  if (rc != LLMT_OK) die(what);
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "llmt: %s: %s\n", what, hipGetErrorString(e));
    exit(EXIT_FAILURE);
  }
}

struct Compat {
  llmt_ctx* ctx = nullptr;
  int seq_len = 0;
  int wfmt = LLMT_WEIGHTS_F16;
  const MW* model = nullptr;
  const void* model_key = nullptr;  // first frozen weight pointer seen for `model`
  _Float16* conv = nullptr;         // fp32 -> fp16 staging for fp32-only weights
  int8_t* q8 = nullptr;             // int8 staging (fp32 weights quantised for an int8 context)
  float* s32 = nullptr;             // its fp32 scales
  _Float16* s16 = nullptr;          // fp16 scales of one layer's seven matrices
  AdamHp* hp_dev = nullptr;
  AdamHp* hp_host = nullptr;
};
Compat g;

Ctx* native() { return reinterpret_cast<Ctx*>(g.ctx); }

size_t adapter_numel(int p, int is_b) {
  const size_t q = LLMT_NUM_HEADS * LLMT_HEAD_DIM, kv = LLMT_NUM_KV_HEADS * LLMT_HEAD_DIM,
               h = LLMT_HIDDEN_SIZE, r = LLMT_LORA_RANK;
  const size_t d_out[4] = {q, kv, kv, h}, d_in[4] = {h, h, h, q};
  return is_b ? d_out[p] * r : r * d_in[p];
}

size_t layer_numel() {
  size_t n = 0;
  for (int p = 0; p < 4; ++p) n += adapter_numel(p, 0) + adapter_numel(p, 1);
  return n;
}

size_t arena_offset(int l, int p, int is_b) {
  size_t off = (size_t)l * layer_numel();
  for (int q = 0; q < p; ++q) off += adapter_numel(q, 0) + adapter_numel(q, 1);
  return off + (is_b ? adapter_numel(p, 0) : 0);
}

LoraAdapter* adapter(LoraWeights* w, int l, int p) {
  return p == 0 ? &w->wq[l] : p == 1 ? &w->wk[l] : p == 2 ? &w->wv[l] : &w->wo[l];
}
const LoraAdapter* adapter(const LoraWeights* w, int l, int p) {
  return adapter(const_cast<LoraWeights*>(w), l, p);
}
LoraGrad* grad(LoraGrads* gr, int l, int p) {
  return p == 0 ? &gr->wq[l] : p == 1 ? &gr->wk[l] : p == 2 ? &gr->wv[l] : &gr->wo[l];
}
const LoraGrad* grad(const LoraGrads* gr, int l, int p) {
  return grad(const_cast<LoraGrads*>(gr), l, p);
}

// The arena base if every A/B pointer (kind 0 params, 1 m, 2 v) sits at its
// native arena offset, else NULL.
float* arena_of(const LoraWeights* w, int kind) {
  auto ptr = [&](const LoraAdapter* a, int is_b) -> float* {
    if (kind == 0) return is_b ? a->B : a->A;
    if (kind == 1) return is_b ? a->mB : a->mA;
    return is_b ? a->vB : a->vA;
  };
  float* base = ptr(&w->wq[0], 0);
  if (!base) return nullptr;
  for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
    for (int p = 0; p < 4; ++p)
      for (int b = 0; b < 2; ++b)
        if (ptr(adapter(w, l, p), b) != base + arena_offset(l, p, b)) return nullptr;
  return base;
}

float* grad_arena_of(const LoraGrads* gr) {
  float* base = gr->wq[0].dA;
  if (!base) return nullptr;
  for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
    for (int p = 0; p < 4; ++p) {
      const LoraGrad* gg = grad(gr, l, p);
      if (gg->dA != base + arena_offset(l, p, 0) || gg->dB != base + arena_offset(l, p, 1))
        return nullptr;
    }
  return base;
}

__global__ void scale_add_kernel(float* dst, const float* src, float s, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    dst[i] += s * src[i];
}

__global__ void zero_kernel(float* dst, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    dst[i] = 0.f;
}

unsigned grid_for(long long n) {
  const long long b = (n + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 16384 ? 16384 : b));
}

void scale_add(float* dst, const float* src, float s, long long n, hipStream_t st) {
  hipLaunchKernelGGL(scale_add_kernel, dim3(grid_for(n)), dim3(256), 0, st, dst, src, s, n);
  check_hip(hipGetLastError(), "scale_add");
}

// y[row, :] += scale * (x[row, :] A^T) B^T, h_buf[row, :] = x A^T
// (src/kernels/lora.cu:181-202); one workgroup per row.
__global__ __launch_bounds__(256) void lora_add_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ A,
                                                       const float* __restrict__ B, int d_in,
                                                       int d_out, float scale, float* y,
                                                       float* h_buf) {
  __shared__ float red[16][4];
  __shared__ float hs[16];
  const int t = blockIdx.x;
  const float* xr = x + (long long)t * d_in;
  for (int r = 0; r < 16; ++r) {
    float s = 0.f;
    for (int c = threadIdx.x; c < d_in; c += 256) s += xr[c] * A[(long long)r * d_in + c];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[r][threadIdx.x >> 6] = s;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const float h = red[threadIdx.x][0] + red[threadIdx.x][1] + red[threadIdx.x][2] +
                    red[threadIdx.x][3];
    hs[threadIdx.x] = h;
    if (h_buf) h_buf[(long long)t * 16 + threadIdx.x] = h;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < d_out; j += 256) {
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += hs[r] * B[(long long)j * 16 + r];
    y[(long long)t * d_out + j] += scale * s;
  }
}

// int8 row q [rows, cols] times its fp32 row scale, as fp16 (an int8-only
// lm_head, src/main.cu:64, as the fp16 operand of the logits GEMM).
__global__ void dequant_rows_kernel(const int8_t* __restrict__ q, const float* __restrict__ s,
                                    long long cols, long long n, _Float16* __restrict__ out) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    out[i] = (_Float16)((float)q[i] * s[i / cols]);
}

// Frozen-weight format of `m`: layer 0's fp16 pads decide fp16; without
// them, int8 pads (src/main.cu:49-55) make an int8 context; else fp16 from
// the fp32 fields.
int weight_format(const MW* m) {
  const LW& w = m->layers[0];
  return !w._pad[0] && w._pad[7] && w._pad[8] ? LLMT_WEIGHTS_I8 : LLMT_WEIGHTS_F16;
}

// Create (or re-create for a new seq_len or weight format) the compat context.
void ensure_ctx(int seq_len, int wfmt) {
  if (g.ctx && g.seq_len == seq_len && g.wfmt == wfmt) return;
  if (g.ctx) {
    llmt_ctx_destroy(g.ctx);
    g.ctx = nullptr;
    g.model = nullptr;
  }
  llmt_dims d;
  llmt_dims_qwen3_1_7b(&d);
  check_rc(llmt_ctx_create(&d, 1, seq_len, wfmt, nullptr, &g.ctx), "context");
  g.seq_len = seq_len;
  g.wfmt = wfmt;
}

// Upload the frozen weights of `m` (once per model), by the src/main.cu:40-55
// slot map: in an fp16 context the fp16 pads _pad[0..6] when given, else the
// fp32 fields converted on the device; in an int8 context the (int8, fp32
// scale) pairs _pad[7..20], the scales rounded to fp16 (the int8 GEMMs'
// scale type), else the fp32 fields quantised on the device
// (src/kernels/quantize.cu:8-44).
void ensure_weights(const MW* m) {
  const LW& w0 = m->layers[0];
  const void* key = w0._pad[0] ? w0._pad[0] : w0._pad[7] ? w0._pad[7] : (const void*)w0.wq;
  if (g.model == m && g.model_key == key) return;
  Ctx* c = native();
  const size_t big = (size_t)c->V * c->H;
  const size_t H = c->H, Q = c->Q, KV = c->KV, I = c->I;
  if (!g.conv) check_hip(hipMalloc((void**)&g.conv, big * 2), "staging");
  auto f16 = [&](const float* f32, void* pad, size_t n, size_t off) -> const void* {
    if (pad) return pad;
    if (!f32) {
      fprintf(stderr, "llmt: a frozen weight is NULL in both its fp32 and fp16 slots\n");
      exit(EXIT_FAILURE);
    }
    check_hip(f32_to_f16(f32, g.conv + off, n, c->st), "fp32->fp16");
    return g.conv + off;
  };
  const size_t rows[7] = {Q, KV, KV, H, I, I, H}, cols[7] = {H, H, H, Q, H, H, I};
  if (g.wfmt == LLMT_WEIGHTS_I8) {
    const size_t layer_elems = H * (2 * Q + 2 * KV + 3 * I), nsc = 2 * I + Q + 2 * KV + 2 * H;
    if (!g.q8) {
      check_hip(hipMalloc((void**)&g.q8, layer_elems), "staging");
      check_hip(hipMalloc((void**)&g.s32, nsc * 4), "staging");
      check_hip(hipMalloc((void**)&g.s16, nsc * 2), "staging");
    }
    for (int l = 0; l < c->L; ++l) {
      const LW& w = m->layers[l];
      const float* f32[7] = {w.wq, w.wk, w.wv, w.wo, w.w_gate, w.w_up, w.w_down};
      const int8_t* qp[7];
      const void* sp[7];
      size_t o = 0, so = 0;
      for (int k = 0; k < 7; ++k) {
        const int8_t* q = (const int8_t*)w._pad[7 + 2 * k];
        const float* sc = (const float*)w._pad[8 + 2 * k];
        if (!q || !sc) {  // quantise the fp32 field
          if (!f32[k]) {
            fprintf(stderr, "llmt: layer %d weight %d is NULL in its fp32 and int8 slots\n", l, k);
            exit(EXIT_FAILURE);
          }
          check_hip(quantize_rows_i8(f32[k], (int)rows[k], (int)cols[k], g.q8 + o, g.s32 + so,
                                     c->st),
                    "quantize");
          q = g.q8 + o;
          sc = g.s32 + so;
        }
        check_hip(f32_scale_to_f16(sc, g.s16 + so, (int)rows[k], c->st), "scale");
        qp[k] = q;
        sp[k] = g.s16 + so;
        o += rows[k] * cols[k];
        so += rows[k];
      }
      check_rc(llmt_set_layer_i8(g.ctx, l, qp, sp, w.attn_norm, w.ffn_norm, w.q_norm, w.k_norm),
               "set layer");
    }
  } else {
    for (int l = 0; l < c->L; ++l) {
      const LW& w = m->layers[l];
      const float* f32[7] = {w.wq, w.wk, w.wv, w.wo, w.w_gate, w.w_up, w.w_down};
      const void* wp[7];
      size_t o = 0;
      for (int k = 0; k < 7; ++k) {
        wp[k] = f16(f32[k], w._pad[k], rows[k] * cols[k], o);
        o += rows[k] * cols[k];
      }
      check_rc(llmt_set_layer_f16(g.ctx, l, wp[0], wp[1], wp[2], wp[3], wp[4], wp[5], wp[6],
                                  w.attn_norm, w.ffn_norm, w.q_norm, w.k_norm),
               "set layer");
    }
  }
  // The token gather reads embed_table (src/kernels/embed.cu:6-20) and the
  // logits read lm_head (src/kernels/lora_forward.cu:304), each loaded from
  // its own file by the reference (src/train.cu:56-88).  The head comes from
  // the fp16 pad (src/main.cu:63), else the fp32 field, else the int8 pair
  // (src/main.cu:64, values _pad[1], fp32 row scales _pad[2]) as fp16
  // q * scale; it stands for the embedding too when embed_table is NULL
  // (tied).  Distinct sources make an untied head.
  const bool head_i8 = !m->_pad[0] && !m->lm_head && m->_pad[1] && m->_pad[2];
  const void* head_src = m->_pad[0] ? m->_pad[0]
                         : m->lm_head ? (const void*)m->lm_head
                         : head_i8    ? m->_pad[1]
                                      : nullptr;
  const void* emb_src = m->embed_table ? (const void*)m->embed_table : head_src;
  if (!emb_src) {
    fprintf(stderr, "llmt: neither an embedding nor an lm_head is given\n");
    exit(EXIT_FAILURE);
  }
  // The head as an fp16 buffer in the staging area (which it then occupies).
  auto head16 = [&]() -> const void* {
    if (m->_pad[0]) return m->_pad[0];
    if (m->lm_head) return f16(m->lm_head, nullptr, big, 0);
    hipLaunchKernelGGL(dequant_rows_kernel, dim3(grid_for((long long)big)), dim3(256), 0, c->st,
                       (const int8_t*)m->_pad[1], (const float*)m->_pad[2], (long long)H,
                       (long long)big, g.conv);
    check_hip(hipGetLastError(), "lm_head dequant");
    return g.conv;
  };
  const void* e = m->embed_table ? f16(m->embed_table, nullptr, big, 0) : head16();
  // (synchronous: the staging area is free again afterwards.)  It also ties
  // the head to the embedding.
  check_rc(llmt_set_embed_f16(g.ctx, e, m->final_norm), "set embedding");
  if (head_src && head_src != emb_src) check_rc(llmt_set_lm_head_f16(g.ctx, head16()), "set lm_head");
  g.model = m;
  g.model_key = key;
}

// Parameters (kind 0) of `w` into the context's arena, then the fp16 shadows.
void gather_params(const LoraWeights* w) {
  Ctx* c = native();
  const size_t n = c->lora_numel;
  if (float* base = arena_of(w, 0)) {
    check_hip(hipMemcpyAsync(c->lora_p, base, n * 4, hipMemcpyDeviceToDevice, c->st), "gather");
  } else {
    for (int l = 0; l < c->L; ++l)
      for (int p = 0; p < 4; ++p)
        for (int b = 0; b < 2; ++b) {
          const LoraAdapter* a = adapter(w, l, p);
          check_hip(hipMemcpyAsync(c->lora_p + arena_offset(l, p, b), b ? a->B : a->A,
                                   adapter_numel(p, b) * 4, hipMemcpyDeviceToDevice, c->st),
                    "gather");
        }
  }
  check_hip(c->refresh_shadows(), "shadows");
}

}  // namespace

extern "C" {

// ------------------------------------------------------------------ adapters

void lora_weights_init(LoraWeights* lora) {
  const size_t n = layer_numel() * LLMT_NUM_LAYERS;
  float *p, *m, *v;
  check_hip(hipMalloc((void**)&p, n * 4), "lora_weights_init");
  check_hip(hipMalloc((void**)&m, n * 4), "lora_weights_init");
  check_hip(hipMalloc((void**)&v, n * 4), "lora_weights_init");
  check_hip(hipMemset(m, 0, n * 4), "lora_weights_init");
  check_hip(hipMemset(v, 0, n * 4), "lora_weights_init");
  for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
    for (int q = 0; q < 4; ++q) {
      LoraAdapter* a = adapter(lora, l, q);
      a->A = p + arena_offset(l, q, 0);
      a->B = p + arena_offset(l, q, 1);
      a->mA = m + arena_offset(l, q, 0);
      a->mB = m + arena_offset(l, q, 1);
      a->vA = v + arena_offset(l, q, 0);
      a->vB = v + arena_offset(l, q, 1);
      a->d_in = (int)(adapter_numel(q, 0) / LLMT_LORA_RANK);
      a->d_out = (int)(adapter_numel(q, 1) / LLMT_LORA_RANK);
    }
  // src/kernels/lora.cu:40-62: A ~ 0.02 N(0, 1), B = 0 (this library's own
  // seeded generator; the reference's cuRAND stream is not reproduced).
  AdamShadow sh{};
  sh.per_layer = (long long)layer_numel();
  for (int q = 0; q < 4; ++q)
    for (int b = 0; b < 2; ++b) sh.seg_off[2 * q + b] = (long long)arena_offset(0, q, b);
  check_hip(lora_init(p, m, v, (long long)n, 0x5eedull, 0.02f, 0.0f, sh, nullptr),
            "lora_weights_init");
  check_hip(hipDeviceSynchronize(), "lora_weights_init");
}

void lora_weights_free(LoraWeights* lora) {
  if (float* p = arena_of(lora, 0)) {
    hipFree(p);
    hipFree(arena_of(lora, 1));
    hipFree(arena_of(lora, 2));
  } else {
    for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
      for (int q = 0; q < 4; ++q) {
        LoraAdapter* a = adapter(lora, l, q);
        hipFree(a->A); hipFree(a->B); hipFree(a->mA); hipFree(a->vA); hipFree(a->mB); hipFree(a->vB);
      }
  }
  memset(lora, 0, sizeof(*lora));
}

void lora_grads_alloc(LoraGrads* grads, const LoraWeights* lora) {
  (void)lora;
  const size_t n = layer_numel() * LLMT_NUM_LAYERS;
  float* base;
  check_hip(hipMalloc((void**)&base, n * 4), "lora_grads_alloc");
  for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
    for (int q = 0; q < 4; ++q) {
      grad(grads, l, q)->dA = base + arena_offset(l, q, 0);
      grad(grads, l, q)->dB = base + arena_offset(l, q, 1);
    }
}

void lora_grads_free(LoraGrads* grads) {
  if (float* base = grad_arena_of(grads)) {
    hipFree(base);
  } else {
    for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
      for (int q = 0; q < 4; ++q) {
        hipFree(grad(grads, l, q)->dA);
        hipFree(grad(grads, l, q)->dB);
      }
  }
  memset(grads, 0, sizeof(*grads));
}

void lora_grads_zero(LoraGrads* grads) {
  if (float* base = grad_arena_of(grads)) {
    gpu_zero(base, (int)(layer_numel() * LLMT_NUM_LAYERS));
  } else {
    for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
      for (int q = 0; q < 4; ++q) {
        gpu_zero(grad(grads, l, q)->dA, (int)adapter_numel(q, 0));
        gpu_zero(grad(grads, l, q)->dB, (int)adapter_numel(q, 1));
      }
  }
}

// The stashes are library-private and live in the context: the struct's
// pointers are left NULL (the reference's callers never read them).
void lora_acts_alloc(LoraActs* acts, int seq_len) {
  (void)seq_len;
  memset(acts, 0, sizeof(*acts));
}

void lora_acts_free(LoraActs* acts, int seq_len) {
  (void)seq_len;
  memset(acts, 0, sizeof(*acts));
}

void lora_forward_add(const float* x, const LoraAdapter* a, float* y, float* h_buf, int seq) {
  hipLaunchKernelGGL(lora_add_kernel, dim3(seq), dim3(256), 0, nullptr, x, a->A, a->B, a->d_in,
                     a->d_out, LLMT_LORA_SCALE, y, h_buf);
  check_hip(hipGetLastError(), "lora_forward_add");
}

void scale_add_inplace(float* dst, const float* src, float scale, int n) {
  scale_add(dst, src, scale, n, nullptr);
}

void gpu_zero(float* buf, int n) {
  hipLaunchKernelGGL(zero_kernel, dim3(grid_for(n)), dim3(256), 0, nullptr, buf, (long long)n);
  check_hip(hipGetLastError(), "gpu_zero");
}

// src/kernels/lora.cu:235-246: bias corrections in fp32 with powf; one
// multi-tensor launch when the adapters live in lora_weights_init's arenas.
void adamw_step_lora(LoraWeights* lora, const LoraGrads* grads, float lr, float beta1,
                     float beta2, float eps, float wd, int step) {
  if (!g.hp_dev) {
    check_hip(hipMalloc((void**)&g.hp_dev, sizeof(AdamHp)), "adamw");
    check_hip(hipHostMalloc((void**)&g.hp_host, sizeof(AdamHp), hipHostMallocDefault), "adamw");
  }
  check_hip(hipDeviceSynchronize(), "adamw");  // the staging slot is free
  AdamHp h{lr, beta1, beta2, eps, wd, 1.0f - powf(beta1, (float)step),
           1.0f - powf(beta2, (float)step)};
  *g.hp_host = h;
  check_hip(hipMemcpy(g.hp_dev, g.hp_host, sizeof(AdamHp), hipMemcpyHostToDevice), "adamw");
  AdamShadow none{};
  float *p = arena_of(lora, 0), *m = arena_of(lora, 1), *v = arena_of(lora, 2);
  const float* gr = grad_arena_of(grads);
  if (p && m && v && gr) {
    check_hip(adamw(p, gr, m, v, (long long)(layer_numel() * LLMT_NUM_LAYERS), g.hp_dev, 1, none,
                    nullptr),
              "adamw");
    return;
  }
  for (int l = 0; l < LLMT_NUM_LAYERS; ++l)
    for (int q = 0; q < 4; ++q) {
      LoraAdapter* a = adapter(lora, l, q);
      const LoraGrad* gg = grad(grads, l, q);
      check_hip(adamw(a->A, gg->dA, a->mA, a->vA, (long long)adapter_numel(q, 0), g.hp_dev, 1,
                      none, nullptr),
                "adamw");
      check_hip(adamw(a->B, gg->dB, a->mB, a->vB, (long long)adapter_numel(q, 1), g.hp_dev, 1,
                      none, nullptr),
                "adamw");
    }
}

// ------------------------------------------------------------------ the step

void transformer_forward_lora(const int* token_ids, const MW* model, const LoraWeights* lora,
                              float* hidden, float* residual, float* norm_out, float* q, float* k,
                              float* v, float* k_exp, float* v_exp, float* attn_out,
                              float* gate_buf, float* up_buf, float* logits, LoraActs* acts,
                              int seq_len) {
  (void)hidden; (void)residual; (void)norm_out; (void)q; (void)k; (void)v; (void)k_exp;
  (void)v_exp; (void)attn_out; (void)gate_buf; (void)up_buf; (void)acts;
  if (seq_len < 2) {
    fprintf(stderr, "llmt: seq_len must be at least 2 (got %d)\n", seq_len);
    exit(EXIT_FAILURE);
  }
  ensure_ctx(seq_len, weight_format(model));
  ensure_weights(model);
  gather_params(lora);
  Ctx* c = native();
  check_hip(c->clear_pad_rows(1), "pad rows");
  if (c->rows(1) == seq_len) {
    check_hip(c->forward(token_ids, 1, logits), "forward");
  } else {  // the logits GEMM writes rows(1) rows: the caller's buffer holds seq_len
    check_hip(c->forward(token_ids, 1, c->logits), "forward");
    check_hip(hipMemcpyAsync(logits, c->logits, (size_t)seq_len * c->V * sizeof(float),
                             hipMemcpyDeviceToDevice, c->st),
              "logits");
  }
}

float cross_entropy_forward(const float* logits, const int* targets, float* dlogits,
                            int seq_len) {
  if (!g.ctx || g.seq_len != seq_len) {
    fprintf(stderr, "llmt: cross_entropy_forward before transformer_forward_lora\n");
    exit(EXIT_FAILURE);
  }
  Ctx* c = native();
  check_hip(c->ce(logits, targets, 1, dlogits), "cross_entropy");
  check_hip(hipMemcpyAsync(c->host_loss, c->loss_dev, 4, hipMemcpyDeviceToHost, c->st), "loss");
  check_hip(hipStreamSynchronize(c->st), "loss");
  return *c->host_loss;
}

void transformer_backward_lora(const float* d_logits, const MW* model, const LoraWeights* lora,
                               const LoraActs* acts, LoraGrads* grads, float* d_hidden,
                               float* d_hidden2, float* d_norm, float* d_q, float* d_k,
                               float* d_v, float* d_q_exp, float* d_k_exp, float* d_v_exp,
                               float* d_pre_o, float* d_gate, float* d_up, float* dh_tmp,
                               float* dx_lora, int seq_len) {
  (void)model; (void)lora; (void)acts; (void)d_hidden; (void)d_hidden2; (void)d_norm; (void)d_q;
  (void)d_k; (void)d_v; (void)d_q_exp; (void)d_k_exp; (void)d_v_exp; (void)d_pre_o; (void)d_gate;
  (void)d_up; (void)dh_tmp; (void)dx_lora;
  if (!g.ctx || g.seq_len != seq_len) {
    fprintf(stderr, "llmt: transformer_backward_lora before transformer_forward_lora\n");
    exit(EXIT_FAILURE);
  }
  Ctx* c = native();
  // The caller's dlogits (= (p - onehot) / (S - 1)) as the fp16 operand the
  // lm_head dX GEMM reads (scaled by (S - 1) * 2^14, undone in its epilogue).
  check_hip(f32_to_f16_scaled(d_logits, c->grad16, (size_t)seq_len * c->V,
                              (float)(seq_len - 1) * kGradLogitScale, c->st),
            "dlogits");
  check_hip(c->backward(1, 0), "backward");
  // accumulate into the caller's gradients (src/kernels/lora_backward.cu:50-90)
  if (float* base = grad_arena_of(grads)) {
    scale_add(base, c->lora_g, 1.0f, (long long)c->lora_numel, c->st);
  } else {
    for (int l = 0; l < c->L; ++l)
      for (int q = 0; q < 4; ++q) {
        LoraGrad* gg = grad(grads, l, q);
        scale_add(gg->dA, c->lora_g + arena_offset(l, q, 0), 1.0f, (long long)adapter_numel(q, 0),
                  c->st);
        scale_add(gg->dB, c->lora_g + arena_offset(l, q, 1), 1.0f, (long long)adapter_numel(q, 1),
                  c->st);
      }
  }
  check_hip(hipStreamSynchronize(c->st), "backward");
}

}  // extern "C"
