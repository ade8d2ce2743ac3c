// rows.hip — the per-token-row kernels of the step: embedding gather, and the
// epilogues that consume split-K GEMM partials and fuse everything that lives
// on one token row (LoRA up-projection, QK-RMSNorm + RoPE, residual adds,
// RMSNorm forward/backward, SwiGLU forward/backward, the attention-backward
// row statistics).  One workgroup of 256 threads (4 waves) per token row
// unless noted; rows are staged in LDS so each input is read from HBM once.
//
// The reference runs these as separate fp32 kernels on the default stream
// (src/kernels/rmsnorm.cu, rope.cu, activation.cu, elementwise.cu, embed.cu,
// plus src/kernels/lora.cu:181-202 for the LoRA add); here they are fused
// into the GEMM consumers so the [T, N] intermediates never make a second
// round trip through HBM.
//
// Gradient operands of the backward GEMMs are fp16 with a power-of-two scale
// per token row (row max in [2^13, 2^14)); the producer writes rinv = 1/scale
// next to the operand and the consuming epilogue multiplies the GEMM result
// row by it.  The scale is a power of two, so applying and removing it is
// exact in fp32.
#include "ops.h"

namespace llmt {

namespace {

constexpr int RT = 256;  // threads per row workgroup
constexpr int RW = RT / 64;
constexpr int HD = 128;  // head_dim
constexpr int R = 16;    // LoRA rank

// Split-K partial sums, in split order (deterministic), with RB8 splits'
// loads in flight per thread: row epilogues are latency-bound, so every
// load of a batch is issued before the first add.
constexpr int RB8 = 8;

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float4 sum_splits4(const float* p, int split, long long ss) {
  float4 v = ld4(p);
  for (int k = 1; k < split; k += 2 * RB8) {
    float4 x[2 * RB8];
#pragma unroll
    for (int i = 0; i < 2 * RB8; ++i) x[i] = ld4(p + (long long)min(k + i, split - 1) * ss);
#pragma unroll
    for (int i = 0; i < 2 * RB8; ++i)
      if (k + i < split) v = add4(v, x[i]);
  }
  return v;
}

__device__ __forceinline__ void sum_splits8(const float* p, int split, long long ss, float4& a,
                                            float4& b) {
  a = ld4(p);
  b = ld4(p + 4);
  for (int k = 1; k < split; k += RB8) {
    float4 x[RB8], y[RB8];
#pragma unroll
    for (int i = 0; i < RB8; ++i) {
      const float* q = p + (long long)min(k + i, split - 1) * ss;
      x[i] = ld4(q);
      y[i] = ld4(q + 4);
    }
#pragma unroll
    for (int i = 0; i < RB8; ++i)
      if (k + i < split) {
        a = add4(a, x[i]);
        b = add4(b, y[i]);
      }
  }
}

// Row t of a split-K GEMM output into LDS: ys[c] (c < n, n % 8 == 0) = the
// split sum plus the LoRA up-projection terms covering c; hs[j] (j < in.nh)
// = the raw h columns.  Thread -> 8-column pieces.  Ends with a barrier.
__device__ void fetch_row(const RowIn& in, int t, int n, float* ys, float* hs) {
  const float* prow = in.part + (long long)t * in.ldp;
  const int tid = threadIdx.x;
  if (tid < in.nh / 4) {
    const float4 h = sum_splits4(prow + in.hcol + 4 * tid, in.split, in.ss);
    hs[4 * tid] = h.x;
    hs[4 * tid + 1] = h.y;
    hs[4 * tid + 2] = h.z;
    hs[4 * tid + 3] = h.w;
  }
  for (int pc = tid; pc < n / 8; pc += RT) {
    float4 a, b;
    sum_splits8(prow + 8 * pc, in.split, in.ss, a, b);
    *reinterpret_cast<float4*>(ys + 8 * pc) = a;
    *reinterpret_cast<float4*>(ys + 8 * pc + 4) = b;
  }
  __syncthreads();
  if (in.nterm == 0) return;
  for (int pc = tid; pc < n / 8; pc += RT) {
    const int c = 8 * pc;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < in.nterm; ++q) {
      const LoraTerm& m = in.term[q];
      if (c < m.c0 || c >= m.c0 + m.n) continue;
      half8 wv[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        wv[r] = *reinterpret_cast<const half8*>(m.sh + packed_index(m.row0 + r, c, m.kp));
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float h = hs[m.hidx + r];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += h * (float)wv[r][e];
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ys[c + e] += in.lscale * acc[e];
  }
  __syncthreads();
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Two block sums at once (one barrier pair).
__device__ __forceinline__ float2 block_sum2(float a, float b, float* red) {
  a = wave_sum(a);
  b = wave_sum(b);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[w] = a;
    red[RW + w] = b;
  }
  __syncthreads();
  float x = 0.f, y = 0.f;
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    x += red[i];
    y += red[RW + i];
  }
  __syncthreads();
  return make_float2(x, y);
}

// ---------------------------------------------------------------- forward

// src/kernels/embed.cu:6-20 (int32 row gather, ids clamped into [0, V)) fused
// with the first layer's attention RMSNorm (src/kernels/rmsnorm.cu:6-29).
__global__ __launch_bounds__(RT) void embed_norm_kernel(const int* __restrict__ tok,
                                                        const _Float16* __restrict__ E, int V,
                                                        int H, const float* __restrict__ w,
                                                        float eps, float* __restrict__ x,
                                                        _Float16* __restrict__ xn) {
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  const int id = min(max(tok[t], 0), V - 1);
  // E is fragment-packed (K = H): the row's 8-element pieces are contiguous.
  float ss = 0.f;
  for (int c = threadIdx.x * 8; c < H; c += RT * 8) {
    const half8 v = *reinterpret_cast<const half8*>(E + packed_index(id, c, H));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float f = (float)v[i];
      x[(long long)t * H + c + i] = f;
      ss += f * f;
    }
  }
  const float r = rsqrtf(block_sum2(ss, 0.f, red).x / H + eps);
  for (int c = threadIdx.x; c < H; c += RT)
    xn[(long long)t * H + c] = (_Float16)(x[(long long)t * H + c] * r * w[c]);
}

// After the fused Q/K/V(+LoRA-A) GEMM, whose reduction already added
// s * (x A^T) B^T per projection (src/kernels/lora.cu:181-202): stash
// q_raw/k_raw (fp32, the QK-norm backward input) and h = x A^T, then per head
// QK-RMSNorm
// (src/kernels/rmsnorm.cu:36-41 with 128-wide rows) and half-split RoPE
// (src/kernels/rope.cu:7-27): lane l of a wave owns the rotation pair
// (l, l + 64).  Writes q, k (normed, rotated) and v as fp16 [T, Q + 2 KV].
__global__ __launch_bounds__(RT) void qkv_post_kernel(const QkvPostArgs a) {
  extern __shared__ float ys[];  // [NT]
  __shared__ float hs[64];
  const int t = blockIdx.x;
  const int Q = a.nq * HD, KV = a.nkv * HD, NT = Q + 2 * KV;
  fetch_row(a.in, t, NT, ys, hs);
  if (threadIdx.x < a.in.nh) a.hbuf[(long long)t * 64 + threadIdx.x] = hs[threadIdx.x];
  for (int c = threadIdx.x; c < NT; c += RT) {
    const float y = ys[c];
    if (c < Q + KV)
      a.qkraw[(long long)t * (Q + KV) + c] = y;
    else
      a.qkv16[(long long)t * NT + c] = (_Float16)y;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos = t % a.S;
  const float cs = a.cosT[pos * (HD / 2) + lane], sn = a.sinT[pos * (HD / 2) + lane];
  for (int hh = wave; hh < a.nq + a.nkv; hh += RW) {
    const int base = hh * HD;
    const float* w = hh < a.nq ? a.qn : a.kn;
    const float x0 = ys[base + lane], x1 = ys[base + 64 + lane];
    const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / HD + a.eps);
    const float y0 = x0 * r * w[lane], y1 = x1 * r * w[lane + 64];
    a.qkv16[(long long)t * NT + base + lane] = (_Float16)(y0 * cs - y1 * sn);
    a.qkv16[(long long)t * NT + base + 64 + lane] = (_Float16)(y1 * cs + y0 * sn);
  }
}

// After the O(+LoRA-A) GEMM (LoRA term added by its reduction):
// x_mid = x_in + oW^T + s (o A^T) B^T (residual, src/kernels/elementwise.cu:
// 4-15), stash h_o, then the FFN RMSNorm -> fp16.
__global__ __launch_bounds__(RT) void o_post_kernel(const RowIn in,
                                                    const float* __restrict__ x_in,
                                                    const float* __restrict__ w, float eps, int H,
                                                    float* __restrict__ hbuf,
                                                    float* __restrict__ x_mid,
                                                    _Float16* __restrict__ xn2) {
  extern __shared__ float ys[];  // [H]
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  fetch_row(in, t, H, ys, hs);
  if (threadIdx.x < in.nh) hbuf[(long long)t * 64 + 3 * R + threadIdx.x] = hs[threadIdx.x];
  float ssq = 0.f;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float xm = x_in[(long long)t * H + c] + ys[c];
    x_mid[(long long)t * H + c] = xm;
    ys[c] = xm;
    ssq += xm * xm;
  }
  const float r = rsqrtf(block_sum2(ssq, 0.f, red).x / H + eps);
  for (int c = threadIdx.x; c < H; c += RT)
    xn2[(long long)t * H + c] = (_Float16)(ys[c] * r * w[c]);
}

// After the fused gate/up GEMM: stash g, u (fp32) and a = silu(g) * u
// (src/kernels/activation.cu:5-18) as the fp16 operand of the down GEMM.
__global__ __launch_bounds__(RT) void gu_post_kernel(const RowIn in, int I, long long n4,
                                                     float* __restrict__ gu,
                                                     _Float16* __restrict__ a16) {
  for (long long i = (long long)blockIdx.x * RT + threadIdx.x; i < n4;
       i += (long long)gridDim.x * RT) {
    const long long t = i / (I / 4);
    const int c = (int)(i - t * (I / 4)) * 4;
    const float* p = in.part + t * in.ldp + c;
    const float4 g = sum_splits4(p, in.split, in.ss);
    const float4 u = sum_splits4(p + I, in.split, in.ss);
    *reinterpret_cast<float4*>(gu + t * 2 * I + c) = g;
    *reinterpret_cast<float4*>(gu + t * 2 * I + I + c) = u;
    half4 o;
    o[0] = (_Float16)(silu(g.x) * u.x);
    o[1] = (_Float16)(silu(g.y) * u.y);
    o[2] = (_Float16)(silu(g.z) * u.z);
    o[3] = (_Float16)(silu(g.w) * u.w);
    *reinterpret_cast<half4*>(a16 + t * I + c) = o;
  }
}

// After the down GEMM: x_out = x_mid + aW_down^T, then the next RMSNorm
// (the next layer's attention norm, or the final norm) -> fp16.
__global__ __launch_bounds__(RT) void resid_norm_kernel(const RowIn in,
                                                        const float* __restrict__ x_res,
                                                        const float* __restrict__ w, float eps,
                                                        int H, float* __restrict__ x_out,
                                                        _Float16* __restrict__ xn) {
  extern __shared__ float ys[];
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  fetch_row(in, t, H, ys, hs);
  float ssq = 0.f;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float v = x_res[(long long)t * H + c] + ys[c];
    x_out[(long long)t * H + c] = v;
    ys[c] = v;
    ssq += v * v;
  }
  const float r = rsqrtf(block_sum2(ssq, 0.f, red).x / H + eps);
  for (int c = threadIdx.x; c < H; c += RT) xn[(long long)t * H + c] = (_Float16)(ys[c] * r * w[c]);
}

// QK-RMSNorm + RoPE forward from fp16 raw q/k (the standalone attention
// block of config C3): raw [T, NT] fp16 -> qkv16 [T, NT] fp16, v copied.
__global__ __launch_bounds__(RT) void qk_norm_rope_kernel(const _Float16* __restrict__ raw,
                                                          const float* __restrict__ qn,
                                                          const float* __restrict__ kn,
                                                          const float* __restrict__ cosT,
                                                          const float* __restrict__ sinT, int S,
                                                          int nq, int nkv, float eps,
                                                          _Float16* __restrict__ out) {
  const int t = blockIdx.x;
  const int NT = (nq + 2 * nkv) * HD;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos = t % S;
  const float cs = cosT[pos * (HD / 2) + lane], sn = sinT[pos * (HD / 2) + lane];
  const _Float16* x = raw + (long long)t * NT;
  _Float16* o = out + (long long)t * NT;
  for (int hh = wave; hh < nq + 2 * nkv; hh += RW) {
    const int base = hh * HD;
    const float x0 = (float)x[base + lane], x1 = (float)x[base + 64 + lane];
    if (hh >= nq + nkv) {
      o[base + lane] = (_Float16)x0;
      o[base + 64 + lane] = (_Float16)x1;
      continue;
    }
    const float* w = hh < nq ? qn : kn;
    const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / HD + eps);
    const float y0 = x0 * r * w[lane], y1 = x1 * r * w[lane + 64];
    o[base + lane] = (_Float16)(y0 * cs - y1 * sn);
    o[base + 64 + lane] = (_Float16)(y1 * cs + y0 * sn);
  }
}

// ---------------------------------------------------------------- backward

// Generic "GEMM dX -> RMSNorm backward -> residual" row epilogue
// (src/kernels/rmsnorm.cu:53-95 plus the caller's residual adds,
// src/kernels/lora_backward.cu:297-300, 400-403).  d = GEMM row * rinv_in[t]
// * gscale; for nlora adapters the GEMM's reduction already added the LoRA
// input gradient s * (dh_p A_p) (src/kernels/lora_backward.cu:87 with the
// layout fixed), and dh_p, in the extra columns [H + 16p, H + 16p + 16), is
// stashed (unscaled) for the adapter gradients.
// dres_out = dres_in + rmsnorm_bwd(d, x, w); also written to dmid_out when
// given, and as the next fp16 gradient operand (g16, rinv_out).
__global__ __launch_bounds__(RT) void norm_bwd_kernel(const NormBwdArgs a) {
  extern __shared__ float ds[];  // [H]
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  const int H = a.H;
  fetch_row(a.in, t, H, ds, hs);
  const float rs = (a.rinv_in ? a.rinv_in[t] : 1.0f) * a.gscale;
  if (threadIdx.x < a.in.nh)
    a.dh_out[(long long)t * 64 + a.dh_col + threadIdx.x] = hs[threadIdx.x] * rs;
  const float* x = a.x + (long long)t * H;
  float dot = 0.f, ssx = 0.f;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float d = ds[c] * rs;
    ds[c] = d;
    const float xv = x[c];
    dot += d * a.w[c] * xv;
    ssx += xv * xv;
  }
  const float2 s2 = block_sum2(dot, ssx, red);
  const float r = rsqrtf(s2.y / H + a.eps);
  const float coef = r * r / H * s2.x;
  float amax = 0.f;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float dx = r * (ds[c] * a.w[c] - coef * x[c]);
    const float v = (a.dres_in ? a.dres_in[(long long)t * H + c] : 0.f) + dx;
    a.dres_out[(long long)t * H + c] = v;
    if (a.dmid_out) a.dmid_out[(long long)t * H + c] = v;
    ds[c] = v;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) a.rinv_out[t] = 1.0f / sc;
  for (int c = threadIdx.x; c < H; c += RT) a.g16[(long long)t * H + c] = (_Float16)(ds[c] * sc);
}

// dX of the down projection -> SwiGLU backward (src/kernels/activation.cu:
// 26-43 with d_up = dy * silu(g), i.e. without the reference's aliasing of
// d_gate and d_swiglu at src/kernels/lora_backward.cu:287) -> [dg | du] fp16.
__global__ __launch_bounds__(RT) void swiglu_bwd_kernel(const RowIn in,
                                                        const float* __restrict__ rinv_in,
                                                        const float* __restrict__ gu, int I,
                                                        _Float16* __restrict__ dgu16,
                                                        float* __restrict__ rinv_out) {
  extern __shared__ float ds[];  // [2 I]
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  fetch_row(in, t, I, ds, hs);
  const float rs = rinv_in[t];
  const float* gr = gu + (long long)t * 2 * I;
  float amax = 0.f;
  for (int c = threadIdx.x; c < I; c += RT) {
    const float da = ds[c] * rs;
    const float g = gr[c], u = gr[I + c];
    const float sg = 1.0f / (1.0f + __expf(-g));
    const float dg = da * u * (sg * (1.0f + g * (1.0f - sg)));
    const float du = da * (g * sg);
    ds[c] = dg;
    ds[I + c] = du;
    amax = fmaxf(amax, fmaxf(fabsf(dg), fabsf(du)));
  }
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) rinv_out[t] = 1.0f / sc;
  for (int c = threadIdx.x; c < 2 * I; c += RT)
    dgu16[(long long)t * 2 * I + c] = (_Float16)(ds[c] * sc);
}

// dX of the O projection (+ dh_o in the LoRA-B^T columns; the reduction
// already added s (dh_o A_o)): d_o = row * rinv; writes d_o fp32 (attention
// dO), dh_o, the row's max |d_o| and the flash-backward row statistic
// delta[b, h, s] = sum_d dO * O.
__global__ __launch_bounds__(RT) void o_dx_post_kernel(const RowIn in,
                                                       const float* __restrict__ rinv_in,
                                                       const _Float16* __restrict__ o16, int nq,
                                                       int S, float* __restrict__ dh_out,
                                                       float* __restrict__ dO,
                                                       float* __restrict__ delta,
                                                       float* __restrict__ damax) {
  extern __shared__ float ds[];  // [Q]
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  const int Q = nq * HD;
  fetch_row(in, t, Q, ds, hs);
  const float rs = rinv_in[t];
  if (threadIdx.x < in.nh) dh_out[(long long)t * 64 + 3 * R + threadIdx.x] = hs[threadIdx.x] * rs;
  float amax = 0.f;
  for (int c = threadIdx.x; c < Q; c += RT) {
    const float d = ds[c] * rs;
    dO[(long long)t * Q + c] = d;
    ds[c] = d;
    amax = fmaxf(amax, fabsf(d));
  }
  amax = block_max<RW>(amax, red);  // (also orders the ds[] writes)
  if (threadIdx.x == 0) damax[t] = amax;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = t / S, s = t - b * S;
  const _Float16* o = o16 + (long long)t * Q;
  for (int h = wave; h < nq; h += RW) {
    const int base = h * HD;
    const float v = wave_sum(ds[base + lane] * (float)o[base + lane] +
                             ds[base + 64 + lane] * (float)o[base + 64 + lane]);
    if (lane == 0) delta[((long long)b * nq + h) * S + s] = v;
  }
}

// Attention gradients (w.r.t. the normed, rotated q/k and v) -> RoPE
// backward (inverse rotation, src/kernels/rope.cu:57-89) -> QK-RMSNorm
// backward with x = q_raw/k_raw (src/kernels/rmsnorm.cu:53-95) ->
// dy = [dq_raw | dk_raw | dv] fp32 (the LoRA dB operand) and fp16 (scaled).
__global__ __launch_bounds__(RT) void qk_bwd_kernel(const QkBwdArgs a) {
  extern __shared__ float ds[];  // [NT]
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  const int Q = a.nq * HD, KV = a.nkv * HD, NT = Q + 2 * KV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos = t % a.S;
  const float cs = a.cosT[pos * (HD / 2) + lane], sn = a.sinT[pos * (HD / 2) + lane];
  const float* g = a.dqkv + (long long)t * a.ld_dqkv;
  for (int hh = wave; hh < a.nq + a.nkv; hh += RW) {
    const int base = hh * HD;
    const float d0 = g[base + lane], d1 = g[base + 64 + lane];
    const float n0 = d0 * cs + d1 * sn, n1 = d1 * cs - d0 * sn;
    const float* w = hh < a.nq ? a.qn : a.kn;
    const float w0 = w[lane], w1 = w[lane + 64];
    const float* xr = a.qkraw + (long long)t * (Q + KV) + base;
    const float x0 = xr[lane], x1 = xr[lane + 64];
    const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / HD + a.eps);
    const float dot = wave_sum(n0 * w0 * x0 + n1 * w1 * x1);
    const float coef = r * r / HD * dot;
    ds[base + lane] = r * (n0 * w0 - coef * x0);
    ds[base + 64 + lane] = r * (n1 * w1 - coef * x1);
  }
  for (int c = Q + KV + threadIdx.x; c < NT; c += RT) ds[c] = g[c];
  __syncthreads();
  float amax = 0.f;
  for (int c = threadIdx.x; c < NT; c += RT) {
    const float v = ds[c];
    a.dy32[(long long)t * NT + c] = v;
    amax = fmaxf(amax, fabsf(v));
  }
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) a.rinv_out[t] = 1.0f / sc;
  for (int c = threadIdx.x; c < NT; c += RT) a.g16[(long long)t * NT + c] = (_Float16)(ds[c] * sc);
}

// x_out = x; xn = fp16(rmsnorm(x) * w).
__global__ __launch_bounds__(RT) void copy_norm_kernel(const float* __restrict__ x,
                                                       const float* __restrict__ w, float eps,
                                                       int H, float* x_out,
                                                       _Float16* __restrict__ xn) {
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  float ss = 0.f;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float v = x[(long long)t * H + c];
    ss += v * v;
  }
  const float r = rsqrtf(block_sum2(ss, 0.f, red).x / H + eps);
  for (int c = threadIdx.x; c < H; c += RT) {
    const float v = x[(long long)t * H + c];
    x_out[(long long)t * H + c] = v;
    xn[(long long)t * H + c] = (_Float16)(v * r * w[c]);
  }
}

// dres = dy; g16 = fp16(dy * sc); rinv = 1 / sc (sc: the row's power-of-two scale).
__global__ __launch_bounds__(RT) void grad_rows_kernel(const float* dy, int H, float* dres,
                                                       _Float16* __restrict__ g16,
                                                       float* __restrict__ rinv) {
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  float amax = 0.f;
  for (int c = threadIdx.x; c < H; c += RT) amax = fmaxf(amax, fabsf(dy[(long long)t * H + c]));
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) rinv[t] = 1.0f / sc;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float v = dy[(long long)t * H + c];
    dres[(long long)t * H + c] = v;
    g16[(long long)t * H + c] = (_Float16)(v * sc);
  }
}

__global__ void f16_to_f32_rows_kernel(const _Float16* __restrict__ s, long long lds, int rows,
                                       int cols, float* __restrict__ d, long long ldd) {
  const long long n = (long long)rows * cols;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / cols, c = i - r * cols;
    d[r * ldd + c] = (float)s[r * lds + c];
  }
}

__global__ void f32_to_f16_scaled_kernel(const float* __restrict__ s, _Float16* __restrict__ d,
                                         size_t n, float scale) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    d[i] = (_Float16)(s[i] * scale);
}

inline unsigned grid_elems(long long n) {
  long long g = (n + RT - 1) / RT;
  return (unsigned)(g > 65536 ? 65536 : (g < 1 ? 1 : g));
}

}  // namespace

static bool row_in_ok(const RowIn& in, int n, const char* who) {
  bool ok = in.nh % 4 == 0 && in.nh >= 0 && in.nh <= 64 && in.nterm >= 0 && in.nterm <= 3 &&
            n % 8 == 0 && in.ldp % 4 == 0 && in.split >= 1 && (in.split == 1 || in.ss % 4 == 0) &&
            in.hcol % 4 == 0;
  for (int q = 0; q < in.nterm && ok; ++q)
    ok = in.term[q].c0 % 8 == 0 && in.term[q].n % 8 == 0 && in.term[q].hidx + R <= in.nh;
  if (!ok) set_error("%s: unsupported row-input layout (n=%d nh=%d nterm=%d)", who, n, in.nh, in.nterm);
  return ok;
}

hipError_t copy_norm(const float* x, const float* w, float eps, int H, int T, float* x_out,
                     _Float16* xn, hipStream_t st) {
  hipLaunchKernelGGL(copy_norm_kernel, dim3(T), dim3(RT), 0, st, x, w, eps, H, x_out, xn);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t grad_rows(const float* dy, int H, int T, float* dres, _Float16* g16, float* rinv,
                     hipStream_t st) {
  hipLaunchKernelGGL(grad_rows_kernel, dim3(T), dim3(RT), 0, st, dy, H, dres, g16, rinv);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t f16_to_f32_rows(const _Float16* src, long long lds, int rows, int cols, float* dst,
                           long long ldd, hipStream_t st) {
  hipLaunchKernelGGL(f16_to_f32_rows_kernel, dim3(grid_elems((long long)rows * cols)), dim3(RT), 0,
                     st, src, lds, rows, cols, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t f32_to_f16_scaled(const float* src, _Float16* dst, size_t n, float scale,
                             hipStream_t st) {
  hipLaunchKernelGGL(f32_to_f16_scaled_kernel, dim3(grid_elems((long long)n)), dim3(RT), 0, st, src,
                     dst, n, scale);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t embed_norm(const int* tok, const _Float16* E, int V, int H, const float* w, float eps,
                      int T, float* x, _Float16* xn, hipStream_t st) {
  hipLaunchKernelGGL(embed_norm_kernel, dim3(T), dim3(RT), 0, st, tok, E, V, H, w, eps, x, xn);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t qkv_post(const QkvPostArgs& a, int T, hipStream_t st) {
  const int NT = (a.nq + 2 * a.nkv) * HD;
  if (!row_in_ok(a.in, NT, "qkv_post")) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qkv_post_kernel, dim3(T), dim3(RT), NT * sizeof(float), st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}


hipError_t o_post(const RowIn& in, const float* x_in, const float* w, float eps, int H, int T,
                  float* hbuf, float* x_mid, _Float16* xn2, hipStream_t st) {
  if (!row_in_ok(in, H, "o_post")) return hipErrorInvalidValue;
  hipLaunchKernelGGL(o_post_kernel, dim3(T), dim3(RT), H * sizeof(float), st, in, x_in, w, eps, H,
                     hbuf, x_mid, xn2);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t gu_post(const RowIn& in, int I, int T, float* gu, _Float16* a16, hipStream_t st) {
  if (!row_in_ok(in, I, "gu_post") || in.nterm) return hipErrorInvalidValue;
  const long long n4 = (long long)T * (I / 4);
  hipLaunchKernelGGL(gu_post_kernel, dim3(grid_elems(n4)), dim3(RT), 0, st, in, I, n4, gu, a16);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t resid_norm(const RowIn& in, const float* x_res, const float* w, float eps, int H, int T,
                      float* x_out, _Float16* xn, hipStream_t st) {
  if (!row_in_ok(in, H, "resid_norm")) return hipErrorInvalidValue;
  hipLaunchKernelGGL(resid_norm_kernel, dim3(T), dim3(RT), H * sizeof(float), st, in, x_res, w, eps,
                     H, x_out, xn);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t qk_norm_rope(const _Float16* raw, const float* qn, const float* kn, const float* cosT,
                        const float* sinT, int S, int nq, int nkv, float eps, int T, _Float16* out,
                        hipStream_t st) {
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(T), dim3(RT), 0, st, raw, qn, kn, cosT, sinT, S, nq,
                     nkv, eps, out);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t norm_bwd(const NormBwdArgs& a, int T, hipStream_t st) {
  if (!row_in_ok(a.in, a.H, "norm_bwd")) return hipErrorInvalidValue;
  hipLaunchKernelGGL(norm_bwd_kernel, dim3(T), dim3(RT), a.H * sizeof(float), st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t swiglu_bwd(const RowIn& in, const float* rinv_in, const float* gu, int I, int T,
                      _Float16* dgu16, float* rinv_out, hipStream_t st) {
  if (!row_in_ok(in, I, "swiglu_bwd")) return hipErrorInvalidValue;
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(T), dim3(RT), 2 * I * sizeof(float), st, in, rinv_in,
                     gu, I, dgu16, rinv_out);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t o_dx_post(const RowIn& in, const float* rinv_in, const _Float16* o16, int nq, int S,
                     int T, float* dh_out, float* dO, float* delta, float* damax, hipStream_t st) {
  if (!row_in_ok(in, nq * HD, "o_dx_post")) return hipErrorInvalidValue;
  hipLaunchKernelGGL(o_dx_post_kernel, dim3(T), dim3(RT), nq * HD * sizeof(float), st, in, rinv_in,
                     o16, nq, S, dh_out, dO, delta, damax);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t qk_bwd(const QkBwdArgs& a, int T, hipStream_t st) {
  const int NT = (a.nq + 2 * a.nkv) * HD;
  hipLaunchKernelGGL(qk_bwd_kernel, dim3(T), dim3(RT), NT * sizeof(float), st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
