// rows.hip — the per-token-row kernels of the step: embedding gather, and the
// epilogues that consume split-K GEMM partials and fuse everything that lives
// on one token row (LoRA up-projection, QK-RMSNorm + RoPE, residual adds,
// RMSNorm forward/backward, SwiGLU forward/backward, the attention-backward
// row statistics).  One workgroup of 512 threads (8 waves) per token row
// unless noted.  At the headline shape these kernels are latency-bound (128
// rows, a few hundred KB each), so a thread owns 4-column pieces of the row
// in registers and issues every independent load (split-K partials, h
// columns, side inputs) before the first use: one memory round trip, then
// LDS-only block reductions.
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
#include <algorithm>
#include <stdlib.h>

#include <type_traits>

#include "ops.h"

namespace llmt {

namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int RT = 512;  // threads per row workgroup
constexpr int RW = RT / 64;
constexpr int HD = 128;  // head_dim
constexpr int R = 16;    // LoRA rank

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
// A load of data read once (a stash of the forward, a residual stream):
// nontemporal when NT, so it does not displace cached operands.
template <bool NT>
__device__ __forceinline__ float4 ld4s(const float* p) {
  if constexpr (NT) {
    const floatx4 v = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
  } else {
    return ld4(p);
  }
}
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
__device__ __forceinline__ float4 mul4(float4 a, float s) {
  return make_float4(a.x * s, a.y * s, a.z * s, a.w * s);
}
__device__ __forceinline__ float4 mul4v(float4 a, float4 b) {
  return make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
}
__device__ __forceinline__ void st_h4(_Float16* p, float4 v) {
  half4 h;
  h[0] = (_Float16)v.x;
  h[1] = (_Float16)v.y;
  h[2] = (_Float16)v.z;
  h[3] = (_Float16)v.w;
  *reinterpret_cast<half4*>(p) = h;
}
__device__ __forceinline__ float amax4(float4 v) {
  return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Split-K partial sums in split order (deterministic), every load of a
// batch issued before the first add.
__device__ __forceinline__ float4 sum_splits4(const float* p, int split, long long ss) {
  constexpr int SB = 16;
  float4 v = ld4(p);
  for (int k = 1; k < split; k += SB) {
    float4 x[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) x[i] = ld4(p + (long long)min(k + i, split - 1) * ss);
#pragma unroll
    for (int i = 0; i < SB; ++i) v = k + i < split ? add4(v, x[i]) : v;
  }
  return v;
}

// This thread's pieces of row t of a split-K GEMM output: piece p is columns
// 4 (tid + p RT) .. + 3 (live when < n; dead pieces hold column 0's values),
// plus (HH) this thread's four raw h columns when tid < nh / 4 (others hold
// group 0's).  One loop for both, with up to 24 loads in flight per batch
// and branch-free in-order adds, so a row costs one memory round trip per
// batch of splits.
// SC: the input may carry RowIn::split_col (only kernels instantiated with
// it accept such inputs; row_in_ok).
template <int P, bool HH, int LOADS = 24, bool SC = false>
__device__ __forceinline__ void load_row(const RowIn& in, int t, int n, float4 (&v)[P], float4& h) {
  const float* prow = in.part + (long long)t * in.ldp;
  int off[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    off[p] = c < n ? c : 0;
    v[p] = ld4(prow + off[p]);
  }
  const int hoff = in.hcol + 4 * ((int)threadIdx.x < in.nh / 4 ? (int)threadIdx.x : 0);
  if (HH) h = ld4(prow + hoff);
  if constexpr (SC) {
    // two partials, the second one only for columns at or past split_col
    // (GemmArgs::split_col; a piece's 64 lanes cover 256 columns and
    // split_col is a multiple of 256, so the condition is uniform over a
    // wave).  Kept apart from the general loop below, whose register use it
    // would otherwise raise.
    const float* q = prow + in.ss;
#pragma unroll
    for (int p = 0; p < P; ++p)
      if (off[p] >= in.split_col) v[p] = add4(v[p], ld4(q + off[p]));
    if (HH) h = add4(h, ld4(q + hoff));
    return;
  }
  constexpr int SB = LOADS / (P + (HH ? 1 : 0));
  for (int k = 1; k < in.split; k += SB) {
    float4 x[SB][P], y[SB];
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const float* q = prow + (long long)min(k + i, in.split - 1) * in.ss;
#pragma unroll
      for (int p = 0; p < P; ++p) x[i][p] = ld4(q + off[p]);
      if (HH) y[i] = ld4(q + hoff);
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const bool ok = k + i < in.split;
#pragma unroll
      for (int p = 0; p < P; ++p) v[p] = ok ? add4(v[p], x[i][p]) : v[p];
      if (HH) h = ok ? add4(h, y[i]) : h;
    }
  }
}

// load_row with h, then mid() (more loads independent of the row), as one
// memory round trip: for 2, 4 or 8 splits straight-line code issues every
// split's loads, then mid(), then sums in split order (load_row's split
// loop would wait for the loads issued before it); other counts take
// load_row, then mid().  C2 (B1 x S128): the attention norm backward with
// its adapter terms 8.5 -> 7.5 us, the FFN norm backward 5.1 -> 4.4 us.
template <int P, int NS, bool HH, typename F>
__device__ __forceinline__ void load_row_ns(const RowIn& in, int t, int n, float4 (&v)[P],
                                            float4& h, F&& mid) {
  const float* prow = in.part + (long long)t * in.ldp;
  int off[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    off[p] = c < n ? c : 0;
  }
  const int hoff = in.hcol + 4 * ((int)threadIdx.x < in.nh / 4 ? (int)threadIdx.x : 0);
  float4 x[NS][P], y[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const float* q = prow + (long long)i * in.ss;
#pragma unroll
    for (int p = 0; p < P; ++p) x[i][p] = ld4(q + off[p]);
    if (HH) y[i] = ld4(q + hoff);
  }
  mid();
#pragma unroll
  for (int p = 0; p < P; ++p) v[p] = x[0][p];
  if (HH) h = y[0];
#pragma unroll
  for (int i = 1; i < NS; ++i) {
#pragma unroll
    for (int p = 0; p < P; ++p) v[p] = add4(v[p], x[i][p]);
    if (HH) h = add4(h, y[i]);
  }
}
template <int P, bool HH = true, typename F>
__device__ __forceinline__ void load_row_then(const RowIn& in, int t, int n, float4 (&v)[P],
                                              float4& h, F&& mid) {
  switch (in.split) {
    case 2: load_row_ns<P, 2, HH>(in, t, n, v, h, mid); break;
    case 4: load_row_ns<P, 4, HH>(in, t, n, v, h, mid); break;
    case 8: load_row_ns<P, 8, HH>(in, t, n, v, h, mid); break;
    default:
      load_row<P, HH>(in, t, n, v, h);
      mid();
  }
}

template <int P, bool SC = false>
__device__ __forceinline__ void load_partials(const RowIn& in, int t, int n, float4 (&v)[P]) {
  float4 h;
  if constexpr (SC) {
    load_row<P, false, 24, SC>(in, t, n, v, h);
  } else {
    auto none = []() {};
    load_row_then<P, false>(in, t, n, v, h, none);
  }
}

__device__ __forceinline__ void store_h(const RowIn& in, float4 h, float* hs) {
  if ((int)threadIdx.x < in.nh / 4) *reinterpret_cast<float4*>(hs + 4 * threadIdx.x) = h;
}

// LoRA up-projection of this thread's pieces, split into a load phase (no
// dependence on h, issued with the partials) and an apply phase:
//   v[p] += lscale * sum over the terms covering the piece (at most NTM, in
//   term order) of sum_r hs[hidx + r] * shadow(row0 + r, c .. c + 3).
template <int P, int NTM>
struct LoraRegs {
  half4 w[P][NTM][R];
  int hidx[P][NTM];  // -1: unused slot
};

// NTM == 1: the piece is covered by at most one term (the forward q/k/v
// column ranges); NTM == 3: term q goes to slot q.
template <int P, int NTM>
__device__ __forceinline__ void lora_load(const RowIn& in, int n, LoraRegs<P, NTM>& L) {
  static_assert(NTM == 1 || NTM == 3, "one covering term, or one slot per term");
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
#pragma unroll
    for (int s = 0; s < NTM; ++s) L.hidx[p][s] = -1;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int s = NTM == 1 ? 0 : q;
      const bool use = q < in.nterm && c < n && c >= in.term[q].c0 && c < in.term[q].c0 + in.term[q].n;
      if (use) {
        const LoraTerm& m = in.term[q];
        L.hidx[p][s] = m.hidx;
#pragma unroll
        for (int r = 0; r < R; ++r)
          L.w[p][s][r] = *reinterpret_cast<const half4*>(m.shr + (long long)(m.row0 + r) * m.kp + c);
      }
    }
  }
}

template <int P, int NTM>
__device__ __forceinline__ void lora_apply(const RowIn& in, const float* hs,
                                           const LoraRegs<P, NTM>& L, float4 (&v)[P]) {
#pragma unroll
  for (int p = 0; p < P; ++p) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < NTM; ++s) {
      if (L.hidx[p][s] < 0) continue;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float h = hs[L.hidx[p][s] + r];
        acc.x += h * (float)L.w[p][s][r][0];
        acc.y += h * (float)L.w[p][s][r][1];
        acc.z += h * (float)L.w[p][s][r][2];
        acc.w += h * (float)L.w[p][s][r][3];
      }
    }
    v[p] = add4(v[p], mul4(acc, in.lscale));
  }
}

// lora_apply for NR rows of one piece per thread (hs[i]: row i's h values),
// each adapter value converted once and used for every row, in the one-row
// form's order of adds.
template <int NR, int NTM>
__device__ __forceinline__ void lora_apply_rows(const RowIn& in, const float (*hs)[64],
                                                const LoraRegs<1, NTM>& L, float4 (&v)[NR]) {
  float4 acc[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int s = 0; s < NTM; ++s) {
    if (L.hidx[0][s] < 0) continue;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float w0 = (float)L.w[0][s][r][0], w1 = (float)L.w[0][s][r][1];
      const float w2 = (float)L.w[0][s][r][2], w3 = (float)L.w[0][s][r][3];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        const float h = hs[i][L.hidx[0][s] + r];
        acc[i].x += h * w0;
        acc[i].y += h * w1;
        acc[i].z += h * w2;
        acc[i].w += h * w3;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) v[i] = add4(v[i], mul4(acc[i], in.lscale));
}

__device__ __forceinline__ float silu(float g) { return g * sigmoid_rcp(g); }

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
  // A thread keeps its pieces (EP of them, H <= 8 EP RT) in registers for
  // both passes, so the normed operand is written without reading x back.
  constexpr int EP = 2;
  half8 v[EP];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < EP; ++p) {
    const int c = (threadIdx.x + p * RT) * 8;
    v[p] = c < H ? *reinterpret_cast<const half8*>(E + packed_index(id, c, H)) : half8{};
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += (float)v[p][i] * (float)v[p][i];
  }
  const float r = rsqrtf(block_sum2(ss, 0.f, red).x / H + eps);
#pragma unroll
  for (int p = 0; p < EP; ++p) {
    const int c = (threadIdx.x + p * RT) * 8;
    if (c >= H) continue;
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[p][i];
    float4* xo = reinterpret_cast<float4*>(x + (long long)t * H + c);
    xo[0] = make_float4(f[0], f[1], f[2], f[3]);
    xo[1] = make_float4(f[4], f[5], f[6], f[7]);
    const float4 w0 = *reinterpret_cast<const float4*>(w + c);
    const float4 w1 = *reinterpret_cast<const float4*>(w + c + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    half8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (_Float16)(f[i] * r * wv[i]);
    *reinterpret_cast<half8*>(xn + (long long)t * H + c) = o;
  }
}

// After the fused Q/K/V(+LoRA-A) GEMM: y = sum of the split partials plus
// s (x A^T) B^T per projection (src/kernels/lora.cu:181-202, h = x A^T from
// the GEMM's extra columns); stash q_raw/k_raw (fp32, the QK-norm backward
// input) and h, then per head QK-RMSNorm (src/kernels/rmsnorm.cu:36-41 with
// 128-wide rows) and half-split RoPE (src/kernels/rope.cu:7-27).  Writes q, k
// (normed, rotated) and v as fp16 [T, Q + 2 KV].
// Tiled by head: workgroup (head hh of the q | k | v heads, 16 rows), four
// waves of four rows each; lane l owns columns l and l + 64 of the head (its
// rotation pair), so the norm is a wave sum and the adapter slice a lane
// needs is 2 x 16 values held in registers for all its rows.  Every load of
// a wave's rows (partials of every split, the 16 h columns) is issued before
// the first use.
constexpr int QH_ROWS = 16;

// NS > 0: exactly NS split partials, every load issued before the first sum
// (the launch picks NS = 2 or 4; NS = 0 loops over any count).
template <int NS = 0>
__global__ __launch_bounds__(256) void qkv_post_kernel(const QkvPostArgs a, int T) {
  constexpr int RPW = QH_ROWS / 4;
  const int hh = blockIdx.x;
  // the wave index as a scalar: row bases are then SGPR pairs, not per-lane
  // 64-bit address math
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Q = a.nq * HD, KV = a.nkv * HD, NT = Q + 2 * KV;
  const int base = hh * HD;
  const int term = hh < a.nq ? 0 : (hh < a.nq + a.nkv ? 1 : 2);
  const RowIn& in = a.in;
  const bool lora = term < in.nterm;
  const int hcol = in.hcol + R * term;
  float b0[R], b1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    b0[r] = 0.f;
    b1[r] = 0.f;
  }
  if (lora) {
    const LoraTerm& m = in.term[term];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      b0[r] = (float)m.shr[(long long)(m.row0 + r) * m.kp + base + lane];
      b1[r] = (float)m.shr[(long long)(m.row0 + r) * m.kp + base + 64 + lane];
    }
  }
  const int t0 = blockIdx.y * QH_ROWS + w;
  float x0[RPW], x1[RPW], hv[RPW];
  if constexpr (NS > 0) {
    float y0[NS][RPW], y1[NS][RPW], yh[NS][RPW];
#pragma unroll
    for (int k = 0; k < NS; ++k)
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int t = min(t0 + 4 * i, T - 1);
        const float* prow = in.part + (long long)k * in.ss + (long long)t * in.ldp;
        y0[k][i] = prow[base + lane];
        y1[k][i] = prow[base + 64 + lane];
        yh[k][i] = lora ? prow[hcol + (lane & 15)] : 0.f;
      }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      x0[i] = y0[0][i];
      x1[i] = y1[0][i];
      hv[i] = yh[0][i];
#pragma unroll
      for (int k = 1; k < NS; ++k) {
        x0[i] += y0[k][i];
        x1[i] += y1[k][i];
        hv[i] += yh[k][i];
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int t = min(t0 + 4 * i, T - 1);
      const float* prow = in.part + (long long)t * in.ldp;
      x0[i] = prow[base + lane];
      x1[i] = prow[base + 64 + lane];
      hv[i] = lora ? prow[hcol + (lane & 15)] : 0.f;
    }
    for (int k = 1; k < in.split; ++k) {
      float y0[RPW], y1[RPW], yh[RPW];
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        const int t = min(t0 + 4 * i, T - 1);
        const float* prow = in.part + (long long)k * in.ss + (long long)t * in.ldp;
        y0[i] = prow[base + lane];
        y1[i] = prow[base + 64 + lane];
        yh[i] = lora ? prow[hcol + (lane & 15)] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < RPW; ++i) {
        x0[i] += y0[i];
        x1[i] += y1[i];
        hv[i] += yh[i];
      }
    }
  }
  const bool qk = hh < a.nq + a.nkv;
  const float* nw = hh < a.nq ? a.qn : a.kn;
  const float w0 = qk ? nw[lane] : 0.f, w1 = qk ? nw[lane + 64] : 0.f;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int t = t0 + 4 * i;
    if (t >= T) break;
    float v0 = x0[i], v1 = x1[i];
    if (lora) {
      float acc0 = 0.f, acc1 = 0.f;
      // lane r of every 16-lane row holds h[r]
      static_for<R>([&](auto rc) {
        const float h = bcast16<decltype(rc)::value>(hv[i]);
        acc0 += h * b0[decltype(rc)::value];
        acc1 += h * b1[decltype(rc)::value];
      });
      v0 += acc0 * in.lscale;
      v1 += acc1 * in.lscale;
      // the first head of each projection stashes its 16 h columns
      if ((hh == 0 || hh == a.nq || hh == a.nq + a.nkv) && lane < R)
        a.hbuf[(long long)t * 64 + R * term + lane] = hv[i];
    }
    _Float16* out = a.qkv16 + (long long)t * NT + base;
    if (!qk) {
      out[lane] = (_Float16)v0;
      out[64 + lane] = (_Float16)v1;
      continue;
    }
    _Float16* raw = a.qkraw + (long long)t * (Q + KV) + base;
    raw[lane] = (_Float16)v0;
    raw[64 + lane] = (_Float16)v1;
    const float r = rsqrtf(wave_sum(v0 * v0 + v1 * v1) / HD + a.eps);
    const int pos = t % a.S;
    const float cs = a.cosT[pos * (HD / 2) + lane], sn = a.sinT[pos * (HD / 2) + lane];
    const float y0 = v0 * r * w0, y1 = v1 * r * w1;
    out[lane] = (_Float16)(y0 * cs - y1 * sn);
    out[64 + lane] = (_Float16)(y1 * cs + y0 * sn);
  }
}

// After the O(+LoRA-A) GEMM (LoRA term added by its reduction):
// x_mid = x_in + oW^T + s (o A^T) B^T (residual, src/kernels/elementwise.cu:
// 4-15), stash h_o, then the FFN RMSNorm -> fp16.
template <int P>
__global__ __launch_bounds__(RT) void o_post_kernel(const RowIn in,
                                                    const float* __restrict__ x_in,
                                                    const float* __restrict__ w, float eps, int H,
                                                    float* __restrict__ hbuf,
                                                    float* __restrict__ x_mid,
                                                    _Float16* __restrict__ xn2) {
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  float4 wv[P], xi[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = min(4 * ((int)threadIdx.x + p * RT), H - 4);
    wv[p] = ld4(w + c);
    xi[p] = ld4(x_in + (long long)t * H + c);
  }
  float4 v[P], hv;
  load_row<P, true>(in, t, H, v, hv);
  LoraRegs<P, 1> L;
  lora_load<P, 1>(in, H, L);
  store_h(in, hv, hs);
  if ((int)threadIdx.x < in.nh / 4)
    *reinterpret_cast<float4*>(hbuf + (long long)t * 64 + 3 * R + 4 * threadIdx.x) = hv;
  __syncthreads();
  lora_apply<P, 1>(in, hs, L, v);
  float ssq = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= H) continue;
    v[p] = add4(xi[p], v[p]);
    *reinterpret_cast<float4*>(x_mid + (long long)t * H + c) = v[p];
    ssq += v[p].x * v[p].x + v[p].y * v[p].y + v[p].z * v[p].z + v[p].w * v[p].w;
  }
  const float r = rsqrtf(block_sum2(ssq, 0.f, red).x / H + eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= H) continue;
    st_h4(xn2 + (long long)t * H + c,
          make_float4(v[p].x * r * wv[p].x, v[p].y * r * wv[p].y, v[p].z * r * wv[p].z,
                      v[p].w * r * wv[p].w));
  }
}

// Split-K sums of NR rows' pieces (columns 4 tid .. + 3, live when < n) and,
// with HH, of this thread's four raw h columns (tid < nh / 4), rows t0 ..
// t0 + NR - 1 clamped to T - 1: every row's loads of a split are issued
// before that split's in-order adds, so NR rows cost one memory round trip
// per split.
template <int NR, bool HH>
__device__ __forceinline__ void load_rows(const RowIn& in, int t0, int T, int n, float4 (&v)[NR],
                                          float4 (&h)[NR]) {
  const int c = 4 * (int)threadIdx.x;
  const int off = c < n ? c : 0;
  const int hoff = in.hcol + 4 * ((int)threadIdx.x < in.nh / 4 ? (int)threadIdx.x : 0);
  const float* prow[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    prow[i] = in.part + (long long)min(t0 + i, T - 1) * in.ldp;
    v[i] = ld4(prow[i] + off);
    if (HH) h[i] = ld4(prow[i] + hoff);
  }
  for (int k = 1; k < in.split; ++k) {
    float4 x[NR], y[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      x[i] = ld4(prow[i] + (long long)k * in.ss + off);
      if (HH) y[i] = ld4(prow[i] + (long long)k * in.ss + hoff);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      v[i] = add4(v[i], x[i]);
      if (HH) h[i] = add4(h[i], y[i]);
    }
  }
}

// load_rows then mid() as one memory round trip, as load_row_then (NR <= 2
// rows, 4 or 8 splits; load_rows waits for each split before issuing the
// next).  C2: o_dx_post 6.1 -> 4.6 us (one row, load_row_then), o_post at
// two rows 5.8 us.
template <int NR, bool HH, int NS, typename F>
__device__ __forceinline__ void load_rows_ns(const RowIn& in, int t0, int T, int n,
                                             float4 (&v)[NR], float4 (&h)[NR], F&& mid) {
  const int c = 4 * (int)threadIdx.x;
  const int off = c < n ? c : 0;
  const int hoff = in.hcol + 4 * ((int)threadIdx.x < in.nh / 4 ? (int)threadIdx.x : 0);
  const float* prow[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) prow[i] = in.part + (long long)min(t0 + i, T - 1) * in.ldp;
  float4 x[NS][NR], y[NS][NR];
#pragma unroll
  for (int k = 0; k < NS; ++k)
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const float* q = prow[i] + (long long)k * in.ss;
      x[k][i] = ld4(q + off);
      if (HH) y[k][i] = ld4(q + hoff);
    }
  mid();
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    v[i] = x[0][i];
    if (HH) h[i] = y[0][i];
  }
#pragma unroll
  for (int k = 1; k < NS; ++k)
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      v[i] = add4(v[i], x[k][i]);
      if (HH) h[i] = add4(h[i], y[k][i]);
    }
}
// NS > 0: the NS-split straight-line form (the launch picks it for NR <= 2
// and 4 or 8 splits); NS = 0: load_rows, then mid().
template <int NR, bool HH, int NS, typename F>
__device__ __forceinline__ void load_rows_then(const RowIn& in, int t0, int T, int n,
                                               float4 (&v)[NR], float4 (&h)[NR], F&& mid) {
  if constexpr (NS > 0) {
    load_rows_ns<NR, HH, NS>(in, t0, T, n, v, h, mid);
  } else {
    load_rows<NR, HH>(in, t0, T, n, v, h);
    mid();
  }
}

// NR block sums at once (one barrier pair).
template <int NR>
__device__ __forceinline__ void block_sums(float (&a)[NR], float* red) {
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    a[i] = wave_sum(a[i]);
    if ((threadIdx.x & 63) == 0) red[i * RW + w] = a[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    float x = 0.f;
#pragma unroll
    for (int q = 0; q < RW; ++q) x += red[i * RW + q];
    a[i] = x;
  }
  __syncthreads();
}

// o_post for rows of one piece per thread at large T: NR rows a workgroup
// side by side (each thread's four columns of every row), so their loads
// share one memory round trip, their row sums one barrier pair and the
// adapter values (loaded once) every row.  (The one-row kernel spends a
// round trip and three barrier phases a row; rows handled one after another
// in a workgroup, adapter values loaded once, measured no faster than it.)
template <int NR, int NS = 0>
__global__ __launch_bounds__(RT) void o_post_rows_kernel(const RowIn in,
                                                         const float* __restrict__ x_in,
                                                         const float* __restrict__ w, float eps,
                                                         int H, float* __restrict__ hbuf,
                                                         float* __restrict__ x_mid,
                                                         _Float16* __restrict__ xn2, int T) {
  __shared__ float red[NR * RW];
  __shared__ float hs[NR][64];
  const int t0 = blockIdx.x * NR;
  const int c = 4 * (int)threadIdx.x;
  const int cc = min(c, H - 4);
  const bool live = c < H;
  float4 xi[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) xi[i] = ld4(x_in + (long long)min(t0 + i, T - 1) * H + cc);
  float4 v[NR], hv[NR];
  float4 wv;
  LoraRegs<1, 1> L;
  auto mid = [&]() __attribute__((always_inline)) {
    wv = ld4(w + cc);
    lora_load<1, 1>(in, H, L);
  };
  load_rows_then<NR, true, NS>(in, t0, T, H, v, hv, mid);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    store_h(in, hv[i], hs[i]);
    if ((int)threadIdx.x < in.nh / 4 && t0 + i < T)
      *reinterpret_cast<float4*>(hbuf + (long long)(t0 + i) * 64 + 3 * R + 4 * threadIdx.x) = hv[i];
  }
  __syncthreads();
  lora_apply_rows<NR, 1>(in, hs, L, v);
  float ssq[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    v[i] = add4(xi[i], v[i]);
    if (live && t0 + i < T) *reinterpret_cast<float4*>(x_mid + (long long)(t0 + i) * H + c) = v[i];
    ssq[i] = live ? v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w : 0.f;
  }
  block_sums<NR>(ssq, red);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float r = rsqrtf(ssq[i] / H + eps);
    if (live && t0 + i < T)
      st_h4(xn2 + (long long)(t0 + i) * H + c,
            make_float4(v[i].x * r * wv.x, v[i].y * r * wv.y, v[i].z * r * wv.z,
                        v[i].w * r * wv.w));
  }
}

// NR block maxima at once (one barrier pair).
template <int NR>
__device__ __forceinline__ void block_maxes(float (&a)[NR], float* red) {
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    a[i] = wave_max(a[i]);
    if ((threadIdx.x & 63) == 0) red[i * RW + w] = a[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    float x = red[i * RW];
#pragma unroll
    for (int q = 1; q < RW; ++q) x = fmaxf(x, red[i * RW + q]);
    a[i] = x;
  }
  __syncthreads();
}

// resid_norm for rows of one piece per thread at large T, NR rows a
// workgroup side by side (as o_post_rows_kernel).
template <int NR, int NS = 0>
__global__ __launch_bounds__(RT) void resid_norm_rows_kernel(const RowIn in,
                                                             const float* __restrict__ x_res,
                                                             const float* __restrict__ w,
                                                             float eps, int H,
                                                             float* __restrict__ x_out,
                                                             _Float16* __restrict__ xn, int T) {
  __shared__ float red[NR * RW];
  const int t0 = blockIdx.x * NR;
  const int c = 4 * (int)threadIdx.x;
  const int cc = min(c, H - 4);
  const bool live = c < H;
  float4 xr[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) xr[i] = ld4(x_res + (long long)min(t0 + i, T - 1) * H + cc);
  float4 v[NR], hv[NR];
  float4 wv;
  auto mid = [&]() __attribute__((always_inline)) { wv = ld4(w + cc); };
  load_rows_then<NR, false, NS>(in, t0, T, H, v, hv, mid);
  float ssq[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    v[i] = add4(xr[i], v[i]);
    if (live && t0 + i < T) *reinterpret_cast<float4*>(x_out + (long long)(t0 + i) * H + c) = v[i];
    ssq[i] = live ? v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w : 0.f;
  }
  block_sums<NR>(ssq, red);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float r = rsqrtf(ssq[i] / H + eps);
    if (live && t0 + i < T)
      st_h4(xn + (long long)(t0 + i) * H + c,
            make_float4(v[i].x * r * wv.x, v[i].y * r * wv.y, v[i].z * r * wv.z,
                        v[i].w * r * wv.w));
  }
}

// After the fused gate/up GEMM: stash g, u (fp16, for the backward) and
// a = silu(g) * u (src/kernels/activation.cu:5-18) from the fp32 sums as the
// fp16 operand of the down GEMM.
__global__ __launch_bounds__(RT) void gu_post_kernel(const RowIn in, int I, long long n4,
                                                     _Float16* __restrict__ gu,
                                                     _Float16* __restrict__ a16) {
  for (long long i = (long long)blockIdx.x * RT + threadIdx.x; i < n4;
       i += (long long)gridDim.x * RT) {
    const long long t = i / (I / 4);
    const int c = (int)(i - t * (I / 4)) * 4;
    const float* p = in.part + t * in.ldp + c;
    const float4 g = sum_splits4(p, in.split, in.ss);
    const float4 u = sum_splits4(p + I, in.split, in.ss);
    st_h4(gu + t * 2 * I + c, g);
    st_h4(gu + t * 2 * I + I + c, u);
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
template <int P>
__global__ __launch_bounds__(RT) void resid_norm_kernel(const RowIn in,
                                                        const float* __restrict__ x_res,
                                                        const float* __restrict__ w, float eps,
                                                        int H, float* __restrict__ x_out,
                                                        _Float16* __restrict__ xn) {
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  float4 xr[P], wv[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = min(4 * ((int)threadIdx.x + p * RT), H - 4);
    xr[p] = ld4(x_res + (long long)t * H + c);
    wv[p] = ld4(w + c);
  }
  float4 v[P];
  load_partials<P>(in, t, H, v);
  float ssq = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= H) continue;
    v[p] = add4(xr[p], v[p]);
    *reinterpret_cast<float4*>(x_out + (long long)t * H + c) = v[p];
    ssq += v[p].x * v[p].x + v[p].y * v[p].y + v[p].z * v[p].z + v[p].w * v[p].w;
  }
  const float r = rsqrtf(block_sum2(ssq, 0.f, red).x / H + eps);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= H) continue;
    st_h4(xn + (long long)t * H + c,
          make_float4(v[p].x * r * wv[p].x, v[p].y * r * wv[p].y, v[p].z * r * wv[p].z,
                      v[p].w * r * wv[p].w));
  }
}

// Per-head QK-RMSNorm + RoPE on [T, nh, 128] rows (the attention block API's
// k input; its q goes through the same map inside the attention forward, and
// the training step fuses this into qkv_post): 16 lanes per (token, head)
// row, lane j holding the RoPE pairs (d, d + 64) for d = 4 j .. 4 j + 3, so
// every access is 8 (fp16) or 16 (fp32) bytes a lane.
//   y = rope(x * r * w), r = rsqrt(mean x^2 + eps)
// (src/kernels/rmsnorm.cu:6-41; src/kernels/rope.cu:7-46).
constexpr int HN_ROWS = RT / 16;  // rows a workgroup

__device__ __forceinline__ float4 ldh4(const _Float16* p) {
  const half4 h = *reinterpret_cast<const half4*>(p);
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

// Launch arguments: tensor blockIdx.y of segs; every 16-lane group owns HN_R
// rows spaced a grid stride apart, all of whose loads are issued before the
// math (one memory round trip per group of rows).
constexpr int HN_R = 4;
struct HeadNormArgs {
  HeadRows seg[2];
  const float* cosT;
  const float* sinT;
  int S, T;
  float eps;
};

__global__ __launch_bounds__(RT) void head_norm_rope_kernel(const HeadNormArgs a) {
  const HeadRows& sg = a.seg[blockIdx.y];
  const int j = threadIdx.x & 15;
  const long long nrows = (long long)a.T * sg.nh;
  const long long r0 = (long long)blockIdx.x * HN_ROWS + (threadIdx.x >> 4);
  const long long stride = (long long)gridDim.x * HN_ROWS;
  const float4 w0 = ld4(sg.w + 4 * j), w1 = ld4(sg.w + 64 + 4 * j);
  float4 x0[HN_R], x1[HN_R], cs[HN_R], sn[HN_R];
#pragma unroll
  for (int i = 0; i < HN_R; ++i) {
    const long long row = min(r0 + i * stride, nrows - 1);
    // 32-bit division (rows < 2^31, checked on the host): the 64-bit form
    // expands to about a hundred instructions a row
    const int pos = (int)(((unsigned)row / (unsigned)sg.nh) % (unsigned)a.S);
    cs[i] = ld4(a.cosT + pos * (HD / 2) + 4 * j);
    sn[i] = ld4(a.sinT + pos * (HD / 2) + 4 * j);
    x0[i] = ldh4(sg.x + row * HD + 4 * j);
    x1[i] = ldh4(sg.x + row * HD + 64 + 4 * j);
  }
  _Float16* out = sg.out;
#pragma unroll
  for (int i = 0; i < HN_R; ++i) {
    const long long row = r0 + i * stride;
    const float ss = x0[i].x * x0[i].x + x0[i].y * x0[i].y + x0[i].z * x0[i].z +
                     x0[i].w * x0[i].w + x1[i].x * x1[i].x + x1[i].y * x1[i].y +
                     x1[i].z * x1[i].z + x1[i].w * x1[i].w;
    const float r = rsqrtf(sum16_dpp(ss) / HD + a.eps);
    if (row >= nrows) continue;  // whole 16-lane groups (after the group sum)
    const float a0[4] = {x0[i].x * r * w0.x, x0[i].y * r * w0.y, x0[i].z * r * w0.z,
                         x0[i].w * r * w0.w};
    const float a1[4] = {x1[i].x * r * w1.x, x1[i].y * r * w1.y, x1[i].z * r * w1.z,
                         x1[i].w * r * w1.w};
    const float c[4] = {cs[i].x, cs[i].y, cs[i].z, cs[i].w};
    const float s4[4] = {sn[i].x, sn[i].y, sn[i].z, sn[i].w};
    half4 o0, o1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o0[e] = (_Float16)(a0[e] * c[e] - a1[e] * s4[e]);
      o1[e] = (_Float16)(a1[e] * c[e] + a0[e] * s4[e]);
    }
    *reinterpret_cast<half4*>(out + row * HD + 4 * j) = o0;
    *reinterpret_cast<half4*>(out + row * HD + 64 + 4 * j) = o1;
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
template <int P>
__global__ __launch_bounds__(RT) void norm_bwd_kernel(const NormBwdArgs a) {
  __shared__ float red[2 * RW];
  __shared__ float hs[64];
  const int t = blockIdx.x;
  const int H = a.H;
  float4 xv[P], wv[P], dr[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = min(4 * ((int)threadIdx.x + p * RT), H - 4);
    xv[p] = ld4(a.x + (long long)t * H + c);
    wv[p] = ld4(a.w + c);
    dr[p] = a.dres_in ? ld4(a.dres_in + (long long)t * H + c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float rs = (a.rinv_in ? a.rinv_in[t] : 1.0f) * a.gscale;
  float4 v[P], hv;
  LoraRegs<P, 3> L;
  bool have_l = false;
  if constexpr (P == 1) {  // (wider rows would spill)
    // the row's partials and the adapter values in one round trip
    load_row_then<P>(a.in, t, H, v, hv, [&]() __attribute__((always_inline)) {
      if (a.in.nterm) lora_load<P, 3>(a.in, H, L);
    });
    have_l = true;
  } else {
    load_row<P, true>(a.in, t, H, v, hv);
  }
  store_h(a.in, hv, hs);
  if ((int)threadIdx.x < a.in.nh / 4)
    *reinterpret_cast<float4*>(a.dh_out + (long long)t * 64 + a.dh_col + 4 * threadIdx.x) =
        mul4(hv, rs);
  if (a.in.nterm) {
    if (!have_l) lora_load<P, 3>(a.in, H, L);
    __syncthreads();
    lora_apply<P, 3>(a.in, hs, L, v);
  }
  float dot = 0.f, ssx = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= H) continue;
    v[p] = mul4(v[p], rs);
    dot += v[p].x * wv[p].x * xv[p].x + v[p].y * wv[p].y * xv[p].y + v[p].z * wv[p].z * xv[p].z +
           v[p].w * wv[p].w * xv[p].w;
    ssx += xv[p].x * xv[p].x + xv[p].y * xv[p].y + xv[p].z * xv[p].z + xv[p].w * xv[p].w;
  }
  const float2 s2 = block_sum2(dot, ssx, red);
  const float r = rsqrtf(s2.y / H + a.eps);
  const float coef = r * r / H * s2.x;
  float amax = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= H) continue;
    const float4 d = v[p], x = xv[p], ww = wv[p];
    v[p] = make_float4(dr[p].x + r * (d.x * ww.x - coef * x.x), dr[p].y + r * (d.y * ww.y - coef * x.y),
                       dr[p].z + r * (d.z * ww.z - coef * x.z), dr[p].w + r * (d.w * ww.w - coef * x.w));
    *reinterpret_cast<float4*>(a.dres_out + (long long)t * H + c) = v[p];
    if (a.dmid_out) *reinterpret_cast<float4*>(a.dmid_out + (long long)t * H + c) = v[p];
    if (a.g16_ks) v[p] = mul4v(v[p], ldh4(a.g16_ks + c));
    amax = fmaxf(amax, amax4(v[p]));
  }
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) a.rinv_out[t] = 1.0f / sc;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c < H) st_h4(a.g16 + (long long)t * H + c, mul4(v[p], sc));
  }
}

// norm_bwd for rows of one piece per thread at large T, NR rows a workgroup
// side by side (as o_post_rows_kernel), with no adapter terms or with three
// (LORA: the attention norm's q, k, v terms, each over all H columns, whose
// 48 x 4 values a thread loads once for all its rows).
// The attention norm's LoRA dx term s (dh_q A_q + dh_k A_k + dh_v A_v) of
// NR rows on MFMA (16 x 16 x 16 fp16: rows x ranks of one adapter times
// ranks x 16 columns): wave w takes columns 256 w .. of the row, A operand
// = the rows' dh values (rows past NR zero), scaled by 2^-10 into fp16 range
// (dh is in the GEMM's scaled units), B operand = 4 consecutive ranks of one
// column from the transposed copy at [H][48].  The 16 x 16 results go
// through LDS (out[NR][H], H <= 4 RT) to the thread that owns the column.
constexpr float kLoraMfmaScale = 1.0f / 1024.0f;

template <int NR>
__device__ __forceinline__ void lora_rows_mfma(const NormBwdArgs& a, const float (*hs)[64],
                                               float* out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kq = lane >> 4, n = lane & 15;
  half4 aop[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const float4 h4 = n < NR ? *reinterpret_cast<const float4*>(&hs[n][a.in.term[q].hidx + 4 * kq])
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    aop[q] = half4{(_Float16)(h4.x * kLoraMfmaScale), (_Float16)(h4.y * kLoraMfmaScale),
                   (_Float16)(h4.z * kLoraMfmaScale), (_Float16)(h4.w * kLoraMfmaScale)};
  }
  const int H = a.H;
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) {
    const int cb = 256 * wave + 64 * cg;
    if (cb >= H) break;  // wave-uniform
    half4 b[3][4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int col = min(cb + 16 * nb + n, H - 1);
#pragma unroll
      for (int q = 0; q < 3; ++q)
        b[q][nb] = *reinterpret_cast<const half4*>(a.lora_at + (long long)col * (3 * R) + q * R + 4 * kq);
    }
    floatx4 acc[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 3; ++q)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(aop[q], b[q][nb], acc[nb], 0, 0, 0);
    }
    // lane: rows 4 kq + i of column cb + 16 nb + n
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 4 * kq + i;
      if (row >= NR) continue;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int col = cb + 16 * nb + n;
        if (col < H) out[row * H + col] = acc[nb][i];
      }
    }
  }
}

// LM: 0 no adapter terms, 1 the q/k/v terms on VALU, 2 on MFMA
// (lora_rows_mfma: 255 -> 229 VGPRs, C4 52.6 -> 45.9 us a layer).
template <int NR, int LM, bool NT = false>
__global__ __launch_bounds__(RT) void norm_bwd_rows_kernel(const NormBwdArgs a, int T) {
  constexpr bool LORA = LM > 0;
  __shared__ float red[2 * NR * RW];
  __shared__ __attribute__((aligned(16))) float hs[NR][64];
  const int H = a.H;
  const int t0 = blockIdx.x * NR;
  const int c = 4 * (int)threadIdx.x;
  const int cc = min(c, H - 4);
  const bool live = c < H;
  float4 xv[NR], dr[NR];
  float rs[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int t = min(t0 + i, T - 1);
    xv[i] = ld4s<NT>(a.x + (long long)t * H + cc);
    dr[i] = a.dres_in ? ld4s<NT>(a.dres_in + (long long)t * H + cc) : make_float4(0.f, 0.f, 0.f, 0.f);
    rs[i] = (a.rinv_in ? a.rinv_in[t] : 1.0f) * a.gscale;
  }
  float4 v[NR], hv[NR];
  load_rows<NR, true>(a.in, t0, T, H, v, hv);
  const float4 ww = ld4(a.w + cc);
  const float4 ks4 = a.g16_ks ? ldh4(a.g16_ks + cc) : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    if (LORA) store_h(a.in, hv[i], hs[i]);
    if ((int)threadIdx.x < a.in.nh / 4 && t0 + i < T)
      *reinterpret_cast<float4*>(a.dh_out + (long long)(t0 + i) * 64 + a.dh_col + 4 * threadIdx.x) =
          mul4(hv[i], rs[i]);
  }
  if constexpr (LM == 2) {
    __shared__ __attribute__((aligned(16))) float lora_out[NR * 4 * RT];  // [NR][H]
    __syncthreads();
    lora_rows_mfma<NR>(a, hs, lora_out);
    __syncthreads();
    const float ls = a.in.lscale / kLoraMfmaScale;
#pragma unroll
    for (int i = 0; i < NR; ++i)
      v[i] = add4(v[i], mul4(*reinterpret_cast<const float4*>(&lora_out[i * H + cc]), ls));
  } else if constexpr (LM == 1) {
    LoraRegs<1, 3> L;
    lora_load<1, 3>(a.in, H, L);
    __syncthreads();
    lora_apply_rows<NR, 3>(a.in, hs, L, v);
  }
  float s2[2 * NR];  // dot(d w, x), then sum x^2, of each row
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float4 d = mul4(v[i], rs[i]), x = xv[i];
    v[i] = d;
    s2[i] = live ? d.x * ww.x * x.x + d.y * ww.y * x.y + d.z * ww.z * x.z + d.w * ww.w * x.w : 0.f;
    s2[NR + i] = live ? x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w : 0.f;
  }
  block_sums<2 * NR>(s2, red);
  float amax[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float r = rsqrtf(s2[NR + i] / H + a.eps);
    const float coef = r * r / H * s2[i];
    const float4 d = v[i], x = xv[i];
    v[i] = make_float4(dr[i].x + r * (d.x * ww.x - coef * x.x), dr[i].y + r * (d.y * ww.y - coef * x.y),
                       dr[i].z + r * (d.z * ww.z - coef * x.z), dr[i].w + r * (d.w * ww.w - coef * x.w));
    if (live && t0 + i < T) {
      *reinterpret_cast<float4*>(a.dres_out + (long long)(t0 + i) * H + c) = v[i];
      if (a.dmid_out) *reinterpret_cast<float4*>(a.dmid_out + (long long)(t0 + i) * H + c) = v[i];
    }
    v[i] = mul4v(v[i], ks4);
    amax[i] = live ? amax4(v[i]) : 0.f;
  }
  block_maxes<NR>(amax, red);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    if (t0 + i >= T) continue;
    const float sc = pow2_scale_for(amax[i]);
    if (threadIdx.x == 0) a.rinv_out[t0 + i] = 1.0f / sc;
    if (live) st_h4(a.g16 + (long long)(t0 + i) * H + c, mul4(v[i], sc));
  }
}

// dX of the down projection -> SwiGLU backward (src/kernels/activation.cu:
// 26-43 with d_up = dy * silu(g), i.e. without the reference's aliasing of
// d_gate and d_swiglu at src/kernels/lora_backward.cu:287) -> [dg | du] fp16.
template <int P, bool SC = false, bool NTG = false>
__global__ __launch_bounds__(RT) void swiglu_bwd_kernel(const RowIn in,
                                                        const float* __restrict__ rinv_in,
                                                        const _Float16* __restrict__ gu, int I,
                                                        _Float16* __restrict__ dgu16,
                                                        float* __restrict__ rinv_out,
                                                        const _Float16* __restrict__ ks) {
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  const _Float16* gr = gu + (long long)t * 2 * I;
  float4 g4[P], u4[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = min(4 * ((int)threadIdx.x + p * RT), I - 4);
    if (NTG) {
      const half4 a = __builtin_nontemporal_load(reinterpret_cast<const half4*>(gr + c));
      const half4 b = __builtin_nontemporal_load(reinterpret_cast<const half4*>(gr + I + c));
      g4[p] = make_float4((float)a[0], (float)a[1], (float)a[2], (float)a[3]);
      u4[p] = make_float4((float)b[0], (float)b[1], (float)b[2], (float)b[3]);
    } else {
      g4[p] = ldh4(gr + c);
      u4[p] = ldh4(gr + I + c);
    }
  }
  const float rs = rinv_in[t];
  float4 v[P];
  load_partials<P, SC>(in, t, I, v);
  float4 dg[P], du[P];
  float amax = 0.f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float da[4] = {v[p].x * rs, v[p].y * rs, v[p].z * rs, v[p].w * rs};
    const float g[4] = {g4[p].x, g4[p].y, g4[p].z, g4[p].w};
    const float u[4] = {u4[p].x, u4[p].y, u4[p].z, u4[p].w};
    float o1[4], o2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float sg = sigmoid_rcp(g[e]);
      o1[e] = da[e] * u[e] * (sg * (1.0f + g[e] * (1.0f - sg)));
      o2[e] = da[e] * (g[e] * sg);
    }
    dg[p] = make_float4(o1[0], o1[1], o1[2], o1[3]);
    du[p] = make_float4(o2[0], o2[1], o2[2], o2[3]);
    if (ks) {
      const int c = min(4 * ((int)threadIdx.x + p * RT), I - 4);
      dg[p] = mul4v(dg[p], ldh4(ks + c));
      du[p] = mul4v(du[p], ldh4(ks + I + c));
    }
    if (4 * ((int)threadIdx.x + p * RT) < I) amax = fmaxf(amax, fmaxf(amax4(dg[p]), amax4(du[p])));
  }
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) rinv_out[t] = 1.0f / sc;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    if (c >= I) continue;
    st_h4(dgu16 + (long long)t * 2 * I + c, mul4(dg[p], sc));
    st_h4(dgu16 + (long long)t * 2 * I + I + c, mul4(du[p], sc));
  }
}

// dX of the O projection (+ dh_o in the LoRA-B^T columns; the reduction
// adds s (dh_o A_o)): d_o = row * rinv; writes dh_o, the attention
// backward's dO operand and the flash-backward row statistic
// delta[b, h, s] = sum_d dO * O.  dO goes out as fp16 per (row, head), scaled
// by the power of two of that head's max |dO| (inverse in dsc[b, h, s]).
// Tiled by head: workgroup = head h x 8 rows, four waves of two rows, lane l
// owns columns 2l, 2l + 1 of the head (8-byte loads of every split partial),
// so delta and the head's max are wave reductions and a lane's adapter slice
// (2 x 16 values) stays in registers for both its rows.
constexpr int OD_ROWS = 8;

__global__ __launch_bounds__(256) void o_dx_post_kernel(const RowIn in,
                                                        const float* __restrict__ rinv_in,
                                                        const _Float16* __restrict__ o16, int nq,
                                                        int S, int T, float* __restrict__ dh_out,
                                                        _Float16* __restrict__ dO16,
                                                        float* __restrict__ delta,
                                                        float* __restrict__ dsc) {
  constexpr int RPW = OD_ROWS / 4;
  const int h = blockIdx.x;
  // the wave index as a scalar: row bases are then SGPR pairs, not per-lane
  // 64-bit address math
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int Q = nq * HD, col = h * HD + 2 * lane;
  const bool lora = in.nterm > 0;
  float b0[R], b1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    b0[r] = 0.f;
    b1[r] = 0.f;
  }
  if (lora) {
    const LoraTerm& m = in.term[0];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const half2v bb = *reinterpret_cast<const half2v*>(m.shr + (long long)(m.row0 + r) * m.kp + col);
      b0[r] = (float)bb[0];
      b1[r] = (float)bb[1];
    }
  }
  const int t0 = blockIdx.y * OD_ROWS + w;
  float2 x[RPW];
  float hv[RPW];
  half2v oo[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int t = min(t0 + 4 * i, T - 1);
    const float* prow = in.part + (long long)t * in.ldp;
    x[i] = *reinterpret_cast<const float2*>(prow + col);
    hv[i] = lora ? prow[in.hcol + (lane & 15)] : 0.f;
    oo[i] = *reinterpret_cast<const half2v*>(o16 + (long long)t * Q + col);
  }
  for (int k = 1; k < in.split; ++k) {
    float2 y[RPW];
    float yh[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int t = min(t0 + 4 * i, T - 1);
      const float* prow = in.part + (long long)k * in.ss + (long long)t * in.ldp;
      y[i] = *reinterpret_cast<const float2*>(prow + col);
      yh[i] = lora ? prow[in.hcol + (lane & 15)] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      x[i].x += y[i].x;
      x[i].y += y[i].y;
      hv[i] += yh[i];
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int t = t0 + 4 * i;
    if (t >= T) break;
    const float rs = rinv_in[t];
    float v0 = x[i].x, v1 = x[i].y;
    if (lora) {
      float acc0 = 0.f, acc1 = 0.f;
      // lane r of every 16-lane row holds h[r]
      static_for<R>([&](auto rc) {
        const float hr = bcast16<decltype(rc)::value>(hv[i]);
        acc0 += hr * b0[decltype(rc)::value];
        acc1 += hr * b1[decltype(rc)::value];
      });
      v0 += acc0 * in.lscale;
      v1 += acc1 * in.lscale;
      if (h == 0 && lane < R) dh_out[(long long)t * 64 + 3 * R + lane] = hv[i] * rs;
    }
    const float d0 = v0 * rs, d1 = v1 * rs;
    const int b = t / S, s = t - b * S;
    const long long bhs = ((long long)b * nq + h) * S + s;
    const float dl = wave_sum(d0 * (float)oo[i][0] + d1 * (float)oo[i][1]);
    const float amax = wave_max(fmaxf(fabsf(d0), fabsf(d1)));
    const float sc = pow2_scale_for(amax, kDoScaleExp);
    if (lane == 0) {
      delta[bhs] = dl;
      dsc[bhs] = pow2_inv_scale_for(amax, kDoScaleExp);
    }
    half2v o2;
    o2[0] = (_Float16)(d0 * sc);
    o2[1] = (_Float16)(d1 * sc);
    *reinterpret_cast<half2v*>(dO16 + (long long)t * Q + col) = o2;
  }
}

// The same epilogue with one token row per workgroup, for GEMMs with many
// split partials (a thread sums 16-byte pieces of every split, one load
// each): thread i owns columns 4 i .. 4 i + 3 of piece p, so a head is 32
// consecutive threads and its delta and max are 32-lane shuffle sums.
template <int P>
__global__ __launch_bounds__(RT) void o_dx_post_row_kernel(const RowIn in,
                                                           const float* __restrict__ rinv_in,
                                                           const _Float16* __restrict__ o16,
                                                           int nq, int S,
                                                           float* __restrict__ dh_out,
                                                           _Float16* __restrict__ dO16,
                                                           float* __restrict__ delta,
                                                           float* __restrict__ dsc) {
  __shared__ float hs[64];
  const int t = blockIdx.x;
  const int Q = nq * HD;
  half4 ov[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = min(4 * ((int)threadIdx.x + p * RT), Q - 4);
    ov[p] = *reinterpret_cast<const half4*>(o16 + (long long)t * Q + c);
  }
  const float rs = rinv_in[t];
  float4 v[P], hv;
  LoraRegs<P, 1> L;
  if constexpr (P == 1) {  // (wider rows would spill)
    load_row_then<P>(in, t, Q, v, hv,
                     [&]() __attribute__((always_inline)) { lora_load<P, 1>(in, Q, L); });
  } else {
    load_row<P, true>(in, t, Q, v, hv);
    lora_load<P, 1>(in, Q, L);
  }
  store_h(in, hv, hs);
  if ((int)threadIdx.x < in.nh / 4)
    *reinterpret_cast<float4*>(dh_out + (long long)t * 64 + 3 * R + 4 * threadIdx.x) = mul4(hv, rs);
  __syncthreads();
  lora_apply<P, 1>(in, hs, L, v);
  const int b = t / S, s = t - b * S;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int c = 4 * ((int)threadIdx.x + p * RT);
    const bool live = c < Q;  // uniform over the head's 32 threads
    const float4 d = mul4(v[p], rs);
    float part = live ? d.x * (float)ov[p][0] + d.y * (float)ov[p][1] + d.z * (float)ov[p][2] +
                            d.w * (float)ov[p][3]
                      : 0.f;
    float amax = live ? amax4(d) : 0.f;
    part = sum32(part);
    amax = max32(amax);
    if (!live) continue;
    st_h4(dO16 + (long long)t * Q + c, mul4(d, pow2_scale_for(amax, kDoScaleExp)));
    if ((threadIdx.x & 31) == 0) {
      const long long bhs = ((long long)b * nq + c / HD) * S + s;
      delta[bhs] = part;
      dsc[bhs] = pow2_inv_scale_for(amax, kDoScaleExp);
    }
  }
}

// Attention gradients (w.r.t. the normed, rotated q/k and v) -> RoPE
// backward (inverse rotation, src/kernels/rope.cu:57-89) -> QK-RMSNorm
// backward with x = q_raw/k_raw (src/kernels/rmsnorm.cu:53-95) ->
// dy = [dq_raw | dk_raw | dv] fp32 (the LoRA dB operand) and fp16 (scaled).
// HPW > 0: every load of a row (a wave's nq + nkv <= HPW RW heads, then
// KV <= 2 RT v columns) is issued before any of the math (the rows are
// latency-bound at small T).  HPW = 0: one head at a time, any shape.
template <int HPW>
__global__ __launch_bounds__(RT) void qk_bwd_kernel(const QkBwdArgs a) {
  extern __shared__ float ds[];  // [NT]
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  const int Q = a.nq * HD, KV = a.nkv * HD, NT = Q + 2 * KV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pos = t % a.S;
  const float cs = a.cosT[pos * (HD / 2) + lane], sn = a.sinT[pos * (HD / 2) + lane];
  const float* g = a.dqkv + (long long)t * a.ld_dqkv;
  auto head = [&](int hh, float d0, float d1, float x0, float x1, float w0,
                  float w1) __attribute__((always_inline)) {
    const int base = hh * HD;
    const float n0 = d0 * cs + d1 * sn, n1 = d1 * cs - d0 * sn;
    const float r = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / HD + a.eps);
    const float dot = wave_sum(n0 * w0 * x0 + n1 * w1 * x1);
    const float coef = r * r / HD * dot;
    ds[base + lane] = r * (n0 * w0 - coef * x0);
    ds[base + 64 + lane] = r * (n1 * w1 - coef * x1);
  };
  const _Float16* xrow = a.qkraw + (long long)t * (Q + KV);
  if constexpr (HPW > 0) {
    const float wq0 = a.qn[lane], wq1 = a.qn[lane + 64], wk0 = a.kn[lane], wk1 = a.kn[lane + 64];
    float vv[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = Q + KV + threadIdx.x + u * RT;
      vv[u] = g[c < NT ? c : Q + KV];
    }
    float d0[HPW], d1[HPW], x0[HPW], x1[HPW];
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const int hh = __builtin_amdgcn_readfirstlane(wave + k * RW);
      const int base = (hh < a.nq + a.nkv ? hh : 0) * HD;
      d0[k] = g[base + lane];
      d1[k] = g[base + 64 + lane];
      x0[k] = (float)xrow[base + lane];
      x1[k] = (float)xrow[base + 64 + lane];
    }
#pragma unroll
    for (int k = 0; k < HPW; ++k)
      if (wave + k * RW < a.nq + a.nkv) {
        const bool isq = wave + k * RW < a.nq;
        head(wave + k * RW, d0[k], d1[k], x0[k], x1[k], isq ? wq0 : wk0, isq ? wq1 : wk1);
      }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = Q + KV + threadIdx.x + u * RT;
      if (c < NT) ds[c] = vv[u];
    }
  } else {
    for (int hh = wave; hh < a.nq + a.nkv; hh += RW) {
      const int base = hh * HD;
      const float* w = hh < a.nq ? a.qn : a.kn;
      head(hh, g[base + lane], g[base + 64 + lane], xrow[base + lane], xrow[base + 64 + lane],
           w[lane], w[lane + 64]);
    }
    for (int c = Q + KV + threadIdx.x; c < NT; c += RT) ds[c] = g[c];
  }
  __syncthreads();
  // the operand is times the per-column factor when one is given (dy32, the
  // fp32 gradient, is not); a thread rescales only the columns it owns
  // NT <= 8 RT (Qwen3-1.7B: 4096 = 8 x 512): thread i owns the eight
  // columns 8 i .., so its fp32 reads of ds and its fp16 operand store are
  // 16 bytes each (eight 2-byte stores a thread column by column)
  const int c8 = 8 * (int)threadIdx.x;
  const bool own8 = c8 < NT;
  if (NT <= 8 * RT) {
    float v[8];
    float amax = 0.f;
    if (own8) {
      const float4 lo = *reinterpret_cast<const float4*>(&ds[c8]);
      const float4 hi = *reinterpret_cast<const float4*>(&ds[c8 + 4]);
      if (a.dy32) {
        *reinterpret_cast<float4*>(a.dy32 + (long long)t * NT + c8) = lo;
        *reinterpret_cast<float4*>(a.dy32 + (long long)t * NT + c8 + 4) = hi;
      }
      v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
      v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = block_max<RW>(amax, red);
    const float sc = pow2_scale_for(amax);
    if (threadIdx.x == 0) a.rinv_out[t] = 1.0f / sc;
    if (own8) {
      half8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (_Float16)(v[e] * sc);
      *reinterpret_cast<half8*>(a.g16 + (long long)t * NT + c8) = o;
    }
    return;
  }
  // wider rows: a column a thread per pass
  float amax = 0.f;
  for (int c = threadIdx.x; c < NT; c += RT) {
    const float v = ds[c];
    if (a.dy32) a.dy32[(long long)t * NT + c] = v;
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

// dres = dy; g16 = fp16(dy ks * sc); rinv = 1 / sc (sc: the row's power-of-two
// scale; ks the operand's per-column factor, 1 when ks is NULL).
__global__ __launch_bounds__(RT) void grad_rows_kernel(const float* dy, int H, float* dres,
                                                       _Float16* __restrict__ g16,
                                                       float* __restrict__ rinv,
                                                       const _Float16* __restrict__ ks) {
  __shared__ float red[2 * RW];
  const int t = blockIdx.x;
  float amax = 0.f;
  for (int c = threadIdx.x; c < H; c += RT)
    amax = fmaxf(amax, fabsf(dy[(long long)t * H + c] * (ks ? (float)ks[c] : 1.0f)));
  amax = block_max<RW>(amax, red);
  const float sc = pow2_scale_for(amax);
  if (threadIdx.x == 0) rinv[t] = 1.0f / sc;
  for (int c = threadIdx.x; c < H; c += RT) {
    const float v = dy[(long long)t * H + c];
    dres[(long long)t * H + c] = v;
    g16[(long long)t * H + c] = (_Float16)(v * (ks ? (float)ks[c] : 1.0f) * sc);
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

// Token rows a workgroup of the parallel-rows epilogues (o_post, resid_norm,
// norm_bwd with rows of one piece per thread): NR rows side by side share a
// memory round trip, a barrier pair per reduction and (o_post, the attention
// norm's backward) the adapter values.  At T >= 2048 each kernel takes the
// count measured best for it (C4, 4096 rows, us at NR = 1 / 2 / 4 / 8):
// resid_norm 37.1 / 24.2 / 24.5 / 25.6, norm_bwd 41.5 / 32.1 / 34.5 / 41.7,
// o_post 52.8 / 32.1 / 30.5 / 35.3, norm_bwd with the three adapter terms
// 82.3 / 76.7 / 68.0 / 58.7 (its 196 KB of adapter values per workgroup).
// At short T (the B1 x S128 step) one row a workgroup keeps more CUs busy,
// except for resid_norm (4.84 against 4.39 us at two rows, 128 rows) and
// o_post (5.95 against 5.70 us; norm_bwd 5.0 / 5.9 / 9.0, with the adapter
// terms 8.4 / 9.7 / 13.0 at 1 / 2 / 4 rows).
// LLMT_ROWS_PER_WG (1, 2, 3, 4 or 8) overrides all of them.
static int rows_per_wg(int T, int P, int large_t, int small_t = 1) {
  if (P != 1) return 1;
  const char* e = getenv("LLMT_ROWS_PER_WG");
  if (e && *e) {
    const int v = atoi(e);
    if (v == 1 || v == 2 || v == 3 || v == 4 || v == 8) return v;
  }
  return T >= 2048 ? large_t : small_t;
}

// split_col_ok: the kernel reads its partials through load_row, which alone
// honours RowIn::split_col.
static bool row_in_ok(const RowIn& in, int n, const char* who, bool split_col_ok = false) {
  bool ok = in.nh % 4 == 0 && in.nh >= 0 && in.nh <= 64 && in.nterm >= 0 && in.nterm <= 3 &&
            n % 4 == 0 && in.ldp % 4 == 0 && in.split >= 1 && (in.split == 1 || in.ss % 4 == 0) &&
            in.hcol % 4 == 0 && in.split_col >= 0 && in.split_col % 4 == 0 &&
            (in.split_col == 0 || split_col_ok);
  for (int q = 0; q < in.nterm && ok; ++q)
    ok = in.term[q].c0 % 4 == 0 && in.term[q].n % 4 == 0 && in.term[q].hidx + R <= in.nh;
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
                     const _Float16* ks, hipStream_t st) {
  hipLaunchKernelGGL(grad_rows_kernel, dim3(T), dim3(RT), 0, st, dy, H, dres, g16, rinv, ks);
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
  if (H % 8 || H > 2 * 8 * RT || ((uintptr_t)x | (uintptr_t)xn | (uintptr_t)w) % 16) {
    set_error("embed_norm: H=%d (a multiple of 8, at most %d) and 16-byte aligned rows required",
              H, 2 * 8 * RT);
    return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(embed_norm_kernel, dim3(T), dim3(RT), 0, st, tok, E, V, H, w, eps, x, xn);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t qkv_post(const QkvPostArgs& a, int T, hipStream_t st) {
  const int Q = a.nq * HD, KV = a.nkv * HD, NT = Q + 2 * KV;
  if (!row_in_ok(a.in, NT, "qkv_post")) return hipErrorInvalidValue;
  // adapter terms q, k, v over their own column ranges, h columns in order
  bool ok = a.in.nterm == 0 || (a.in.nterm == 3 && a.in.nh == 3 * R);
  const int c0[3] = {0, Q, Q + KV}, n[3] = {Q, KV, KV};
  for (int q = 0; q < a.in.nterm && ok; ++q)
    ok = a.in.term[q].c0 == c0[q] && a.in.term[q].n == n[q] && a.in.term[q].hidx == R * q;
  if (!ok) {
    set_error("qkv_post: LoRA terms must be q, k, v over their own columns");
    return hipErrorInvalidValue;
  }
  const dim3 grid(a.nq + 2 * a.nkv, (T + QH_ROWS - 1) / QH_ROWS);
  // (2 or 4 split partials, the B1 x S128 step: one memory round trip,
  // 4.47 -> 4.33 us a layer)
  if (a.in.split == 2)
    hipLaunchKernelGGL(qkv_post_kernel<2>, grid, dim3(256), 0, st, a, T);
  else if (a.in.split == 4)
    hipLaunchKernelGGL(qkv_post_kernel<4>, grid, dim3(256), 0, st, a, T);
  else
    hipLaunchKernelGGL(qkv_post_kernel<0>, grid, dim3(256), 0, st, a, T);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}


hipError_t o_post(const RowIn& in, const float* x_in, const float* w, float eps, int H, int T,
                  float* hbuf, float* x_mid, _Float16* xn2, hipStream_t st) {
  if (!row_in_ok(in, H, "o_post")) return hipErrorInvalidValue;
  const int P = (H + 4 * RT - 1) / (4 * RT);
  const int nr = rows_per_wg(T, P, 4, 2);
  const dim3 g((T + nr - 1) / nr);
  switch (P * 10 + nr) {
    case 11: hipLaunchKernelGGL((o_post_kernel<1>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2); break;
    case 12:
      // (4 or 8 split partials: every load of the two rows in one round trip)
      if (in.split == 4)
        hipLaunchKernelGGL((o_post_rows_kernel<2, 4>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2, T);
      else if (in.split == 8)
        hipLaunchKernelGGL((o_post_rows_kernel<2, 8>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2, T);
      else
        hipLaunchKernelGGL((o_post_rows_kernel<2>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2, T);
      break;
    case 13: hipLaunchKernelGGL((o_post_rows_kernel<3>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2, T); break;
    case 14: hipLaunchKernelGGL((o_post_rows_kernel<4>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2, T); break;
    case 18: hipLaunchKernelGGL((o_post_rows_kernel<8>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2, T); break;
    case 21: hipLaunchKernelGGL((o_post_kernel<2>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2); break;
    case 31: hipLaunchKernelGGL((o_post_kernel<3>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2); break;
    case 41: hipLaunchKernelGGL((o_post_kernel<4>), g, dim3(RT), 0, st, in, x_in, w, eps, H, hbuf, x_mid, xn2); break;
    default:
      set_error("o_post: row width %d above %d", H, 16 * RT);
      return hipErrorInvalidValue;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t gu_post(const RowIn& in, int I, int T, _Float16* gu, _Float16* a16, hipStream_t st) {
  if (!row_in_ok(in, I, "gu_post") || in.nterm) return hipErrorInvalidValue;
  const long long n4 = (long long)T * (I / 4);
  hipLaunchKernelGGL(gu_post_kernel, dim3(grid_elems(n4)), dim3(RT), 0, st, in, I, n4, gu, a16);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t resid_norm(const RowIn& in, const float* x_res, const float* w, float eps, int H, int T,
                      float* x_out, _Float16* xn, hipStream_t st) {
  if (!row_in_ok(in, H, "resid_norm")) return hipErrorInvalidValue;
  const int P = (H + 4 * RT - 1) / (4 * RT);
  const int nr = rows_per_wg(T, P, 2, 2);
  const dim3 g((T + nr - 1) / nr);
  switch (P * 10 + nr) {
    case 11: hipLaunchKernelGGL(resid_norm_kernel<1>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn); break;
    case 12:
      if (in.split == 4)
        hipLaunchKernelGGL((resid_norm_rows_kernel<2, 4>), g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn, T);
      else if (in.split == 8)
        hipLaunchKernelGGL((resid_norm_rows_kernel<2, 8>), g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn, T);
      else
        hipLaunchKernelGGL(resid_norm_rows_kernel<2>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn, T);
      break;
    case 13: hipLaunchKernelGGL(resid_norm_rows_kernel<3>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn, T); break;
    case 14: hipLaunchKernelGGL(resid_norm_rows_kernel<4>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn, T); break;
    case 18: hipLaunchKernelGGL(resid_norm_rows_kernel<8>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn, T); break;
    case 21: hipLaunchKernelGGL(resid_norm_kernel<2>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn); break;
    case 31: hipLaunchKernelGGL(resid_norm_kernel<3>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn); break;
    case 41: hipLaunchKernelGGL(resid_norm_kernel<4>, g, dim3(RT), 0, st, in, x_res, w, eps, H, x_out, xn); break;
    default:
      set_error("resid_norm: row width %d above %d", H, 16 * RT);
      return hipErrorInvalidValue;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

// RoPE tables (src/kernels/rope.cu:15-18): angle p / theta^(2 d / 128) in
// double, cos and sin rounded to fp32; [S, 64] each.
__global__ __launch_bounds__(256) void rope_tables_kernel(int S, double theta, float* cosT,
                                                          float* sinT) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= S * 64) return;
  const int p = i >> 6, d = i & 63;
  const double ang = (double)p / pow(theta, 2.0 * d / 128.0);
  cosT[i] = (float)cos(ang);
  sinT[i] = (float)sin(ang);
}

hipError_t rope_tables(int S, double theta, float* cosT, float* sinT, hipStream_t st) {
  hipLaunchKernelGGL(rope_tables_kernel, dim3((S * 64 + 255) / 256), dim3(256), 0, st, S, theta,
                     cosT, sinT);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t head_norm_rope(const HeadRows* segs, int nseg, const float* cosT, const float* sinT,
                          int S, int T, float eps, hipStream_t st) {
  if (nseg < 1 || nseg > 2 || T <= 0 || S <= 0) {
    set_error("head_norm_rope: %d tensors, T=%d, S=%d", nseg, T, S);
    return hipErrorInvalidValue;
  }
  HeadNormArgs a{};
  long long maxrows = 0;
  for (int i = 0; i < nseg; ++i) {
    const HeadRows& r = segs[i];
    const bool al = (uintptr_t)r.w % 16 == 0 && (uintptr_t)r.x % 8 == 0 && (uintptr_t)r.out % 8 == 0;
    if (!r.x || !r.w || !r.out || r.nh <= 0 || !al) {
      set_error("head_norm_rope: tensor %d: bad pointers, alignment (w 16 B; x, out 8 B) or nh=%d",
                i, r.nh);
      return hipErrorInvalidValue;
    }
    if ((long long)T * r.nh >= (1LL << 31)) {
      set_error("head_norm_rope: %lld rows (at most 2^31 - 1)", (long long)T * r.nh);
      return hipErrorInvalidValue;
    }
    a.seg[i] = r;
    maxrows = std::max(maxrows, (long long)T * r.nh);
  }
  a.cosT = cosT;
  a.sinT = sinT;
  a.S = S;
  a.T = T;
  a.eps = eps;
  const dim3 grid((unsigned)((maxrows + HN_ROWS * HN_R - 1) / (HN_ROWS * HN_R)), nseg);
  hipLaunchKernelGGL(head_norm_rope_kernel, grid, dim3(RT), 0, st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t norm_bwd(const NormBwdArgs& a, int T, hipStream_t st) {
  if (!row_in_ok(a.in, a.H, "norm_bwd") || a.dh_col % 4) return hipErrorInvalidValue;
  const int P = (a.H + 4 * RT - 1) / (4 * RT);
  const bool lora = a.in.nterm > 0;
  // the MFMA form of the LoRA term: three full-width q/k/v terms, hidx and
  // adapter rows 16 q, one piece a thread (H <= 4 RT), [NR][H] fp32 of LDS
  NormBwdArgs am = a;
  if (am.lora_at) {
    bool ok = lora && am.in.nterm == 3 && a.H <= 4 * RT && a.H % 16 == 0;
    for (int q = 0; q < am.in.nterm && ok; ++q)
      ok = am.in.term[q].c0 == 0 && am.in.term[q].n == a.H && am.in.term[q].hidx == q * R;
    if (!ok) am.lora_at = nullptr;
  }
  // large T: the VALU LoRA form shares its adapter values over 8 rows; the
  // MFMA form runs 4 (128 VGPRs, two workgroups a CU: C4 50.7 -> 49.0 us
  // against 8 rows at 229 VGPRs; 2 rows 59 us)
  const int nr = rows_per_wg(T, P, lora ? (am.lora_at ? 4 : 8) : 2);
  const dim3 g((T + nr - 1) / nr);
  // the stashed x and the incoming residual gradient are read once: past
  // 32 MB a launch (C4: 33.5 MB each) nontemporal (C4 LoRA form 58.4 ->
  // 56.9 us, the plain form unchanged)
  const bool nt = (long long)T * a.H * 4 >= (32ll << 20);
  auto rows = [&](auto nr_, auto lora_) {
    constexpr int NR = decltype(nr_)::value;
    constexpr bool LO = decltype(lora_)::value;
    if (LO && am.lora_at) {
      if (nt)
        hipLaunchKernelGGL((norm_bwd_rows_kernel<NR, 2, true>), g, dim3(RT), 0, st, am, T);
      else
        hipLaunchKernelGGL((norm_bwd_rows_kernel<NR, 2, false>), g, dim3(RT), 0, st, am, T);
    } else if (nt) {
      hipLaunchKernelGGL((norm_bwd_rows_kernel<NR, LO ? 1 : 0, true>), g, dim3(RT), 0, st, am, T);
    } else {
      hipLaunchKernelGGL((norm_bwd_rows_kernel<NR, LO ? 1 : 0, false>), g, dim3(RT), 0, st, am, T);
    }
  };
  using std::integral_constant;
  using T1 = integral_constant<bool, true>;
  using F1 = integral_constant<bool, false>;
  switch (P * 100 + nr * 10 + (lora ? 1 : 0)) {
    case 110: case 111: hipLaunchKernelGGL(norm_bwd_kernel<1>, g, dim3(RT), 0, st, a); break;
    case 120: rows(integral_constant<int, 2>(), F1()); break;
    case 121: rows(integral_constant<int, 2>(), T1()); break;
    case 130: rows(integral_constant<int, 3>(), F1()); break;
    case 131: rows(integral_constant<int, 3>(), T1()); break;
    case 140: rows(integral_constant<int, 4>(), F1()); break;
    case 141: rows(integral_constant<int, 4>(), T1()); break;
    case 180: rows(integral_constant<int, 8>(), F1()); break;
    case 181: rows(integral_constant<int, 8>(), T1()); break;
    case 210: case 211: hipLaunchKernelGGL(norm_bwd_kernel<2>, g, dim3(RT), 0, st, a); break;
    case 310: case 311: hipLaunchKernelGGL(norm_bwd_kernel<3>, g, dim3(RT), 0, st, a); break;
    case 410: case 411: hipLaunchKernelGGL(norm_bwd_kernel<4>, g, dim3(RT), 0, st, a); break;
    default:
      set_error("norm_bwd: row width %d above %d", a.H, 16 * RT);
      return hipErrorInvalidValue;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t swiglu_bwd(const RowIn& in, const float* rinv_in, const _Float16* gu, int I, int T,
                      _Float16* dgu16, float* rinv_out, const _Float16* ks, hipStream_t st) {
  if (!row_in_ok(in, I, "swiglu_bwd", true)) return hipErrorInvalidValue;
  const int P = (I + 4 * RT - 1) / (4 * RT);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(T), dim3(RT), 0, st, in, rinv_in, gu, I, dgu16, rinv_out, ks);
  };
  const bool sc = in.split_col > 0;
  if (sc && in.split != 2) {
    set_error("swiglu_bwd: a split_col input has two partials (got %d)", in.split);
    return hipErrorInvalidValue;
  }
  // the gate/up stash of a layer is read once: past 64 MB (C4: 100 MB) the
  // loads go nontemporal, so it streams past the caches the next GEMM's
  // operand lands in (C4: 53.8 -> 50.8 us a layer in the step)
  const bool nt = (long long)T * I * 4 >= (64ll << 20);
  auto pick = [&](auto p, auto s) {
    constexpr int PP = decltype(p)::value;
    constexpr bool SS = decltype(s)::value;
    if (nt)
      go(swiglu_bwd_kernel<PP, SS, true>);
    else
      go(swiglu_bwd_kernel<PP, SS, false>);
  };
  using std::integral_constant;
  using T1 = integral_constant<bool, true>;
  using F1 = integral_constant<bool, false>;
  switch (P * 2 + (sc ? 1 : 0)) {
    case 2: pick(integral_constant<int, 1>(), F1()); break;
    case 3: pick(integral_constant<int, 1>(), T1()); break;
    case 4: pick(integral_constant<int, 2>(), F1()); break;
    case 5: pick(integral_constant<int, 2>(), T1()); break;
    case 6: pick(integral_constant<int, 3>(), F1()); break;
    case 7: pick(integral_constant<int, 3>(), T1()); break;
    case 8: pick(integral_constant<int, 4>(), F1()); break;
    case 9: pick(integral_constant<int, 4>(), T1()); break;
    default:
      set_error("swiglu_bwd: row width %d above %d", I, 16 * RT);
      return hipErrorInvalidValue;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t o_dx_post(const RowIn& in, const float* rinv_in, const _Float16* o16, int nq, int S,
                     int T, float* dh_out, _Float16* dO16, float* delta, float* dsc,
                     hipStream_t st) {
  const int Q = nq * HD;
  if (!row_in_ok(in, Q, "o_dx_post")) return hipErrorInvalidValue;
  if (in.nterm > 1 || (in.nterm == 1 && (in.term[0].c0 != 0 || in.term[0].n != Q ||
                                         in.term[0].hidx != 0 || in.nh != R))) {
    set_error("o_dx_post: one LoRA term over all %d columns with its 16 h columns", Q);
    return hipErrorInvalidValue;
  }
  // up to two split partials: tiled by head; more: one row per workgroup
  // (16-byte loads of each partial), measured faster at the headline shape
  if (in.split <= 2) {
    hipLaunchKernelGGL(o_dx_post_kernel, dim3(nq, (T + OD_ROWS - 1) / OD_ROWS), dim3(256), 0, st,
                       in, rinv_in, o16, nq, S, T, dh_out, dO16, delta, dsc);
  } else {
    switch ((Q + 4 * RT - 1) / (4 * RT)) {
      case 1: hipLaunchKernelGGL(o_dx_post_row_kernel<1>, dim3(T), dim3(RT), 0, st, in, rinv_in, o16, nq, S, dh_out, dO16, delta, dsc); break;
      case 2: hipLaunchKernelGGL(o_dx_post_row_kernel<2>, dim3(T), dim3(RT), 0, st, in, rinv_in, o16, nq, S, dh_out, dO16, delta, dsc); break;
      case 3: hipLaunchKernelGGL(o_dx_post_row_kernel<3>, dim3(T), dim3(RT), 0, st, in, rinv_in, o16, nq, S, dh_out, dO16, delta, dsc); break;
      case 4: hipLaunchKernelGGL(o_dx_post_row_kernel<4>, dim3(T), dim3(RT), 0, st, in, rinv_in, o16, nq, S, dh_out, dO16, delta, dsc); break;
      default:
        set_error("o_dx_post: row width %d above %d", Q, 16 * RT);
        return hipErrorInvalidValue;
    }
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t qk_bwd(const QkBwdArgs& a, int T, hipStream_t st) {
  const int NT = (a.nq + 2 * a.nkv) * HD;
  const int hpw = (a.nq + a.nkv + RW - 1) / RW;
  const size_t lds = NT * sizeof(float);
  const char* e = getenv("LLMT_QK_BWD_HOIST");
  const bool hoist = (!e || atoi(e) != 0) && hpw <= 4 && a.nkv * HD <= 2 * RT;
  auto go = [&](auto kern) { hipLaunchKernelGGL(kern, dim3(T), dim3(RT), lds, st, a); };
  switch (hoist ? hpw : 0) {
    case 1: go(qk_bwd_kernel<1>); break;
    case 2: go(qk_bwd_kernel<2>); break;
    case 3: go(qk_bwd_kernel<3>); break;
    case 4: go(qk_bwd_kernel<4>); break;
    default: go(qk_bwd_kernel<0>); break;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
