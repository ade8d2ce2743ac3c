// common.h — shared device/host helpers for the gfx950 kernels of libllmt.
#pragma once

#include <hip/hip_runtime.h>
#include <utility>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdio.h>

namespace llmt {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int8_t int8x8 __attribute__((ext_vector_type(8)));

// Error plumbing: every launcher returns hipError_t; the C ABI maps it to
// LLMT_ERR_HIP and records a message.
void set_error(const char* fmt, ...);

#define LLMT_HIP_TRY(expr)                                                     \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      ::llmt::set_error("%s:%d: %s: %s", __FILE__, __LINE__, #expr,            \
                        hipGetErrorString(e_));                                \
      return e_;                                                               \
    }                                                                          \
  } while (0)

#define LLMT_LAUNCH_CHECK() LLMT_HIP_TRY(hipGetLastError())

// fp16 MFMA 16x16x32, fp32 accumulate.  Operand k-order only has to agree
// between A and B: every GEMM here loads both with lane group g = lane/16
// holding k = 8g..8g+7 of the 32-wide step.  D: lane holds rows
// 4*(lane/16)+v (v = 0..3) of column lane%16.
__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Value of another lane of the same 16-lane row through a DPP modifier (a
// VALU operand, no LDS): quad_perm [1,0,3,2] (0xB1) and [2,3,0,1] (0x4E),
// row_half_mirror (0x141, lane i <- 7 - i within 8) and row_mirror (0x140,
// lane i <- 15 - i within 16).  After the two quad steps every lane of a
// quad holds the quad's result, so the two mirrors finish a reduction over
// the 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dpp16(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Lane L of each 16-lane row, broadcast to the whole row (gfx950's DPP
// row_newbcast:L, control 0x150 + L): a VALU operand, so a per-rank
// broadcast needs no v_readlane into an SGPR (and none of the wait states a
// VALU read of a VALU-written SGPR takes).
template <int L>
__device__ __forceinline__ float bcast16(float v) {
  static_assert(L >= 0 && L < 16, "lane within a row");
  // every lane has a source lane, so bound_ctrl changes nothing but lets
  // the compiler fold the move into the consumer as its DPP operand
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + L, 0xF, 0xF, true));
}
// f(std::integral_constant<int, i>) for i = 0 .. N - 1, unrolled.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, dpp16<0xB1>(v));
  v = fmaxf(v, dpp16<0x4E>(v));
  v = fmaxf(v, dpp16<0x141>(v));
  return fmaxf(v, dpp16<0x140>(v));
}
__device__ __forceinline__ float sum16_dpp(float v) {
  v += dpp16<0xB1>(v);
  v += dpp16<0x4E>(v);
  v += dpp16<0x141>(v);
  return v + dpp16<0x140>(v);
}

// Max / sum over the four lanes c, c + 16, c + 32, c + 48 (the 16-lane rows
// of a wave) with gfx950's lane-swap VALU instructions instead of LDS
// permutes: after v_permlane32_swap / v_permlane16_swap of a value with
// itself, lane i holds x[i] and x[i ^ 32] (x[i ^ 16]) in its two results, so
// one max or add finishes each step; every lane gets the same bits (min/max
// and a + b are symmetric).
__device__ __forceinline__ float xg_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xg_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Over the 32 lanes of a half wave (lanes 32 q .. 32 q + 31).
__device__ __forceinline__ float sum32(float x) {
  x = sum16_dpp(x);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max32(float x) {
  x = max16(x);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Over the whole wave; every lane gets the same bits.  All 64 lanes must be
// active (the reductions read their neighbours' registers).
__device__ __forceinline__ float wave_sum(float v) { return xg_sum(sum16_dpp(v)); }
__device__ __forceinline__ float wave_max(float v) { return xg_max(max16(v)); }

// Logistic sigmoid through the hardware reciprocal (v_rcp_f32, 1 ulp)
// rather than an IEEE division (about ten instructions); every use rounds the
// result into an fp16 operand.  x -> -inf gives rcp(inf) = 0, x -> +inf 1.
__device__ __forceinline__ float sigmoid_rcp(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// Online-softmax pairs (m, s = sum exp(x - m)): (m, s) <- the pair of the
// union with (m2, s2).  Empty pairs are (-inf, 0).
__device__ __forceinline__ void softmax_merge(float& m, float& s, float m2, float s2) {
  constexpr float kLog2e = 1.4426950408889634f;
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * __builtin_amdgcn_exp2f((m - mn) * kLog2e) + s2 * __builtin_amdgcn_exp2f((m2 - mn) * kLog2e);
  m = mn;
}

// The pair of NF values x[f] of one row held by each of the 16 lanes of a
// lane group (lanes 16 q .. 16 q + 15): every lane gets it.
template <int NF>
__device__ __forceinline__ float2 softmax_pair16(const float (&x)[NF]) {
  constexpr float kLog2e = 1.4426950408889634f;
  float m = -INFINITY;
#pragma unroll
  for (int f = 0; f < NF; ++f) m = fmaxf(m, x[f]);
  m = max16(m);
  float s = 0.f;
  if (m != -INFINITY) {
    const float m2 = m * kLog2e;
#pragma unroll
    for (int f = 0; f < NF; ++f) s += __builtin_amdgcn_exp2f(fmaf(x[f], kLog2e, -m2));
  }
  return make_float2(m, sum16_dpp(s));
}

// Block-wide reductions for blocks of NW waves; `red` is LDS of >= NW floats.
// Every thread gets the result.  Contains __syncthreads().
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  __syncthreads();
  return t;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) t = fmaxf(t, red[i]);
  __syncthreads();
  return t;
}

// Power-of-two scale that maps a row maximum |x| into [2^(E-1), 2^E): the
// fp16 operands carry it per row and their consumers divide it back out
// exactly.  GEMM operands use E = 14 (fp32 accumulation, no fp16 results);
// amax == 0 or non-finite gives scale 1.
__device__ __forceinline__ float pow2_scale_for(float amax, int E = 14) {
  if (!(amax > 0.f) || !isfinite(amax)) return 1.0f;
  int e;
  frexpf(amax, &e);  // amax = f * 2^e, f in [0.5, 1)
  return ldexpf(1.0f, E - e);
}

// The attention backward's fp16 dO rows: dS = P (dO V^T - delta), a sum of
// 128 products of a dO row with V, is itself rounded to fp16, so dO rows
// leave 2^5 of headroom under the GEMM operands' range.
constexpr int kDoScaleExp = 9;

// Inverse of a row scale as stored beside its scaled fp16 row (0 marks an
// all-zero row, which contributes nothing whatever its scale); the largest
// over a set of rows gives their common scale.
__device__ __forceinline__ float pow2_inv_scale_for(float amax, int E = 14) {
  return amax > 0.f ? 1.0f / pow2_scale_for(amax, E) : 0.f;
}

// Fragment-packed layout of a GEMM B operand [rows, K] (rows % 16 == 0,
// K % 32 == 0): 16-row x 32-k blocks of 512 elements, ordered by row block
// then k block; inside a block, lane l = 16 g + c of a wave holds row c,
// k = 8 g .. 8 g + 7 contiguously.  One MFMA B fragment is therefore one
// contiguous 1 KB (fp16) or 512 B (int8) load per wave.
__host__ __device__ __forceinline__ long long packed_index(long long r, long long k, long long K) {
  return (((r >> 4) * (K >> 5) + (k >> 5)) << 9) + ((((k >> 3) & 3) << 4) + (r & 15)) * 8 + (k & 7);
}

__device__ __forceinline__ float h2f(_Float16 h) { return (float)h; }
__device__ __forceinline__ _Float16 f2h(float f) { return (_Float16)f; }

}  // namespace llmt
