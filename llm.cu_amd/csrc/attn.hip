// attn.hip — causal GQA flash attention (head_dim 128) on fp16 MFMA for
// gfx950: forward (keeps the fp32 log-sum-exp instead of P) and a
// deterministic two-kernel backward (dK/dV per key block with both query
// heads of the GQA group in one workgroup; dQ per query block), recomputing
// P from Q, K and the LSE.
//
// Replaces the reference's naive_attn_kernel (src/kernels/lora_forward.cu:
// 48-135, which stores P [heads, S, S] in fp32), attn_backward_kernel
// (src/kernels/lora_backward.cu:104-186, float atomics) and the expand /
// contract GQA copies (:189-208).  Math: s = q k^T / sqrt(128), causal,
// P = softmax(s); dP = dO V^T; dS = P (dP - delta), delta = rowsum(dO * O);
// dQ = dS K / sqrt(128); dK = dS^T Q / sqrt(128); dV = P^T dO.  Query head h
// reads KV head h / (nq / nkv) (include/config.h:15).
//
// MFMA conventions (v_mfma_f32_16x16x32_f16, c = lane % 16, g = lane / 16):
// an A fragment holds A[c][k-slot (g, i)], a B fragment B[k-slot (g, i)][c],
// the accumulator D[4 g + v][c].  An accumulator is reused as the B operand
// of the next product by pairing two 16-row tiles: k-slot (g, i) <-> row
// 4 g + i of tile 2j (i < 4) or of tile 2j + 1 (i >= 4); the A operand then
// reads the same row order from a transposed LDS copy.  Any fixed slot
// permutation is valid as long as A and B agree.
//
// Tiles: 64 queries x 64 keys per iteration, 4 waves x 16 rows.  Rows and
// keys beyond S are zero-filled and masked, so any S works.
#include "ops.h"

namespace llmt {

namespace {

constexpr int HD = 128;
constexpr int BLK = 64;
constexpr int NTH = 256;
constexpr int RP = HD + 8;   // LDS pitch (halves) of a [64][128] row-major tile
constexpr int TP = BLK + 8;  // LDS pitch (halves) of a [128][64] transposed tile
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// Stage rows [r0, r0 + 64) x 128 of a row-major fp16 matrix (row pitch ld) into
// LDS: row-major copy `rm` (pitch RP) and/or transposed copy `tr` (pitch TP).
// Rows >= nrows are zero.
__device__ __forceinline__ void stage_f16(const _Float16* __restrict__ src, long long ld, int r0,
                                          int nrows, _Float16* rm, _Float16* tr) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = threadIdx.x + NTH * i;
    const int row = idx >> 4, d0 = (idx & 15) * 8;
    half8 x = {};
    if (r0 + row < nrows) x = *reinterpret_cast<const half8*>(src + (long long)(r0 + row) * ld + d0);
    if (rm) *reinterpret_cast<half8*>(rm + row * RP + d0) = x;
    if (tr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) tr[(d0 + e) * TP + row] = x[e];
    }
  }
}

// Same from fp32 with a scale (the attention dO operand).
__device__ __forceinline__ void stage_f32(const float* __restrict__ src, long long ld, int r0,
                                          int nrows, float scale, _Float16* rm, _Float16* tr) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = threadIdx.x + NTH * i;
    const int row = idx >> 4, d0 = (idx & 15) * 8;
    half8 x = {};
    if (r0 + row < nrows) {
      const float4* p = reinterpret_cast<const float4*>(src + (long long)(r0 + row) * ld + d0);
      const float4 a = p[0], b = p[1];
      x[0] = (_Float16)(a.x * scale); x[1] = (_Float16)(a.y * scale);
      x[2] = (_Float16)(a.z * scale); x[3] = (_Float16)(a.w * scale);
      x[4] = (_Float16)(b.x * scale); x[5] = (_Float16)(b.y * scale);
      x[6] = (_Float16)(b.z * scale); x[7] = (_Float16)(b.w * scale);
    }
    if (rm) *reinterpret_cast<half8*>(rm + row * RP + d0) = x;
    if (tr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) tr[(d0 + e) * TP + row] = x[e];
    }
  }
}

// A fragment from a row-major LDS tile: rows m0 + c, k = 32 ks + 8 g + i.
__device__ __forceinline__ half8 frag_rm(const _Float16* t, int m0, int ks, int lane) {
  return *reinterpret_cast<const half8*>(t + (m0 + (lane & 15)) * RP + ks * 32 + (lane >> 4) * 8);
}

// A fragment from a transposed LDS tile [d][row] for the paired-accumulator
// k-slot order: rows d0 + c, k-slots (g, i) -> row 32 j + 4 g + i (i < 4),
// 32 j + 16 + 4 g + i - 4 (i >= 4).
__device__ __forceinline__ half8 frag_tr(const _Float16* t, int d0, int j, int lane) {
  const _Float16* p = t + (d0 + (lane & 15)) * TP + 32 * j + 4 * (lane >> 4);
  const half4v lo = *reinterpret_cast<const half4v*>(p);
  const half4v hi = *reinterpret_cast<const half4v*>(p + 16);
  half8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// B fragment built from two accumulator tiles (see the file comment).
__device__ __forceinline__ half8 pair_frag(const floatx4& a, const floatx4& b) {
  half8 r;
  r[0] = (_Float16)a[0]; r[1] = (_Float16)a[1]; r[2] = (_Float16)a[2]; r[3] = (_Float16)a[3];
  r[4] = (_Float16)b[0]; r[5] = (_Float16)b[1]; r[6] = (_Float16)b[2]; r[7] = (_Float16)b[3];
  return r;
}

// Operand fragment straight from global memory: row `row` (zero if >= n),
// k = 32 ks + 8 g .. + 7.
__device__ __forceinline__ half8 frag_global(const _Float16* base, long long ld, int row, int n,
                                             int ks, int lane) {
  if (row >= n) return half8{};
  return *reinterpret_cast<const half8*>(base + (long long)row * ld + ks * 32 + (lane >> 4) * 8);
}

__device__ __forceinline__ half8 frag_global_f32(const float* base, long long ld, int row, int n,
                                                 int ks, int lane, float scale) {
  half8 r = {};
  if (row >= n) return r;
  const float4* p = reinterpret_cast<const float4*>(base + (long long)row * ld + ks * 32 + (lane >> 4) * 8);
  const float4 a = p[0], b = p[1];
  r[0] = (_Float16)(a.x * scale); r[1] = (_Float16)(a.y * scale);
  r[2] = (_Float16)(a.z * scale); r[3] = (_Float16)(a.w * scale);
  r[4] = (_Float16)(b.x * scale); r[5] = (_Float16)(b.y * scale);
  r[6] = (_Float16)(b.z * scale); r[7] = (_Float16)(b.w * scale);
  return r;
}

// Power-of-two scale for the fp16 dO operand of batch b: from the per-row
// max |dO| of the batch's S rows.  Identical in every workgroup of b.
__device__ float batch_do_scale(const float* __restrict__ damax, int b, int S, float* red) {
  float m = 0.f;
  for (int s = threadIdx.x; s < S; s += NTH) m = fmaxf(m, damax[(long long)b * S + s]);
  m = block_max<NTH / 64>(m, red);
  return pow2_scale_for(m);
}

// ---------------------------------------------------------------- forward
// grid (ceil(S/64), nq, B).  Wave w owns queries q0 + 16 w + c.
__global__ __launch_bounds__(NTH) void attn_fwd_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 Ks[BLK * RP];
  __shared__ __attribute__((aligned(16))) _Float16 VT[HD * TP];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int q = qb * BLK + w * 16 + c;  // this lane's query (B-operand column)
  const float sl2 = a.sm_scale * LOG2E;

  half8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = frag_global(a.q + rowb * a.ldq + h * HD, a.ldq, q, S, ks, lane);

  floatx4 ot[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ot[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  const _Float16* kbase = a.k + rowb * a.ldk + kvh * HD;
  const _Float16* vbase = a.v + rowb * a.ldv + kvh * HD;
  const int nkb = min(qb, (S - 1) / BLK) + 1;
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
    stage_f16(kbase, a.ldk, kb * BLK, S, Ks, nullptr);
    stage_f16(vbase, a.ldv, kb * BLK, S, nullptr, VT);
    __syncthreads();
    floatx4 st[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      st[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) st[mt] = mfma16(frag_rm(Ks, mt * 16, ks, lane), qf[ks], st[mt]);
    }
    float bm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int key = kb * BLK + mt * 16 + 4 * g + v;
        const float s = (key <= q && key < S) ? st[mt][v] * sl2 : -INFINITY;
        st[mt][v] = s;
        bm = fmaxf(bm, s);
      }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = exp2f(m - mu);
    m = mn;
    float ps = 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = exp2f(st[mt][v] - mu);
        st[mt][v] = p;
        ps += p;
      }
    l = l * alpha + ps;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) ot[dt] *= alpha;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const half8 pb = pair_frag(st[2 * j], st[2 * j + 1]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) ot[dt] = mfma16(frag_tr(VT, dt * 16, j, lane), pb, ot[dt]);
    }
  }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (q < S) {
    const float inv = 1.0f / l;
    _Float16* o = a.o + (rowb + q) * a.ldo + h * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      half4v r;
#pragma unroll
      for (int v = 0; v < 4; ++v) r[v] = (_Float16)(ot[dt][v] * inv);
      *reinterpret_cast<half4v*>(o + dt * 16 + 4 * g) = r;
    }
    if (g == 0) a.lse[((long long)b * a.nq + h) * S + q] = (m + __log2f(l)) * LN2;
  }
}

// ---------------------------------------------------------------- dK, dV
// grid (ceil(S/64), nkv, B).  Wave w owns keys k0 + 16 w + c.
__global__ __launch_bounds__(NTH) void attn_bwd_dkdv_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 Qs[BLK * RP];
  __shared__ __attribute__((aligned(16))) _Float16 QT[HD * TP];
  __shared__ __attribute__((aligned(16))) _Float16 Ds[BLK * RP];
  __shared__ __attribute__((aligned(16))) _Float16 DT[HD * TP];
  __shared__ float lse_s[BLK], del_s[BLK];
  __shared__ float red[NTH / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int kb = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int group = a.nq / a.nkv;
  const long long rowb = (long long)b * S;
  const int key = kb * BLK + w * 16 + c;
  const float sl2 = a.sm_scale * LOG2E;
  const float gs = batch_do_scale(a.damax, b, S, red);

  half8 kf[4], vf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    kf[ks] = frag_global(a.k + rowb * a.ldk + kvh * HD, a.ldk, key, S, ks, lane);
    vf[ks] = frag_global(a.v + rowb * a.ldv + kvh * HD, a.ldv, key, S, ks, lane);
  }
  floatx4 dkT[8], dvT[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dkT[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    dvT[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  const int nqb = (S + BLK - 1) / BLK;
  for (int gi = 0; gi < group; ++gi) {
    const int h = kvh * group + gi;
    const float* lse_h = a.lse + ((long long)b * a.nq + h) * S;
    const float* del_h = a.delta + ((long long)b * a.nq + h) * S;
    for (int qb = kb; qb < nqb; ++qb) {
      __syncthreads();
      stage_f16(a.q + rowb * a.ldq + h * HD, a.ldq, qb * BLK, S, Qs, QT);
      stage_f32(a.dO + rowb * a.lddo + h * HD, a.lddo, qb * BLK, S, gs, Ds, DT);
      if (threadIdx.x < BLK) {
        const int qq = qb * BLK + threadIdx.x;
        lse_s[threadIdx.x] = qq < S ? lse_h[qq] * LOG2E : 0.f;
        del_s[threadIdx.x] = qq < S ? del_h[qq] * gs : 0.f;
      }
      __syncthreads();
      floatx4 p[4], ds[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        p[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
        ds[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          p[mt] = mfma16(frag_rm(Qs, mt * 16, ks, lane), kf[ks], p[mt]);
          ds[mt] = mfma16(frag_rm(Ds, mt * 16, ks, lane), vf[ks], ds[mt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int ql = mt * 16 + 4 * g + v;
          const int qq = qb * BLK + ql;
          const bool ok = key <= qq && qq < S && key < S;
          const float pv = ok ? exp2f(p[mt][v] * sl2 - lse_s[ql]) : 0.f;
          p[mt][v] = pv;
          ds[mt][v] = pv * (ds[mt][v] - del_s[ql]);
        }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const half8 pb = pair_frag(p[2 * j], p[2 * j + 1]);
        const half8 db = pair_frag(ds[2 * j], ds[2 * j + 1]);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          dvT[dt] = mfma16(frag_tr(DT, dt * 16, j, lane), pb, dvT[dt]);
          dkT[dt] = mfma16(frag_tr(QT, dt * 16, j, lane), db, dkT[dt]);
        }
      }
    }
  }
  if (key < S) {
    const float inv = 1.0f / gs;
    float* dk = a.dk + (rowb + key) * a.ldgkv + kvh * HD;
    float* dv = a.dv + (rowb + key) * a.ldgkv + kvh * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      *reinterpret_cast<float4*>(dk + dt * 16 + 4 * g) =
          make_float4(dkT[dt][0] * a.sm_scale * inv, dkT[dt][1] * a.sm_scale * inv,
                      dkT[dt][2] * a.sm_scale * inv, dkT[dt][3] * a.sm_scale * inv);
      *reinterpret_cast<float4*>(dv + dt * 16 + 4 * g) =
          make_float4(dvT[dt][0] * inv, dvT[dt][1] * inv, dvT[dt][2] * inv, dvT[dt][3] * inv);
    }
  }
}

// ---------------------------------------------------------------- dQ
// grid (ceil(S/64), nq, B).  Wave w owns queries q0 + 16 w + c.
__global__ __launch_bounds__(NTH) void attn_bwd_dq_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) _Float16 Ks[BLK * RP];
  __shared__ __attribute__((aligned(16))) _Float16 Vs[BLK * RP];
  __shared__ __attribute__((aligned(16))) _Float16 KT[HD * TP];
  __shared__ float red[NTH / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int q = qb * BLK + w * 16 + c;
  const float sl2 = a.sm_scale * LOG2E;
  const float gs = batch_do_scale(a.damax, b, S, red);

  half8 qf[4], df[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    qf[ks] = frag_global(a.q + rowb * a.ldq + h * HD, a.ldq, q, S, ks, lane);
    df[ks] = frag_global_f32(a.dO + rowb * a.lddo + h * HD, a.lddo, q, S, ks, lane, gs);
  }
  const bool qok = q < S;
  const float lse2 = qok ? a.lse[((long long)b * a.nq + h) * S + q] * LOG2E : 0.f;
  const float del = qok ? a.delta[((long long)b * a.nq + h) * S + q] * gs : 0.f;
  floatx4 dqT[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) dqT[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  const _Float16* kbase = a.k + rowb * a.ldk + kvh * HD;
  const _Float16* vbase = a.v + rowb * a.ldv + kvh * HD;
  const int nkb = min(qb, (S - 1) / BLK) + 1;
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
    stage_f16(kbase, a.ldk, kb * BLK, S, Ks, KT);
    stage_f16(vbase, a.ldv, kb * BLK, S, Vs, nullptr);
    __syncthreads();
    floatx4 pt[4], dt_[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      pt[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      dt_[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        pt[mt] = mfma16(frag_rm(Ks, mt * 16, ks, lane), qf[ks], pt[mt]);
        dt_[mt] = mfma16(frag_rm(Vs, mt * 16, ks, lane), df[ks], dt_[mt]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int key = kb * BLK + mt * 16 + 4 * g + v;
        const bool ok = key <= q && key < S && qok;
        const float pv = ok ? exp2f(pt[mt][v] * sl2 - lse2) : 0.f;
        dt_[mt][v] = pv * (dt_[mt][v] - del);
      }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const half8 db = pair_frag(dt_[2 * j], dt_[2 * j + 1]);
#pragma unroll
      for (int d = 0; d < 8; ++d) dqT[d] = mfma16(frag_tr(KT, d * 16, j, lane), db, dqT[d]);
    }
  }
  if (qok) {
    const float f = a.sm_scale / gs;
    float* dq = a.dq + (rowb + q) * a.ldgq + h * HD;
#pragma unroll
    for (int d = 0; d < 8; ++d)
      *reinterpret_cast<float4*>(dq + d * 16 + 4 * g) =
          make_float4(dqT[d][0] * f, dqT[d][1] * f, dqT[d][2] * f, dqT[d][3] * f);
  }
}

// Per token row: delta[b, h, s] = sum_d dO[t, h, d] * O[t, h, d] (one wave
// per head) and damax[t] = max |dO[t, :]|.
__global__ __launch_bounds__(NTH) void attn_delta_kernel(const float* __restrict__ dO, long long ldd,
                                                         const _Float16* __restrict__ o,
                                                         long long ldo, int nq, int S,
                                                         float* __restrict__ delta,
                                                         float* __restrict__ damax) {
  __shared__ float red[NTH / 64];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = t / S, s = t - b * S;
  float amax = 0.f;
  for (int h = w; h < nq; h += NTH / 64) {
    const float* d = dO + (long long)t * ldd + h * HD;
    const _Float16* oo = o + (long long)t * ldo + h * HD;
    const float d0 = d[lane], d1 = d[lane + 64];
    amax = fmaxf(amax, fmaxf(fabsf(d0), fabsf(d1)));
    const float v = wave_sum(d0 * (float)oo[lane] + d1 * (float)oo[lane + 64]);
    if (lane == 0) delta[((long long)b * nq + h) * S + s] = v;
  }
  amax = block_max<NTH / 64>(amax, red);
  if (threadIdx.x == 0) damax[t] = amax;
}

}  // namespace

hipError_t attn_delta(const float* dO, long long ldd, const _Float16* o, long long ldo, int nq,
                      int S, int T, float* delta, float* damax, hipStream_t st) {
  hipLaunchKernelGGL(attn_delta_kernel, dim3(T), dim3(NTH), 0, st, dO, ldd, o, ldo, nq, S, delta,
                     damax);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t attn_fwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0) {
    set_error("attn_fwd: nq=%d nkv=%d S=%d", a.nq, a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  dim3 grid((a.S + BLK - 1) / BLK, a.nq, B);
  hipLaunchKernelGGL(attn_fwd_kernel, grid, dim3(NTH), 0, st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t attn_bwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0) {
    set_error("attn_bwd: nq=%d nkv=%d S=%d", a.nq, a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  dim3 g1((a.S + BLK - 1) / BLK, a.nkv, B);
  hipLaunchKernelGGL(attn_bwd_dkdv_kernel, g1, dim3(NTH), 0, st, a);
  LLMT_LAUNCH_CHECK();
  dim3 g2((a.S + BLK - 1) / BLK, a.nq, B);
  hipLaunchKernelGGL(attn_bwd_dq_kernel, g2, dim3(NTH), 0, st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
