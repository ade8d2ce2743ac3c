// attn.hip — causal GQA flash attention (head_dim 128) on fp16 MFMA for
// gfx950: forward (keeps the fp32 log-sum-exp instead of P) and a
// deterministic backward (dK/dV per key block and query head, dQ per query
// block, both in one launch; the query heads of a GQA group are summed by
// the consumer in a fixed order), recomputing P from Q, K and the LSE.
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
// Tiles: a workgroup owns NW waves x 16 rows (queries, or keys for dK/dV)
// and iterates over 64-row tiles of the other side, staged through LDS; the
// next tile's global loads are issued before the current tile is computed.
// Rows and keys beyond S are zero-filled and masked, so any S works.
#include <stdlib.h>

#include <algorithm>

#include "ops.h"

namespace llmt {

namespace {

constexpr int HD = 128;
constexpr int BLK = 64;
constexpr int RP = HD + 8;   // LDS pitch (halves) of a [64][128] row-major tile
constexpr int TP = BLK + 8;  // LDS pitch (halves) of a [128][64] transposed tile
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// A 64 x 128 fp16 tile (rows r0.., row pitch ld, rows >= nrows zero) in
// registers: thread i of NT holds 16-byte pieces idx = i + NT j.
template <int NT>
struct Tile16 {
  half8 x[1024 / NT];
};

template <int NT>
__device__ __forceinline__ void load_tile(const _Float16* __restrict__ src, long long ld, int r0,
                                          int nrows, Tile16<NT>& t) {
#pragma unroll
  for (int i = 0; i < 1024 / NT; ++i) {
    const int idx = threadIdx.x + NT * i;
    const int row = idx >> 4, d0 = (idx & 15) * 8;
    // branch-free: clamped load, zeroed past the end (keeps every load in flight)
    const half8 x = *reinterpret_cast<const half8*>(src + (long long)min(r0 + row, nrows - 1) * ld + d0);
    t.x[i] = r0 + row < nrows ? x : half8{};
  }
}

// Same from fp32 with a scale (the attention dO operand).
template <int NT>
__device__ __forceinline__ void load_tile_f32(const float* __restrict__ src, long long ld, int r0,
                                              int nrows, float scale, Tile16<NT>& t) {
#pragma unroll
  for (int i = 0; i < 1024 / NT; ++i) {
    const int idx = threadIdx.x + NT * i;
    const int row = idx >> 4, d0 = (idx & 15) * 8;
    const float4* p =
        reinterpret_cast<const float4*>(src + (long long)min(r0 + row, nrows - 1) * ld + d0);
    const float4 a = p[0], b = p[1];
    half8 x;
    x[0] = (_Float16)(a.x * scale); x[1] = (_Float16)(a.y * scale);
    x[2] = (_Float16)(a.z * scale); x[3] = (_Float16)(a.w * scale);
    x[4] = (_Float16)(b.x * scale); x[5] = (_Float16)(b.y * scale);
    x[6] = (_Float16)(b.z * scale); x[7] = (_Float16)(b.w * scale);
    t.x[i] = r0 + row < nrows ? x : half8{};
  }
}

// Registers -> LDS: row-major copy `rm` (pitch RP) and/or transposed copy
// `tr` (pitch TP).
template <int NT>
__device__ __forceinline__ void store_tile(const Tile16<NT>& t, _Float16* rm, _Float16* tr) {
#pragma unroll
  for (int i = 0; i < 1024 / NT; ++i) {
    const int idx = threadIdx.x + NT * i;
    const int row = idx >> 4, d0 = (idx & 15) * 8;
    if (rm) *reinterpret_cast<half8*>(rm + row * RP + d0) = t.x[i];
    if (tr) {
#pragma unroll
      for (int e = 0; e < 8; ++e) tr[(d0 + e) * TP + row] = t.x[i][e];
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
  const half8 x =
      *reinterpret_cast<const half8*>(base + (long long)min(row, n - 1) * ld + ks * 32 + (lane >> 4) * 8);
  return row < n ? x : half8{};
}

__device__ __forceinline__ half8 frag_global_f32(const float* base, long long ld, int row, int n,
                                                 int ks, int lane, float scale) {
  const float4* p =
      reinterpret_cast<const float4*>(base + (long long)min(row, n - 1) * ld + ks * 32 + (lane >> 4) * 8);
  const float4 a = p[0], b = p[1];
  half8 r;
  r[0] = (_Float16)(a.x * scale); r[1] = (_Float16)(a.y * scale);
  r[2] = (_Float16)(a.z * scale); r[3] = (_Float16)(a.w * scale);
  r[4] = (_Float16)(b.x * scale); r[5] = (_Float16)(b.y * scale);
  r[6] = (_Float16)(b.z * scale); r[7] = (_Float16)(b.w * scale);
  return row < n ? r : half8{};
}

// Power-of-two scale for the fp16 dO operand of batch b: from the per-row
// max |dO| of the batch's S rows.  Identical in every workgroup of b.
template <int NT>
__device__ float batch_do_scale(const float* __restrict__ damax, int b, int S, float* red) {
  float m = 0.f;
  for (int s = threadIdx.x; s < S; s += NT) m = fmaxf(m, damax[(long long)b * S + s]);
  m = block_max<NT / 64>(m, red);
  return pow2_scale_for(m);
}

// ---------------------------------------------------------------- forward
// grid (ceil(S / (16 NW)), nq, B).  Wave w owns queries q0 + 16 w + c.
template <int NW>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const AttnArgs a) {
  constexpr int NT = NW * 64, QB = NW * 16;
  __shared__ __attribute__((aligned(16))) _Float16 Ks[BLK * RP];
  __shared__ __attribute__((aligned(16))) _Float16 VT[HD * TP];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int q = qb * QB + w * 16 + c;  // this lane's query (B-operand column)
  const float sl2 = a.sm_scale * LOG2E;

  const _Float16* kbase = a.k + rowb * a.ldk + kvh * HD;
  const _Float16* vbase = a.v + rowb * a.ldv + kvh * HD;
  const int nkb = min((qb * QB + QB - 1) / BLK, (S - 1) / BLK) + 1;
  Tile16<NT> tk, tv;
  load_tile<NT>(kbase, a.ldk, 0, S, tk);
  load_tile<NT>(vbase, a.ldv, 0, S, tv);
  half8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = frag_global(a.q + rowb * a.ldq + h * HD, a.ldq, q, S, ks, lane);

  floatx4 ot[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) ot[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
    store_tile<NT>(tk, Ks, nullptr);
    store_tile<NT>(tv, nullptr, VT);
    __syncthreads();
    if (kb + 1 < nkb) {
      load_tile<NT>(kbase, a.ldk, (kb + 1) * BLK, S, tk);
      load_tile<NT>(vbase, a.ldv, (kb + 1) * BLK, S, tv);
    }
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
// Workgroup (key block kb of 16 NW keys, query head h): wave w owns keys
// k0 + 16 w + c; loops over the 64-query tiles at or after the block.
// Writes this query head's share of dK, dV (fp32) to a.dkvp.
template <int NW>
__device__ void attn_dkdv(const AttnArgs& a, int kb, int h, int b, char* smem) {
  constexpr int NT = NW * 64, KB = NW * 16;
  _Float16* Qs = reinterpret_cast<_Float16*>(smem);
  _Float16* QT = Qs + BLK * RP;
  _Float16* Ds = QT + HD * TP;
  _Float16* DT = Ds + BLK * RP;
  float* lse_s = reinterpret_cast<float*>(DT + HD * TP);
  float* del_s = lse_s + BLK;
  float* red = del_s + BLK;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int key = kb * KB + w * 16 + c;
  const float sl2 = a.sm_scale * LOG2E;
  const float* lse_h = a.lse + ((long long)b * a.nq + h) * S;
  const float* del_h = a.delta + ((long long)b * a.nq + h) * S;
  const _Float16* qbase = a.q + rowb * a.ldq + h * HD;
  const float* dbase = a.dO + rowb * a.lddo + h * HD;
  const int qb0 = (kb * KB) / BLK;
  const int nqb = (S + BLK - 1) / BLK;
  const float gs = batch_do_scale<NT>(a.damax, b, S, red);

  Tile16<NT> tq, td;
  load_tile<NT>(qbase, a.ldq, qb0 * BLK, S, tq);
  load_tile_f32<NT>(dbase, a.lddo, qb0 * BLK, S, gs, td);
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
  for (int qb = qb0; qb < nqb; ++qb) {
    __syncthreads();
    store_tile<NT>(tq, Qs, QT);
    store_tile<NT>(td, Ds, DT);
    for (int i = threadIdx.x; i < BLK; i += NT) {
      const int qq = qb * BLK + i;
      lse_s[i] = qq < S ? lse_h[qq] * LOG2E : 0.f;
      del_s[i] = qq < S ? del_h[qq] * gs : 0.f;
    }
    __syncthreads();
    if (qb + 1 < nqb) {
      load_tile<NT>(qbase, a.ldq, (qb + 1) * BLK, S, tq);
      load_tile_f32<NT>(dbase, a.lddo, (qb + 1) * BLK, S, gs, td);
    }
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
  if (key < S) {
    const float inv = 1.0f / gs;
    const long long ldp = 2LL * a.nq * HD;
    float* dk = a.dkvp + (rowb + key) * ldp + h * HD;
    float* dv = a.dkvp + (rowb + key) * ldp + (a.nq + h) * HD;
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
// Workgroup (query block qb of 16 NW queries, head h): wave w owns queries
// q0 + 16 w + c.
template <int NW>
__device__ void attn_dq(const AttnArgs& a, int qb, int h, int b, char* smem) {
  constexpr int NT = NW * 64, QB = NW * 16;
  _Float16* Ks = reinterpret_cast<_Float16*>(smem);
  _Float16* Vs = Ks + BLK * RP;
  _Float16* KT = Vs + BLK * RP;
  float* red = reinterpret_cast<float*>(KT + HD * TP);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int q = qb * QB + w * 16 + c;
  const float sl2 = a.sm_scale * LOG2E;
  const _Float16* kbase = a.k + rowb * a.ldk + kvh * HD;
  const _Float16* vbase = a.v + rowb * a.ldv + kvh * HD;
  const int nkb = min((qb * QB + QB - 1) / BLK, (S - 1) / BLK) + 1;
  Tile16<NT> tk, tv;
  load_tile<NT>(kbase, a.ldk, 0, S, tk);
  load_tile<NT>(vbase, a.ldv, 0, S, tv);
  const float gs = batch_do_scale<NT>(a.damax, b, S, red);

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

  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();
    store_tile<NT>(tk, Ks, KT);
    store_tile<NT>(tv, Vs, nullptr);
    __syncthreads();
    if (kb + 1 < nkb) {
      load_tile<NT>(kbase, a.ldk, (kb + 1) * BLK, S, tk);
      load_tile<NT>(vbase, a.ldv, (kb + 1) * BLK, S, tv);
    }
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

constexpr size_t kDkdvLds = (size_t)(2 * BLK * RP + 2 * HD * TP) * 2 + (2 * BLK + 16) * 4;
constexpr size_t kDqLds = (size_t)(2 * BLK * RP + HD * TP) * 2 + 16 * 4;

// One launch for both backward halves: blockIdx.x < nkb_blocks are dK/dV
// workgroups (key block, query head), the rest dQ workgroups.
template <int NW>
__global__ __launch_bounds__(NW * 64) void attn_bwd_kernel(const AttnArgs a, int n_kv_blocks) {
  __shared__ __attribute__((aligned(16))) char smem[kDkdvLds > kDqLds ? kDkdvLds : kDqLds];
  const int h = blockIdx.y, b = blockIdx.z;
  if ((int)blockIdx.x < n_kv_blocks)
    attn_dkdv<NW>(a, blockIdx.x, h, b, smem);
  else
    attn_dq<NW>(a, blockIdx.x - n_kv_blocks, h, b, smem);
}

// dK, dV = sum over the query heads of each group of the per-head shares
// (group order, deterministic).
__global__ __launch_bounds__(256) void gqa_sum_kernel(const float* __restrict__ dkvp, int nq,
                                                      int nkv, long long n, float* __restrict__ dk,
                                                      float* __restrict__ dv, long long ldg) {
  const int group = nq / nkv;
  const int KV = nkv * HD;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    const long long t = i / KV;
    const int c = (int)(i - t * KV);
    const int j = c / HD, d = c - j * HD;
    const float* row = dkvp + t * 2LL * nq * HD;
    float sk = 0.f, sv = 0.f;
    for (int gi = 0; gi < group; ++gi) {
      sk += row[(j * group + gi) * HD + d];
      sv += row[(nq + j * group + gi) * HD + d];
    }
    dk[t * ldg + c] = sk;
    dv[t * ldg + c] = sv;
  }
}

// Per token row: delta[b, h, s] = sum_d dO[t, h, d] * O[t, h, d] (one wave
// per head) and damax[t] = max |dO[t, :]|.
__global__ __launch_bounds__(256) void attn_delta_kernel(const float* __restrict__ dO, long long ldd,
                                                         const _Float16* __restrict__ o,
                                                         long long ldo, int nq, int S,
                                                         float* __restrict__ delta,
                                                         float* __restrict__ damax) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = t / S, s = t - b * S;
  float amax = 0.f;
  for (int h = w; h < nq; h += 4) {
    const float* d = dO + (long long)t * ldd + h * HD;
    const _Float16* oo = o + (long long)t * ldo + h * HD;
    const float d0 = d[lane], d1 = d[lane + 64];
    amax = fmaxf(amax, fmaxf(fabsf(d0), fabsf(d1)));
    const float v = wave_sum(d0 * (float)oo[lane] + d1 * (float)oo[lane + 64]);
    if (lane == 0) delta[((long long)b * nq + h) * S + s] = v;
  }
  amax = block_max<4>(amax, red);
  if (threadIdx.x == 0) damax[t] = amax;
}

// Waves per workgroup (16 query or key rows each).  Four measured fastest on
// MI355X at S = 128 as well as at S = 2048 (fewer, longer workgroups beat more
// single-wave ones); LLMT_ATTN_FWD_WAVES / LLMT_ATTN_BWD_WAVES = 1, 2 or 4
// override it for tuning.
int attn_waves(const char* env) {
  const char* e = getenv(env);
  if (e && (e[0] == '1' || e[0] == '2' || e[0] == '4') && !e[1]) return e[0] - '0';
  return 4;
}

}  // namespace

hipError_t attn_delta(const float* dO, long long ldd, const _Float16* o, long long ldo, int nq,
                      int S, int T, float* delta, float* damax, hipStream_t st) {
  hipLaunchKernelGGL(attn_delta_kernel, dim3(T), dim3(256), 0, st, dO, ldd, o, ldo, nq, S, delta,
                     damax);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

template <int NW>
static void launch_fwd(const AttnArgs& a, int B, hipStream_t st) {
  dim3 grid((a.S + NW * 16 - 1) / (NW * 16), a.nq, B);
  hipLaunchKernelGGL(attn_fwd_kernel<NW>, grid, dim3(NW * 64), 0, st, a);
}

template <int NW>
static void launch_bwd(const AttnArgs& a, int B, hipStream_t st) {
  const int nkvb = (a.S + NW * 16 - 1) / (NW * 16);
  dim3 grid(2 * nkvb, a.nq, B);
  hipLaunchKernelGGL(attn_bwd_kernel<NW>, grid, dim3(NW * 64), 0, st, a, nkvb);
}

hipError_t attn_fwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0) {
    set_error("attn_fwd: nq=%d nkv=%d S=%d", a.nq, a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  switch (attn_waves("LLMT_ATTN_FWD_WAVES")) {
    case 1: launch_fwd<1>(a, B, st); break;
    case 2: launch_fwd<2>(a, B, st); break;
    default: launch_fwd<4>(a, B, st); break;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t attn_bwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0 || !a.dkvp) {
    set_error("attn_bwd: nq=%d nkv=%d S=%d (dK/dV share buffer required)", a.nq, a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  switch (attn_waves("LLMT_ATTN_BWD_WAVES")) {
    case 1: launch_bwd<1>(a, B, st); break;
    case 2: launch_bwd<2>(a, B, st); break;
    default: launch_bwd<4>(a, B, st); break;
  }
  LLMT_LAUNCH_CHECK();
  if (a.dk && a.dv) {
    const long long n = (long long)B * a.S * a.nkv * HD;
    const long long g = std::min<long long>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(gqa_sum_kernel, dim3((unsigned)g), dim3(256), 0, st, a.dkvp, a.nq, a.nkv, n,
                       a.dk, a.dv, a.ldgkv);
    LLMT_LAUNCH_CHECK();
  }
  return hipSuccess;
}

}  // namespace llmt
