// attn.hip — causal GQA flash attention forward (head_dim 128) on fp16 MFMA
// for gfx950, keeping per query only the fp32 log-sum-exp of the scaled
// scores (the backward, attn_bwd.hip, recomputes P from Q, K and the LSE),
// and the preparation of a standalone backward's dO operand (attn_delta).
//
// Replaces the reference's naive_attn_kernel (src/kernels/lora_forward.cu:
// 48-135, which stores P [heads, S, S] in fp32) and its GQA expand copies
// (:138-147).  Math: s = q k^T / sqrt(128), causal, P = softmax(s), O = P V.
// Query head h reads KV head h / (nq / nkv) (include/config.h:15).
//
// The shared tile layout, DMA and fragment conventions are in attn_common.h.
// Causality and the sequence end are masked in the diagonal / last tiles
// only, chosen per wave with scalar branches.
#include <algorithm>

#include "attn_common.h"

namespace llmt {

namespace {

#define LLMT_INLINE __attribute__((always_inline))

// ---------------------------------------------------------------- forward
// One 64-key tile of the online softmax for RW 16-query tiles of a wave:
// st holds the raw scores (rows key, column query); on return the fp32
// probabilities relative to the running max, with m, l and the output
// accumulators rescaled.  MASK: apply causality / sequence end.
template <int RW, bool MASK>
__device__ __forceinline__ void softmax_tile(floatx4 (&st)[RW][4], float (&m)[RW], float (&l)[RW],
                                             floatx4 (&ot)[RW][8], float sl2, int key0, int q0,
                                             int S, int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int q = q0 + 16 * r + c;
    float bm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float s = st[r][mt][v];
        if (MASK) {
          const int key = key0 + mt * 16 + 4 * g + v;
          s = (key <= q && key < S) ? s : -INFINITY;
          st[r][mt][v] = s;
        }
        bm = fmaxf(bm, s);
      }
    bm = xg_max(bm);
    const float mn = fmaxf(m[r], bm * sl2);  // sl2 > 0: max commutes with the scale
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m[r] - mu);
    m[r] = mn;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) st[r][mt][v] = __builtin_amdgcn_exp2f(fmaf(st[r][mt][v], sl2, -mu));
    // row sum as a tree (independent adds) rather than one serial chain
    float ps4[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) ps4[mt] = (st[r][mt][0] + st[r][mt][1]) + (st[r][mt][2] + st[r][mt][3]);
    l[r] = l[r] * alpha + ((ps4[0] + ps4[1]) + (ps4[2] + ps4[3]));
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) ot[r][dt] *= alpha;
  }
}

// grid (nq, B, ceil(S / QB)), QB = 16 NW RW queries: blockIdx.z runs the
// longest (last) query blocks first over all heads and batches (workgroups
// are dispatched x fastest), and a workgroup's XCD (its linear index mod 8)
// follows its head, so every XCD gets the same mix of causal block lengths.
// (With the query block on x, XCD k got only blocks k, k + 8, ..: at B4 x
// S2048 the XCDs' work differed by 2.4x.)  Wave w owns queries q0 + 16 r + c
// (r < RW).  LDS: two buffers of (K tile, V tile).
template <int NW, int RW>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const AttnArgs a) {
  constexpr int QB = NW * RW * 16;
  // two LDS buffers of (K tile, V tile) as separate arrays, the tile loop
  // unrolled by two: which buffer a read or a DMA targets is then static, so
  // the reads of tile kb are not made to wait for the DMA of tile kb + 1
  __shared__ __attribute__((aligned(1024))) _Float16 buf0[2 * TILE];
  __shared__ __attribute__((aligned(1024))) _Float16 buf1[2 * TILE];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int qb = gridDim.z - 1 - blockIdx.z, h = blockIdx.x, b = blockIdx.y;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int q0 = qb * QB + w * RW * 16;
  const int qlast = min(q0 + RW * 16, S) - 1;  // last valid query of the wave
  const float sl2 = a.sm_scale * LOG2E;

  const _Float16* kbase = a.k + rowb * a.ldk + kvh * HD;
  const _Float16* vbase = a.v + rowb * a.ldv + kvh * HD;
  const int nkb = min((qb * QB + QB - 1) / BLK, (S - 1) / BLK) + 1;
  TileDma<NW> dk, dv;
  dk.init(a.ldk, w);
  dv.init(a.ldv, w);
  dk.issue(kbase, a.ldk, 0, S, buf0, w);
  dv.issue(vbase, a.ldv, 0, S, buf0 + TILE, w);
  half8 qf[RW][4];
  if (a.qn) {  // the block API: QK-norm + RoPE of the raw q here, q16w for the backward
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int q = q0 + 16 * r + c, qc = min(q, S - 1);
      norm_rope_frag(qf[r], a.qraw + (rowb + qc) * a.ldqr + h * HD, a.qn, a.cosT, a.sinT, qc,
                     a.eps, g);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (q < S)
          *reinterpret_cast<half8*>(a.q16w + (rowb + q) * a.ldq + h * HD + 32 * ks + 8 * g) =
              qf[r][ks];
        else
          qf[r][ks] = half8{};
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        qf[r][ks] = frag_global(a.q + rowb * a.ldq + h * HD, a.ldq, q0 + 16 * r + c, S, ks, lane);
  }

  floatx4 ot[RW][8];
  float m[RW], l[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ot[r][i] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  auto tile = [&](int kb, const _Float16* Ks, _Float16* nb) LLMT_INLINE {
    wait_vm<0>();
    tile_barrier();
    if (kb + 1 < nkb) {
      dk.issue(kbase, a.ldk, (kb + 1) * BLK, S, nb, w);
      dv.issue(vbase, a.ldv, (kb + 1) * BLK, S, nb + TILE, w);
    }
    if (kb * BLK > qlast) return;  // every key after every query of the wave
    const _Float16* Vs = Ks + TILE;
    floatx4 st[RW][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int r = 0; r < RW; ++r) st[r][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const half8 kf = frag_rm(Ks, mt * 16, ks, lane);
#pragma unroll
        for (int r = 0; r < RW; ++r) st[r][mt] = mfma16(kf, qf[r][ks], st[r][mt]);
      }
    }
    // keys of the tile all <= every query of the wave and < S: no mask
    if (kb * BLK + BLK - 1 <= q0 && kb * BLK + BLK <= S)
      softmax_tile<RW, false>(st, m, l, ot, sl2, kb * BLK, q0, S, lane);
    else
      softmax_tile<RW, true>(st, m, l, ot, sl2, kb * BLK, q0, S, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      half8 pb[RW];
#pragma unroll
      for (int r = 0; r < RW; ++r) pb[r] = pair_frag(st[r][2 * j], st[r][2 * j + 1]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const half8 vf = frag_tr(Vs, dt * 16, j, lane);
#pragma unroll
        for (int r = 0; r < RW; ++r) ot[r][dt] = mfma16(vf, pb[r], ot[r][dt]);
      }
    }
  };
  for (int kb = 0; kb < nkb; kb += 2) {
    tile(kb, buf0, buf1);
    if (kb + 1 < nkb) tile(kb + 1, buf1, buf0);
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    float lr = l[r];
    lr = xg_sum(lr);
    const int q = q0 + 16 * r + c;
    const float inv = 1.0f / lr;
    half4v ov[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int v = 0; v < 4; ++v) ov[dt][v] = (_Float16)(ot[r][dt][v] * inv);
    const long long bhq = ((long long)b * a.nq + h) * S + q;
    if (q < S) {
      _Float16* o = a.o + (rowb + q) * a.ldo + h * HD;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<half4v*>(o + dt * 16 + 4 * g) = ov[dt];
      if (g == 0) a.lse[bhq] = (m[r] + __log2f(lr)) * LN2;
    }
    if (a.dout) {
      // the block API: the backward's dO operand for this row and head
      // (delta = sum dO * fp16(O), the row's power-of-two dO scale), every
      // lane taking part in the cross-lane sums
      const _Float16* dr = a.dout + (rowb + min(q, S - 1)) * a.lddo + h * HD;
      half4v dv[8];
      float dl = 0.f, am = 0.f;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        dv[dt] = *reinterpret_cast<const half4v*>(dr + dt * 16 + 4 * g);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          dl += (float)dv[dt][v] * (float)ov[dt][v];
          am = fmaxf(am, fabsf((float)dv[dt][v]));
        }
      }
      dl = xg_sum(dl);
      am = xg_max(am);
      if (q < S) {
        const float sc = pow2_scale_for(am, kDoScaleExp);
        _Float16* d16 = a.dO16w + (rowb + q) * a.ld16 + h * HD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          half4v x;
#pragma unroll
          for (int v = 0; v < 4; ++v) x[v] = (_Float16)((float)dv[dt][v] * sc);
          *reinterpret_cast<half4v*>(d16 + dt * 16 + 4 * g) = x;
        }
        if (g == 0) {
          a.deltaw[bhq] = dl;
          a.dscw[bhq] = pow2_inv_scale_for(am, kDoScaleExp);
        }
      }
    }
  }
}

// Per token row, 16 lanes per head (lane j: dims 8 j .. 8 j + 7, 16-byte
// accesses): delta[b, h, s] = sum_d dO * O, and dO16 = fp16(dO * sc) with sc
// the power-of-two scale of the head's max |dO|, dsc[b, h, s] = 1 / sc (0 for
// an all-zero head row).  A workgroup of 256 threads covers DR token rows x
// 16 heads a pass, every load of a pass issued before its math.
constexpr int DR = 4;
template <typename TD>
__global__ __launch_bounds__(256) void attn_delta_kernel(const TD* __restrict__ dO, long long ldd,
                                                         const _Float16* __restrict__ o,
                                                         long long ldo, int nq, int S, int T,
                                                         float* __restrict__ delta,
                                                         _Float16* __restrict__ dO16,
                                                         long long ld16, float* __restrict__ dsc) {
  const int j = threadIdx.x & 15;
  for (int h = threadIdx.x >> 4; h < nq; h += 16) {  // whole 16-lane groups
    float dv[DR][8];
    half8 ov[DR];
#pragma unroll
    for (int i = 0; i < DR; ++i) {
      const long long t = min((long long)blockIdx.x * DR + i, (long long)T - 1);
      const TD* d = dO + t * ldd + h * HD + 8 * j;
      if constexpr (sizeof(TD) == 2) {
        const half8 x = *reinterpret_cast<const half8*>(d);
#pragma unroll
        for (int e = 0; e < 8; ++e) dv[i][e] = (float)x[e];
      } else {
        const float4 x0 = *reinterpret_cast<const float4*>(d);
        const float4 x1 = *reinterpret_cast<const float4*>(d + 4);
        dv[i][0] = x0.x; dv[i][1] = x0.y; dv[i][2] = x0.z; dv[i][3] = x0.w;
        dv[i][4] = x1.x; dv[i][5] = x1.y; dv[i][6] = x1.z; dv[i][7] = x1.w;
      }
      ov[i] = *reinterpret_cast<const half8*>(o + t * ldo + h * HD + 8 * j);
    }
#pragma unroll
    for (int i = 0; i < DR; ++i) {
      const long long t = (long long)blockIdx.x * DR + i;
      float v = 0.f, amax = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v += dv[i][e] * (float)ov[i][e];
        amax = fmaxf(amax, fabsf(dv[i][e]));
      }
      v = sum16_dpp(v);
      amax = max16(amax);
      if (t >= T) continue;  // whole 16-lane groups (after the group reductions)
      const int b = (int)((unsigned)t / (unsigned)S), s = (int)t - b * S;  // T < 2^31
      const float sc = pow2_scale_for(amax, kDoScaleExp);
      const long long bhs = ((long long)b * nq + h) * S + s;
      if (j == 0) {
        delta[bhs] = v;
        dsc[bhs] = pow2_inv_scale_for(amax, kDoScaleExp);
      }
      half8 o16;
#pragma unroll
      for (int e = 0; e < 8; ++e) o16[e] = (_Float16)(dv[i][e] * sc);
      *reinterpret_cast<half8*>(dO16 + t * ld16 + h * HD + 8 * j) = o16;
    }
  }
}

template <int NW, int RW>
void launch_fwd(const AttnArgs& a, int B, hipStream_t st) {
  constexpr int QB = NW * RW * 16;
  hipLaunchKernelGGL((attn_fwd_kernel<NW, RW>), dim3(a.nq, B, (a.S + QB - 1) / QB), dim3(NW * 64),
                     0, st, a);
}

}  // namespace

hipError_t attn_delta(const void* dO, int dO_is_f16, long long ldd, const _Float16* o,
                      long long ldo, int nq, int S, int T, float* delta, _Float16* dO16,
                      long long ld16, float* dsc, hipStream_t st) {
  // 16-byte accesses: row pitches and bases aligned to them
  const size_t es = dO_is_f16 ? 2 : 4;
  if (((uintptr_t)dO | (uintptr_t)o | (uintptr_t)dO16) % 16 || (ldd * es) % 16 || (ldo * 2) % 16 ||
      (ld16 * 2) % 16) {
    set_error("attn_delta: dO, O and dO16 rows need 16-byte alignment");
    return hipErrorInvalidValue;
  }
  const dim3 grid((T + DR - 1) / DR);
  if (dO_is_f16)
    hipLaunchKernelGGL(attn_delta_kernel<_Float16>, grid, dim3(256), 0, st, (const _Float16*)dO,
                       ldd, o, ldo, nq, S, T, delta, dO16, ld16, dsc);
  else
    hipLaunchKernelGGL(attn_delta_kernel<float>, grid, dim3(256), 0, st, (const float*)dO, ldd, o,
                       ldo, nq, S, T, delta, dO16, ld16, dsc);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t attn_fwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0) {
    set_error("attn_fwd: nq=%d nkv=%d S=%d", a.nq, a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  if ((a.qn && !(a.qraw && a.cosT && a.sinT && a.q16w)) ||
      (a.dout && !(a.dO16w && a.deltaw && a.dscw))) {
    set_error("attn_fwd: the fused q norm needs qraw, the RoPE tables and q16w; the dO "
              "operand needs dO16w, deltaw and dscw");
    return hipErrorInvalidValue;
  }
  const AttnShape s = attn_shape(B, a.S, a.nq);
  switch (s.nw * 10 + s.rw) {
    case 42: launch_fwd<4, 2>(a, B, st); break;
    case 41: launch_fwd<4, 1>(a, B, st); break;
    case 22: launch_fwd<2, 2>(a, B, st); break;
    default: launch_fwd<2, 1>(a, B, st); break;
  }
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
