// attn_bwd.hip — the deterministic causal GQA flash-attention backward
// (head_dim 128) on fp16 MFMA for gfx950, recomputing P from Q, K and the
// forward's log-sum-exp.  Two kinds of workgroups that share no outputs:
//   dQ blocks   (query block, query head): dQ = dS K / sqrt(128), each query
//               row in its own dO scale;
//   dK/dV blocks (key block, KV head): dK = dS^T Q / sqrt(128), dV = P^T dO
//               summed over the query heads of the KV head's GQA group inside
//               the workgroup (heads, then query tiles, in a fixed order; no
//               atomics, no per-head partial results in memory).
// Small grids run both kinds side by side in one launch; large ones as one
// launch each.  dO arrives as fp16 rows each scaled by its own power of two
// (the producer writes the inverse scales): dK/dV, which mix rows, bring each
// row to the group's common scale on the fly.
//
// Replaces the reference's attn_backward_kernel (src/kernels/lora_backward.cu:
// 104-186, float atomics) and its GQA contraction (:189-208).  Math:
// dP = dO V^T; dS = P (dP - delta), delta = rowsum(dO * O); dQ = dS K / sqrt(d);
// dK = dS^T Q / sqrt(d); dV = P^T dO.  Query head h reads KV head
// h / (nq / nkv) (include/config.h:15).  Tile layout, DMA and fragment
// conventions: attn_common.h.
#include <algorithm>
#include <type_traits>

#include "attn_common.h"

namespace llmt {

namespace {

// ---------------------------------------------------------------- dQ
// dS^T for one 64-key tile: dp (rows key, column query) = dP^T in, dS^T out.
template <int RW, bool MASK>
__device__ __forceinline__ void ds_tile_q(const floatx4 (&pt)[RW][4], floatx4 (&dp)[RW][4],
                                          const float (&lse2)[RW], const float (&del)[RW],
                                          float sl2, int key0, int q0, int S, int lane) {
  const int c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int q = q0 + 16 * r + c;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float pv = __builtin_amdgcn_exp2f(fmaf(pt[r][mt][v], sl2, -lse2[r]));
        if (MASK) {
          const int key = key0 + mt * 16 + 4 * g + v;
          pv = (key <= q && key < S && q < S) ? pv : 0.f;
        }
        dp[r][mt][v] = pv * (dp[r][mt][v] - del[r]);
      }
  }
}

// Query block qb of head h, batch b: the forward's tiling (LDS: two
// buffers of K and V tiles, 4 TILE halves).  dQ row q depends on dO row q
// only, so each row stays in its own dO scale 1 / dsc[q] throughout.
template <int NW, int RW>
__device__ __forceinline__ void dq_block(const AttnArgs& a, _Float16* buf0, _Float16* buf1, int qb,
                                         int h, int b) {
  constexpr int QB = NW * RW * 16;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int q0 = qb * QB + w * RW * 16;
  const int qlast = min(q0 + RW * 16, S) - 1;
  const float sl2 = a.sm_scale * LOG2E;
  const _Float16* kbase = a.k + rowb * a.ldk + kvh * HD;
  const _Float16* vbase = a.v + rowb * a.ldv + kvh * HD;
  const int nkb = min((qb * QB + QB - 1) / BLK, (S - 1) / BLK) + 1;
  TileDma<NW> dk, dv;
  dk.init(a.ldk, w);
  dv.init(a.ldv, w);
  dk.issue(kbase, a.ldk, 0, S, buf0, w);
  dv.issue(vbase, a.ldv, 0, S, buf0 + TILE, w);
  half8 qf[RW][4], df[RW][4];
  float lse2[RW], del[RW], fq[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int q = q0 + 16 * r + c;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[r][ks] = frag_global(a.q + rowb * a.ldq + h * HD, a.ldq, q, S, ks, lane);
      df[r][ks] = frag_global(a.dO16 + rowb * a.ld16 + h * HD, a.ld16, q, S, ks, lane);
    }
    const bool ok = q < S;
    lse2[r] = ok ? a.lse[((long long)b * a.nq + h) * S + q] * LOG2E : 0.f;
    const float dsc = ok ? a.dsc[((long long)b * a.nq + h) * S + q] : 0.f;
    del[r] = dsc > 0.f ? a.delta[((long long)b * a.nq + h) * S + q] / dsc : 0.f;
    fq[r] = a.sm_scale * dsc;
  }
  floatx4 dqT[RW][8];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < 8; ++i) dqT[r][i] = floatx4{0.f, 0.f, 0.f, 0.f};

  // key tiles wholly at or before every query of the wave (no mask) first,
  // then the diagonal / sequence-end tiles as a loop of their own (every wave
  // runs nkb iterations, so the per-tile barriers stay matched)
  const int nfull = qlast == q0 + RW * 16 - 1 ? min((q0 + 1) / BLK, nkb) : 0;
  // tile kb lives in buffer kb & 1 (Ks), tile kb + 1 lands in the other (nb)
  auto tile_step = [&](int kb, auto mask_tag, const _Float16* Ks, _Float16* nb)
                       __attribute__((always_inline)) {
    wait_vm<0>();
    tile_barrier();
    if (kb + 1 < nkb) {
      dk.issue(kbase, a.ldk, (kb + 1) * BLK, S, nb, w);
      dv.issue(vbase, a.ldv, (kb + 1) * BLK, S, nb + TILE, w);
    }
    constexpr bool MASK = decltype(mask_tag)::value;
    if (MASK && kb * BLK > qlast) return;  // every key after every query of the wave
    const _Float16* Vs = Ks + TILE;
    floatx4 pt[RW][4], dp[RW][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        pt[r][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
        dp[r][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const half8 kf = frag_rm(Ks, mt * 16, ks, lane);
        const half8 vf = frag_rm(Vs, mt * 16, ks, lane);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          pt[r][mt] = mfma16(kf, qf[r][ks], pt[r][mt]);
          dp[r][mt] = mfma16(vf, df[r][ks], dp[r][mt]);
        }
      }
    }
    sched_reads_ahead<32, 32 * RW, 8, 2 * RW, 2, 0>();
    __builtin_amdgcn_sched_barrier(0);
    ds_tile_q<RW, MASK>(pt, dp, lse2, del, sl2, kb * BLK, q0, S, lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      half8 db[RW];
#pragma unroll
      for (int r = 0; r < RW; ++r) db[r] = pair_frag(dp[r][2 * j], dp[r][2 * j + 1]);
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const half8 kt = frag_tr(Ks, d * 16, j, lane);
#pragma unroll
        for (int r = 0; r < RW; ++r) dqT[r][d] = mfma16(kt, db[r], dqT[r][d]);
      }
    }
    sched_reads_ahead<32, 16 * RW, 8, RW, 2, 1>();
    __builtin_amdgcn_sched_barrier(0);
  };
  // The unmasked tiles in pairs with the buffers named statically: the
  // compiler then sees that a tile's LDS reads and the DMA of the next tile
  // touch different arrays and does not make the reads wait for that DMA
  // (with buffers chosen at run time it waits for every DMA in flight).
  for (int kb = 0; kb < nfull; kb += 2) {
    tile_step(kb, std::false_type{}, buf0, buf1);
    if (kb + 1 < nfull) tile_step(kb + 1, std::false_type{}, buf1, buf0);
  }
  for (int kb = nfull; kb < nkb; ++kb)
    tile_step(kb, std::true_type{}, (kb & 1) ? buf1 : buf0, (kb & 1) ? buf0 : buf1);
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int q = q0 + 16 * r + c;
    const float f = fq[r];
    float dy[8][4];
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int v = 0; v < 4; ++v) dy[d][v] = dqT[r][d][v] * f;
    if (a.qn) {  // the block API: through q's RoPE and norm to d qraw
      const int qc = min(q, S - 1);
      norm_rope_bwd_row(dy, a.qraw + (rowb + qc) * a.ldqr + h * HD, a.qn, a.cosT, a.sinT, qc,
                        a.eps, g);
    }
    if (q < S) {
      float* dq = a.dq + (rowb + q) * a.ldgq + h * HD;
#pragma unroll
      for (int d = 0; d < 8; ++d)
        *reinterpret_cast<float4*>(dq + d * 16 + 4 * g) =
            make_float4(dy[d][0], dy[d][1], dy[d][2], dy[d][3]);
    }
  }
}

// dK and dV rows of one key (dkT / dvT in the group's dO scale gs): dK
// through k's RoPE and norm when the block API asks for it (kn).
__device__ __forceinline__ void store_dkdv(const AttnArgs& a, const floatx4 (&dkT)[8],
                                           const floatx4 (&dvT)[8], float gs, long long rowb,
                                           int key, int j, int g) {
  const float inv = 1.0f / gs;
  const float fk = a.sm_scale * inv;
  float dy[8][4];
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int v = 0; v < 4; ++v) dy[d][v] = dkT[d][v] * fk;
  if (a.kn) {
    const int kc = min(key, a.S - 1);
    norm_rope_bwd_row(dy, a.kraw + (rowb + kc) * a.ldkr + j * HD, a.kn, a.cosT, a.sinT, kc,
                      a.eps, g);
  }
  if (key < a.S) {
    float* dk = a.dk + (rowb + key) * a.ldgkv + j * HD;
    float* dv = a.dv + (rowb + key) * a.ldgkv + j * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      *reinterpret_cast<float4*>(dk + dt * 16 + 4 * g) =
          make_float4(dy[dt][0], dy[dt][1], dy[dt][2], dy[dt][3]);
      *reinterpret_cast<float4*>(dv + dt * 16 + 4 * g) =
          make_float4(dvT[dt][0] * inv, dvT[dt][1] * inv, dvT[dt][2] * inv, dvT[dt][3] * inv);
    }
  }
}

// ---------------------------------------------------------------- dK, dV
// P and dS for 32 queries (half j2 of a 64-query tile; rows query, column
// key), both in the group's dO scale gs: ds arrives in each query row's own
// dO scale, so row q's factor r = gs * dsc[q] (<= 1) brings dP there, and P
// times r is the operand against the row-scaled dO16 of dV.
template <bool MASK>
__device__ __forceinline__ void ds_half_kv(floatx4 (&p)[2], floatx4 (&ds)[2], const float* lse_s,
                                           const float* del_s, const float* dsc_s, float sl2,
                                           float gs, int qq0, int j2, int key, int S, int lane) {
  const int g = lane >> 4;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int r0 = (2 * j2 + u) * 16 + 4 * g;
    const float4 ls = *reinterpret_cast<const float4*>(lse_s + r0);
    const float4 dl = *reinterpret_cast<const float4*>(del_s + r0);
    const float4 sc = *reinterpret_cast<const float4*>(dsc_s + r0);
    const float lv[4] = {ls.x, ls.y, ls.z, ls.w};
    const float dv[4] = {dl.x, dl.y, dl.z, dl.w};
    const float rv[4] = {sc.x * gs, sc.y * gs, sc.z * gs, sc.w * gs};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float pv = __builtin_amdgcn_exp2f(fmaf(p[u][v], sl2, -lv[v] * LOG2E));
      if (MASK) {
        const int qq = qq0 + r0 + v;
        pv = (key <= qq && qq < S) ? pv : 0.f;
      }
      p[u][v] = pv * rv[v];
      ds[u][v] = pv * fmaf(ds[u][v], rv[v], -dv[v] * gs);
    }
  }
}

// Common power-of-two scale of the fp16 dO rows of the query heads of KV
// head j in batch b: the reciprocal of their largest inverse row scale
// (all-zero rows store 0), 1 when every row is zero.  Identical in every
// workgroup of (b, j).  Row t enters the products times r_t = gs * dsc[t]
// <= 1, which brings it to this common scale.
template <int NT>
__device__ float group_do_scale(const float* __restrict__ dsc, int b, int nq, int j, int group,
                                int S, float* red) {
  const float* base = dsc + ((long long)b * nq + (long long)j * group) * S;
  float m = 0.f;
  for (int s = threadIdx.x; s < group * S; s += NT) m = fmaxf(m, base[s]);
  m = block_max<NT / 64>(m, red);
  return m > 0.f ? 1.0f / m : 1.0f;
}

// Scores of half j2 (queries 32 j2 .. 32 j2 + 31 of the tile) against the
// wave's 16 keys: p = Q K^T and ds = dO V^T, rows query, column key.
__device__ __forceinline__ void kv_scores(const _Float16* Qs, const _Float16* Ds,
                                          const half8 (&kf)[4], const half8 (&vf)[4], int j2,
                                          floatx4 (&p)[2], floatx4 (&ds)[2], int lane) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int mt = 2 * j2 + u;
    p[u] = floatx4{0.f, 0.f, 0.f, 0.f};
    ds[u] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      p[u] = mfma16(frag_rm(Qs, mt * 16, ks, lane), kf[ks], p[u]);
      ds[u] = mfma16(frag_rm(Ds, mt * 16, ks, lane), vf[ks], ds[u]);
    }
  }
}

// dV^T += dO^T P and dK^T += Q^T dS over half j2 (P, dS paired into B operands).
__device__ __forceinline__ void kv_accum(const _Float16* Qs, const _Float16* Ds, int j2,
                                         const half8& pb, const half8& db, floatx4 (&dkT)[8],
                                         floatx4 (&dvT)[8], int lane) {
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    dvT[dt] = mfma16(frag_tr(Ds, dt * 16, j2, lane), pb, dvT[dt]);
    dkT[dt] = mfma16(frag_tr(Qs, dt * 16, j2, lane), db, dkT[dt]);
  }
}

// One 64-query tile for a wave's 16 keys, the halves one after the other,
// each phase its own scheduling region with the LDS reads issued ahead of the
// MFMAs.  (Interleaving one half's dS VALU with the other half's MFMAs was
// measured slower at B4 x S2048: 277 against 255 us.)
template <bool MASK>
__device__ __forceinline__ void kv_tile(const _Float16* Qs, const _Float16* Ds,
                                        const float* lse_s, const float* del_s,
                                        const float* dsc_s, const half8 (&kf)[4],
                                        const half8 (&vf)[4], floatx4 (&dkT)[8],
                                        floatx4 (&dvT)[8], float sl2, float gs, int qq0, int key,
                                        int S, int lane) {
#pragma unroll
  for (int j2 = 0; j2 < 2; ++j2) {
    floatx4 p[2], ds[2];
    kv_scores(Qs, Ds, kf, vf, j2, p, ds, lane);
    sched_reads_ahead<16, 16, 6, 2, 2, 0>();
    __builtin_amdgcn_sched_barrier(0);
    ds_half_kv<MASK>(p, ds, lse_s, del_s, dsc_s, sl2, gs, qq0, j2, key, S, lane);
    __builtin_amdgcn_sched_barrier(0);
    kv_accum(Qs, Ds, j2, pair_frag(p[0], p[1]), pair_frag(ds[0], ds[1]), dkT, dvT, lane);
    sched_reads_ahead<32, 16, 8, 2, 4, 1>();
    __builtin_amdgcn_sched_barrier(0);
  }
}

constexpr int KV_BUF = 2 * TILE + 3 * BLK * 2;  // halves per dK/dV LDS buffer

// Workgroup (key block kb of 16 KW NW keys, KV head j, batch b).  Wave w
// owns the keys k0 = kb 16 KW NW + 16 KW w .. as KW 16-key tiles (every Q
// and dO fragment read from LDS feeds KW MFMAs) and runs over the query
// heads of the group and, for each, the 64-query tiles at or after the
// block, in two 32-query halves (P and dS of one half live at a time).
// The kernels use KW = 1: measured at B4 x S2048, one tile a wave at two
// waves per SIMD (184 VGPRs) takes 292 us, two tiles at one wave per SIMD
// (460 registers) 424 us.
// LDS: two buffers of (Q tile, dO16 tile, lse[64], delta[64], dsc[64]); the
// next (head, tile) lands while the current one is computed.
template <int NW, int KW>
__device__ __forceinline__ void dkdv_block(const AttnArgs& a, _Float16* buf0, _Float16* buf1,
                                           float* red, int kb, int j, int b) {
  static_assert(KW == 1, "kv_tile handles one 16-key tile a wave");
  constexpr int NT = NW * 64, KB = NW * 16 * KW;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int S = a.S, group = a.nq / a.nkv;
  const long long rowb = (long long)b * S;
  const int k0 = kb * KB + w * 16 * KW;
  const float sl2 = a.sm_scale * LOG2E;
  const int qb0 = (kb * KB) / BLK;
  const int qlast = (S - 1) / BLK;
  const int nqt = qlast - qb0 + 1;  // query tiles per head
  const int niter = group * nqt;
  // Iteration order: the tiles that need the causal / sequence-end mask (the
  // diagonal tile of each head, then a partial last tile of each head) come
  // first, as their own loop, then the full tiles of each head.
  const int nlast = (S % BLK && nqt > 1) ? 1 : 0;
  const int nmask = group * (1 + nlast), nfull = nqt - 1 - nlast;
  auto tile_of = [&](int it, int& h, int& qb) {
    if (it < group) {
      h = j * group + it;
      qb = qb0;
    } else if (it < nmask) {
      h = j * group + it - group;
      qb = qlast;
    } else {
      h = j * group + (it - nmask) / nfull;
      qb = qb0 + 1 + (it - nmask) % nfull;
    }
  };
  TileDma<NW> dq_, dd_;
  dq_.init(a.ldq, w);
  dd_.init(a.ld16, w);
  auto issue = [&](int it, _Float16* buf) {
    int h, qb;
    tile_of(it, h, qb);
    dq_.issue(a.q + rowb * a.ldq + h * HD, a.ldq, qb * BLK, S, buf, w);
    dd_.issue(a.dO16 + rowb * a.ld16 + h * HD, a.ld16, qb * BLK, S, buf + TILE, w);
    float* vec = reinterpret_cast<float*>(buf + 2 * TILE);
    const long long bh = ((long long)b * a.nq + h) * S;
    if (w == 0) dma_vec64(a.lse + bh, qb * BLK, S, vec);
    if (w == NW - 1) dma_vec64(a.delta + bh, qb * BLK, S, vec + BLK);
    if (w == NW / 2) dma_vec64(a.dsc + bh, qb * BLK, S, vec + 2 * BLK);
  };
  issue(0, buf0);
  const float gs = group_do_scale<NT>(a.dsc, b, a.nq, j, group, S, red);
  half8 kf[KW][4], vf[KW][4];
#pragma unroll
  for (int t = 0; t < KW; ++t)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kf[t][ks] = frag_global(a.k + rowb * a.ldk + j * HD, a.ldk, k0 + 16 * t + c, S, ks, lane);
      vf[t][ks] = frag_global(a.v + rowb * a.ldv + j * HD, a.ldv, k0 + 16 * t + c, S, ks, lane);
    }
  floatx4 dkT[KW][8], dvT[KW][8];
#pragma unroll
  for (int t = 0; t < KW; ++t)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dkT[t][i] = floatx4{0.f, 0.f, 0.f, 0.f};
      dvT[t][i] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  // one iteration: wait for tile it (in buf, buffer it & 1), start tile
  // it + 1 (into nb), run tile it
  auto tile_step = [&](int it, auto mask_tag, const _Float16* buf, _Float16* nb)
                       __attribute__((always_inline)) {
    wait_vm<0>();
    tile_barrier();
    if (it + 1 < niter) issue(it + 1, nb);
    int h, qb;
    tile_of(it, h, qb);
    const _Float16* Qs = buf;
    const _Float16* Ds = buf + TILE;
    const float* lse_s = reinterpret_cast<const float*>(buf + 2 * TILE);
    const float* del_s = lse_s + BLK;
    const float* dsc_s = lse_s + 2 * BLK;
    kv_tile<decltype(mask_tag)::value>(Qs, Ds, lse_s, del_s, dsc_s, kf[0], vf[0], dkT[0], dvT[0],
                                       sl2, gs, qb * BLK, k0 + c, S, lane);
  };
  auto step_rt = [&](int it, auto mask_tag) __attribute__((always_inline)) {
    tile_step(it, mask_tag, (it & 1) ? buf1 : buf0, (it & 1) ? buf0 : buf1);
  };
  for (int it = 0; it < nmask; ++it) step_rt(it, std::true_type{});
  // the full tiles in pairs with statically named buffers (see dq_block)
  int it = nmask;
  if (it < niter && (it & 1)) step_rt(it++, std::false_type{});
  for (; it < niter; it += 2) {
    tile_step(it, std::false_type{}, buf0, buf1);
    if (it + 1 < niter) tile_step(it + 1, std::false_type{}, buf1, buf0);
  }
#pragma unroll
  for (int t = 0; t < KW; ++t) store_dkdv(a, dkT[t], dvT[t], gs, rowb, k0 + 16 * t + c, j, g);
}

// Small grids (the B1 x S128 step: 8 KV heads x 8 key blocks): the NW waves
// of the workgroup all own the same 16 keys and split the group's
// (query head, query tile) iterations between them (wave w takes it = w,
// w + NW, ..), each through LDS buffers of its own (no barriers in the
// loop); their dK/dV sums meet in LDS at the end, in wave order.  Two waves
// keep two buffers each (the next tile lands during the current one); four
// waves one each (4 x 33.5 KB of LDS), refilled once the wave's reads of it
// have returned -- at B1 x S128 (2 query heads x 2 tiles) each wave then
// has a single iteration.
template <int NW>
constexpr int split_bufs() { return NW >= 4 ? 1 : 2; }

template <int NW>
__device__ __forceinline__ void dkdv_block_split(const AttnArgs& a, _Float16* smem, float* red,
                                                 int kb, int j, int b) {
  constexpr int NT = NW * 64;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int S = a.S, group = a.nq / a.nkv;
  const long long rowb = (long long)b * S;
  const int k0 = kb * 16;
  const float sl2 = a.sm_scale * LOG2E;
  const int qb0 = k0 / BLK;
  const int nqt = (S + BLK - 1) / BLK - qb0;
  const int niter = group * nqt;
  constexpr int NB = split_bufs<NW>();
  _Float16* mine = smem + w * NB * KV_BUF;
  TileDma<1> dq_, dd_;
  dq_.init(a.ldq, 0);
  dd_.init(a.ld16, 0);
  auto issue = [&](int it, _Float16* buf) {
    const int h = j * group + it / nqt, qb = qb0 + it % nqt;
    dq_.issue(a.q + rowb * a.ldq + h * HD, a.ldq, qb * BLK, S, buf, 0);
    dd_.issue(a.dO16 + rowb * a.ld16 + h * HD, a.ld16, qb * BLK, S, buf + TILE, 0);
    float* vec = reinterpret_cast<float*>(buf + 2 * TILE);
    const long long bh = ((long long)b * a.nq + h) * S;
    dma_vec64(a.lse + bh, qb * BLK, S, vec);
    dma_vec64(a.delta + bh, qb * BLK, S, vec + BLK);
    dma_vec64(a.dsc + bh, qb * BLK, S, vec + 2 * BLK);
  };
  if (w < niter) issue(w, mine);
  const float gs = group_do_scale<NT>(a.dsc, b, a.nq, j, group, S, red);
  half8 kf[4], vf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    kf[ks] = frag_global(a.k + rowb * a.ldk + j * HD, a.ldk, k0 + c, S, ks, lane);
    vf[ks] = frag_global(a.v + rowb * a.ldv + j * HD, a.ldv, k0 + c, S, ks, lane);
  }
  floatx4 dkT[8], dvT[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dkT[i] = floatx4{0.f, 0.f, 0.f, 0.f};
    dvT[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  int n = 0;
  for (int it = w; it < niter; it += NW, ++n) {
    wait_vm<0>();  // this wave's own tile (its buffers are private)
    asm volatile("" ::: "memory");
    if constexpr (NB == 2)
      if (it + NW < niter) issue(it + NW, mine + ((n + 1) & 1) * KV_BUF);
    const _Float16* buf = mine + (NB == 2 ? (n & 1) * KV_BUF : 0);
    const int qb = qb0 + it % nqt;
    if (qb * BLK + BLK - 1 < k0) {
      if constexpr (NB == 1)
        if (it + NW < niter) issue(it + NW, mine);
      continue;
    }
    const _Float16* Qs = buf;
    const _Float16* Ds = buf + TILE;
    const float* lse_s = reinterpret_cast<const float*>(buf + 2 * TILE);
    const float* del_s = lse_s + BLK;
    const float* dsc_s = lse_s + 2 * BLK;
    const bool full = qb * BLK >= k0 + 15 && qb * BLK + BLK <= S;
    if (full)
      kv_tile<false>(Qs, Ds, lse_s, del_s, dsc_s, kf, vf, dkT, dvT, sl2, gs, qb * BLK, k0 + c, S,
                     lane);
    else
      kv_tile<true>(Qs, Ds, lse_s, del_s, dsc_s, kf, vf, dkT, dvT, sl2, gs, qb * BLK, k0 + c, S,
                    lane);
    if constexpr (NB == 1) {
      if (it + NW < niter) {  // one buffer: refill it once this tile's reads returned
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
        issue(it + NW, mine);
      }
    }
  }
  // waves 1 .. NW-1 hand their sums to wave 0, which adds them in order
  wait_vm<0>();
  __syncthreads();
  floatx4* xch = reinterpret_cast<floatx4*>(smem);
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xch[((w - 1) * 16 + i) * 64 + lane] = dkT[i];
      xch[((w - 1) * 16 + 8 + i) * 64 + lane] = dvT[i];
    }
  }
  __syncthreads();
  if (w > 0) return;
  for (int ww = 1; ww < NW; ++ww)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dkT[i] += xch[((ww - 1) * 16 + i) * 64 + lane];
      dvT[i] += xch[((ww - 1) * 16 + 8 + i) * 64 + lane];
    }
  store_dkdv(a, dkT, dvT, gs, rowb, k0 + c, j, g);
}

// The attention backward of a launch over a grid (B, x): x < nkv nkvb are
// dK/dV blocks (key block x / nkv, KV head x % nkv: the longest key blocks
// first), the next nq nqb dQ blocks (the last, i.e. longest, query blocks
// first).  The batch is the fastest grid index, so the longest blocks of
// every batch are dispatched first (with the batch outermost, at B4 x S2048
// the last batches' 178 us key blocks started only once earlier ones had
// drained, leaving a tail at half occupancy for 45% of the dK/dV launch).
// PART 0: both kinds; 1: dK/dV only; 2: dQ only -- the one-kind forms keep
// their own (smaller) register and LDS budgets.
constexpr int BWD_BUF = KV_BUF > 2 * TILE ? KV_BUF : 2 * TILE;  // halves per buffer

template <int NW, int RW, int PART>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void attn_bwd_kernel(const AttnArgs a, int nkvb, int nqb) {
  // PART 0-2: the two tile buffers as separate arrays (statically named
  // buffers, see dq_block); PART 3: one array split per wave.
  constexpr int BUF = PART == 1 ? KV_BUF : PART == 2 ? 2 * TILE : BWD_BUF;
  constexpr int SMEM3 = NW * split_bufs<NW>() * KV_BUF > 4 * TILE ? NW * split_bufs<NW>() * KV_BUF : 4 * TILE;
  __shared__ __attribute__((aligned(1024))) _Float16 buf0[PART == 3 ? SMEM3 : BUF];
  __shared__ __attribute__((aligned(1024))) _Float16 buf1[PART == 3 ? 8 : BUF];
  __shared__ float red[NW];
  const int x = blockIdx.y, b = blockIdx.x;
  const int nkvx = PART == 2 ? 0 : nkvb * a.nkv;
  if constexpr (PART != 2) {
    if (x < nkvx) {
      if constexpr (PART == 3)
        dkdv_block_split<NW>(a, buf0, red, x / a.nkv, x % a.nkv, b);
      else
        dkdv_block<NW, 1>(a, buf0, buf1, red, x / a.nkv, x % a.nkv, b);
      return;
    }
  }
  if constexpr (PART != 1) {
    const int y = x - nkvx;
    if constexpr (PART == 3)
      dq_block<NW, RW>(a, buf0, buf0 + 2 * TILE, nqb - 1 - y / a.nq, y % a.nq, b);
    else
      dq_block<NW, RW>(a, buf0, buf1, nqb - 1 - y / a.nq, y % a.nq, b);
  }
}

int dkdv_waves(int B, int S, int nkv) {
  const char* e = getenv("LLMT_ATTN_DKDV_WAVES");
  if (e && (e[0] == '2' || e[0] == '4') && !e[1]) return e[0] - '0';
  return (long long)B * nkv * ((S + 63) / 64) >= 256 ? 4 : 2;
}

template <int NW, int RW, int PART>
void launch_bwd(const AttnArgs& a, int B, int nkvb, int nqb, hipStream_t st) {
  const int nx = (PART == 2 ? 0 : nkvb * a.nkv) + (PART == 1 ? 0 : nqb * a.nq);
  hipLaunchKernelGGL((attn_bwd_kernel<NW, RW, PART>), dim3(B, nx), dim3(NW * 64), 0, st, a, nkvb,
                     nqb);
}

// dK/dV key blocks of nwk waves and dQ query blocks of nwq waves x rw tiles:
// one launch when the wave counts agree and the grid is small (under 2048
// workgroups: a second launch would mostly wait on the first one's tail),
// else one launch each.
bool bwd_one_launch(const AttnArgs& a, int B, int nwk, int nwq, int rw) {
  const int nkvb = (a.S + nwk * 16 - 1) / (nwk * 16);
  const int nqb = (a.S + nwq * rw * 16 - 1) / (nwq * rw * 16);
  return nwk == nwq && ((long long)nkvb * a.nkv + (long long)nqb * a.nq) * B < 2048;
}

void launch_attn_bwd(const AttnArgs& a, int B, int nwk, int nwq, int rw, hipStream_t st) {
  const int nkvb = (a.S + nwk * 16 - 1) / (nwk * 16);
  const int nqb = (a.S + nwq * rw * 16 - 1) / (nwq * rw * 16);
  if (bwd_one_launch(a, B, nwk, nwq, rw)) {
    switch (nwq * 10 + rw) {
      case 42: launch_bwd<4, 2, 0>(a, B, nkvb, nqb, st); break;
      case 41: launch_bwd<4, 1, 0>(a, B, nkvb, nqb, st); break;
      case 22: launch_bwd<2, 2, 0>(a, B, nkvb, nqb, st); break;
      default: launch_bwd<2, 1, 0>(a, B, nkvb, nqb, st); break;
    }
    return;
  }
  // dQ first: its sweep leaves Q, K, V and dO warm for the dK/dV launch
  switch (nwq * 10 + rw) {
    case 42: launch_bwd<4, 2, 2>(a, B, 0, nqb, st); break;
    case 41: launch_bwd<4, 1, 2>(a, B, 0, nqb, st); break;
    case 22: launch_bwd<2, 2, 2>(a, B, 0, nqb, st); break;
    default: launch_bwd<2, 1, 2>(a, B, 0, nqb, st); break;
  }
  if (nwk == 4)
    launch_bwd<4, 1, 1>(a, B, nkvb, 0, st);
  else
    launch_bwd<2, 1, 1>(a, B, nkvb, 0, st);
}

}  // namespace

hipError_t attn_bwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0 || !a.dO16 || !a.dsc || !a.dk || !a.dv) {
    set_error("attn_bwd: nq=%d nkv=%d S=%d (fp16 dO, its scales and dK/dV outputs required)",
              a.nq, a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  if ((long long)(a.S + 15) / 16 * (a.nq + a.nkv) > 65535) {
    set_error("attn_bwd: S=%d with %d + %d heads exceeds the grid's y range", a.S, a.nq, a.nkv);
    return hipErrorInvalidValue;
  }
  if ((a.qn && !a.qraw) || (a.kn && !a.kraw) || ((a.qn || a.kn) && !(a.cosT && a.sinT))) {
    set_error("attn_bwd: the fused QK-norm backward needs the raw q / k and the RoPE tables");
    return hipErrorInvalidValue;
  }
  // dQ holds twice the accumulators of the forward: in a launch of its own
  // one 16-row tile a wave (two waves per SIMD) was faster at every S; where
  // dQ and dK/dV blocks share one launch (B8 x S512) the forward's two tiles
  // a wave are (attention backward 54.4 against 58.4 us), the dQ blocks then
  // being as long as the dK/dV ones.  LLMT_ATTN_CFG still selects any shape.
  AttnShape s = attn_shape(B, a.S, a.nq);
  if (!getenv("LLMT_ATTN_CFG")) {
    if (!bwd_one_launch(a, B, dkdv_waves(B, a.S, a.nkv), s.nw, s.rw)) s.rw = 1;
    // tiny grids (the B1 x S128 step): dK/dV blocks of 16 keys whose four
    // waves split the group's query tiles, beside 64-query dQ blocks
    if (!getenv("LLMT_ATTN_DKDV_WAVES") && (long long)B * a.nq * ((a.S + 63) / 64) < 64) {
      launch_bwd<4, 1, 3>(a, B, (a.S + 15) / 16, (a.S + 63) / 64, st);
      LLMT_LAUNCH_CHECK();
      return hipSuccess;
    }
  }
  launch_attn_bwd(a, B, dkdv_waves(B, a.S, a.nkv), s.nw, s.rw, st);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
