// attn.hip — causal GQA flash attention (head_dim 128) on fp16 MFMA for
// gfx950: forward (keeps the fp32 log-sum-exp instead of P) and a
// deterministic backward in one launch (dQ per query block beside dK/dV per
// key block and query head, the query heads of a GQA group summed by the
// consumer in a fixed order), recomputing P from Q, K and the LSE.  The
// backward takes dO as fp16 rows each scaled by its own power of two (the
// producer's row epilogue writes them with the inverse scales): dQ works in
// each row's own scale, dK and dV, which mix rows, bring each row to its
// batch's common scale on the fly.
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
// 4 g + i of tile 2j (i < 4) or of tile 2j + 1 (i >= 4).  The matching A
// operand is a column of a row-major LDS tile, read with the gfx950
// transposing load ds_read_b64_tr_b16 (in each 16-lane group, lane l gets
// element l % 4 of the 8-byte blocks addressed by lanes 4 e + l / 4, e = 0..3).
//
// Tiles: 64 rows x 128 halves (16 KB), moved global -> LDS by buffer loads
// with an LDS destination (16 bytes a lane) into two buffers, so tile i + 1
// lands while tile i is computed; one barrier per tile.  No padding: the
// 16-byte piece p of tile row r sits in slot p ^ (r % 16).  Measured on
// MI355X (cycles per wave instruction, four waves): the row-fragment reads
// (16 rows, one piece) run at the rate of a contiguous ds_read_b128 (28.6;
// unswizzled 128.0), the transposed reads at that of a contiguous
// ds_read_b64_tr_b16 (25.8; unswizzled 64.0).  Rows past S read as zeros
// (buffer range check); causality and the sequence end are masked in the
// diagonal / last tiles only, chosen per wave with scalar branches.
#include <stdlib.h>

#include <algorithm>

#include "ops.h"

namespace llmt {

namespace {

constexpr int HD = 128;
constexpr int BLK = 64;           // rows per LDS tile
constexpr int TILE = BLK * HD;    // halves per LDS tile
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

typedef short short4v __attribute__((ext_vector_type(4)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int r) { return r & 15; }
// Offset (halves) of halves 8 p .. 8 p + 7 of tile row r.
__device__ __forceinline__ int toff(int r, int p) { return r * HD + ((p ^ swz(r)) << 3); }

// s_waitcnt vmcnt(N), lgkmcnt/expcnt left free (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that also keeps the compiler from moving LDS accesses
// across it (the DMA completion is covered by the wait_vm before it).
__device__ __forceinline__ void tile_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// DMA of 64-row tiles through buffer loads with an LDS destination: rows
// past the end of the matrix fall outside the buffer and arrive as zeros.
// Wave w moves the 1 KB chunks w, w + NW, ...: chunk ch holds tile rows
// 4 ch .. 4 ch + 3; lane l fills slot l % 16 of row 4 ch + l / 16.  The
// per-lane byte offsets are fixed for a given row pitch, so a tile costs
// one descriptor (scalar) and 16 / NW loads a wave.
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format

// (non-template wrappers: the host pass drops kernel stubs when templates
// call the LDS-destination buffer load directly)
__device__ __forceinline__ void buffer_lds16(__amdgpu_buffer_rsrc_t rs, void* lds, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 16, off, 0, 0, 0);
}
__device__ __forceinline__ void buffer_lds4(__amdgpu_buffer_rsrc_t rs, void* lds, unsigned off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds, 4, off, 0, 0, 0);
}

template <int NW>
struct TileDma {
  unsigned off[16 / NW];
  __device__ __forceinline__ void init(long long ld, int w) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i) {
      const int r = 4 * (w + NW * i) + (lane >> 4);
      off[i] = (unsigned)(r * ld * 2 + (((lane & 15) ^ swz(r)) << 4));
    }
  }
  // Rows r0 .. r0 + 63 of `src` ([nrows, ld] fp16) into `tile`.
  __device__ __forceinline__ void issue(const _Float16* src, long long ld, int r0, int nrows,
                                        _Float16* tile, int w) const {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(src + (long long)r0 * ld), (short)0, (int)((long long)(nrows - r0) * ld * 2),
        kRsrcWord3);
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i)
      buffer_lds16(rs, tile + (w + NW * i) * 512, off[i]);
  }
};

// src[i0 .. i0 + 63] (fp32, zeros past n) into LDS by one wave.
__device__ __forceinline__ void dma_vec64(const float* src, int i0, int n, float* dst) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(src + i0), (short)0, (n - i0) * 4, kRsrcWord3);
  buffer_lds4(rs, dst, (threadIdx.x & 63) * 4);
}

// Row fragment: rows m0 + c, halves 32 ks + 8 g .. + 7 (piece 4 ks + g).
__device__ __forceinline__ half8 frag_rm(const _Float16* t, int m0, int ks, int lane) {
  return *reinterpret_cast<const half8*>(t + toff(m0 + (lane & 15), 4 * ks + (lane >> 4)));
}

// Column fragment for the paired-accumulator k order: lane (c, g) gets
// tile[32 j + 4 g + i][d0 + c] (i < 4) and tile[32 j + 16 + 4 g + i - 4][d0 + c].
__device__ __forceinline__ half8 frag_tr(const _Float16* t, int d0, int j, int lane) {
  const int jl = lane & 15;
  const int r = 32 * j + 4 * (lane >> 4) + (jl >> 2);
  const int col = d0 + 4 * (jl & 3);
  const int off = (col & 7);
  const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(t + toff(r, col >> 3) + off));
  const short4v hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(t + toff(r + 16, col >> 3) + off));
  const half4v l4 = __builtin_bit_cast(half4v, lo), h4 = __builtin_bit_cast(half4v, hi);
  half8 x;
  x[0] = l4[0]; x[1] = l4[1]; x[2] = l4[2]; x[3] = l4[3];
  x[4] = h4[0]; x[5] = h4[1]; x[6] = h4[2]; x[7] = h4[3];
  return x;
}

// B fragment built from two accumulator tiles (see the file comment).
__device__ __forceinline__ half8 pair_frag(const floatx4& a, const floatx4& b) {
  half8 r;
  r[0] = (_Float16)a[0]; r[1] = (_Float16)a[1]; r[2] = (_Float16)a[2]; r[3] = (_Float16)a[3];
  r[4] = (_Float16)b[0]; r[5] = (_Float16)b[1]; r[6] = (_Float16)b[2]; r[7] = (_Float16)b[3];
  return r;
}

// Operand fragment straight from global memory: row `row` (zero if >= n),
// halves 32 ks + 8 g .. + 7.
__device__ __forceinline__ half8 frag_global(const _Float16* base, long long ld, int row, int n,
                                             int ks, int lane) {
  const half8 x =
      *reinterpret_cast<const half8*>(base + (long long)min(row, n - 1) * ld + ks * 32 + (lane >> 4) * 8);
  return row < n ? x : half8{};
}

// Common power-of-two scale of batch b's fp16 dO rows: the reciprocal of the
// largest per-row inverse scale (all-zero rows store 0), 1 when every row is
// zero.  Identical in every workgroup of b.  Row t enters the products
// times r_t = gs * dsc[t] <= 1, which brings it to this common scale.
template <int NT>
__device__ float batch_do_scale(const float* __restrict__ dsc_bh, int S, float* red) {
  float m = 0.f;
  for (int s = threadIdx.x; s < S; s += NT) m = fmaxf(m, dsc_bh[s]);
  m = block_max<NT / 64>(m, red);
  return m > 0.f ? 1.0f / m : 1.0f;
}

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
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m[r], bm * sl2);  // sl2 > 0: max commutes with the scale
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m[r] - mu);
    m[r] = mn;
    float ps = 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = __builtin_amdgcn_exp2f(fmaf(st[r][mt][v], sl2, -mu));
        st[r][mt][v] = p;
        ps += p;
      }
    l[r] = l[r] * alpha + ps;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) ot[r][dt] *= alpha;
  }
}

// grid (ceil(S / QB), nq, B), QB = 16 NW RW queries; blockIdx.x runs the
// longest (last) query blocks first.  Wave w owns queries q0 + 16 r + c
// (r < RW).  LDS: two buffers of (K tile, V tile).
template <int NW, int RW>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const AttnArgs a) {
  constexpr int QB = NW * RW * 16;
  __shared__ __attribute__((aligned(1024))) _Float16 smem[4 * TILE];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int qb = gridDim.x - 1 - blockIdx.x, h = blockIdx.y, b = blockIdx.z;
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
  dk.issue(kbase, a.ldk, 0, S, smem, w);
  dv.issue(vbase, a.ldv, 0, S, smem + TILE, w);
  half8 qf[RW][4];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[r][ks] = frag_global(a.q + rowb * a.ldq + h * HD, a.ldq, q0 + 16 * r + c, S, ks, lane);

  floatx4 ot[RW][8];
  float m[RW], l[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ot[r][i] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  for (int kb = 0; kb < nkb; ++kb) {
    wait_vm<0>();
    tile_barrier();
    if (kb + 1 < nkb) {
      _Float16* nb = smem + ((kb + 1) & 1) * 2 * TILE;
      dk.issue(kbase, a.ldk, (kb + 1) * BLK, S, nb, w);
      dv.issue(vbase, a.ldv, (kb + 1) * BLK, S, nb + TILE, w);
    }
    if (kb * BLK > qlast) continue;  // every key after every query of the wave
    const _Float16* Ks = smem + (kb & 1) * 2 * TILE;
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
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    float lr = l[r];
    lr += __shfl_xor(lr, 16, 64);
    lr += __shfl_xor(lr, 32, 64);
    const int q = q0 + 16 * r + c;
    if (q < S) {
      const float inv = 1.0f / lr;
      _Float16* o = a.o + (rowb + q) * a.ldo + h * HD;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        half4v x;
#pragma unroll
        for (int v = 0; v < 4; ++v) x[v] = (_Float16)(ot[r][dt][v] * inv);
        *reinterpret_cast<half4v*>(o + dt * 16 + 4 * g) = x;
      }
      if (g == 0) a.lse[((long long)b * a.nq + h) * S + q] = (m[r] + __log2f(lr)) * LN2;
    }
  }
}

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
__device__ __forceinline__ void dq_block(const AttnArgs& a, _Float16* smem, int qb, int h, int b) {
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
  dk.issue(kbase, a.ldk, 0, S, smem, w);
  dv.issue(vbase, a.ldv, 0, S, smem + TILE, w);
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

  for (int kb = 0; kb < nkb; ++kb) {
    wait_vm<0>();
    tile_barrier();
    if (kb + 1 < nkb) {
      _Float16* nb = smem + ((kb + 1) & 1) * 2 * TILE;
      dk.issue(kbase, a.ldk, (kb + 1) * BLK, S, nb, w);
      dv.issue(vbase, a.ldv, (kb + 1) * BLK, S, nb + TILE, w);
    }
    if (kb * BLK > qlast) continue;
    const _Float16* Ks = smem + (kb & 1) * 2 * TILE;
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
    if (kb * BLK + BLK - 1 <= q0 && kb * BLK + BLK <= S && qlast == q0 + RW * 16 - 1)
      ds_tile_q<RW, false>(pt, dp, lse2, del, sl2, kb * BLK, q0, S, lane);
    else
      ds_tile_q<RW, true>(pt, dp, lse2, del, sl2, kb * BLK, q0, S, lane);
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
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int q = q0 + 16 * r + c;
    const float f = fq[r];
    if (q < S) {
      float* dq = a.dq + (rowb + q) * a.ldgq + h * HD;
#pragma unroll
      for (int d = 0; d < 8; ++d)
        *reinterpret_cast<float4*>(dq + d * 16 + 4 * g) =
            make_float4(dqT[r][d][0] * f, dqT[r][d][1] * f, dqT[r][d][2] * f, dqT[r][d][3] * f);
    }
  }
}

// ---------------------------------------------------------------- dK, dV
// P and dS for one 64-query tile (rows query, column key), both in the
// batch's dO scale gs: ds arrives in each query row's own dO scale, so row
// q's factor r = gs * dsc[q] (<= 1) brings dP there, and P times r is the
// operand against the row-scaled dO16 of dV.
template <bool MASK>
__device__ __forceinline__ void ds_tile_kv(floatx4 (&p)[4], floatx4 (&ds)[4], const float* lse_s,
                                           const float* del_s, const float* dsc_s, float sl2,
                                           float gs, int qq0, int key, int S, int lane) {
  const int g = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const float4 ls = *reinterpret_cast<const float4*>(lse_s + mt * 16 + 4 * g);
    const float4 dl = *reinterpret_cast<const float4*>(del_s + mt * 16 + 4 * g);
    const float4 sc = *reinterpret_cast<const float4*>(dsc_s + mt * 16 + 4 * g);
    const float lv[4] = {ls.x, ls.y, ls.z, ls.w};
    const float dv[4] = {dl.x, dl.y, dl.z, dl.w};
    const float rv[4] = {sc.x * gs, sc.y * gs, sc.z * gs, sc.w * gs};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float pv = __builtin_amdgcn_exp2f(fmaf(p[mt][v], sl2, -lv[v] * LOG2E));
      if (MASK) {
        const int qq = qq0 + mt * 16 + 4 * g + v;
        pv = (key <= qq && qq < S) ? pv : 0.f;
      }
      p[mt][v] = pv * rv[v];
      ds[mt][v] = pv * fmaf(ds[mt][v], rv[v], -dv[v] * gs);
    }
  }
}

// grid (ceil(S / (16 NW)), nq, B): workgroup (key block kb of 16 NW keys,
// query head h); wave w owns keys k0 + 16 w + c and loops over the 64-query
// tiles at or after the block.  LDS: two buffers of (Q tile, dO16 tile,
// lse[64], delta[64], dsc[64]).  Writes this query head's share of dK, dV
// (fp32) to a.dkvp.
constexpr int KV_BUF = 2 * TILE + 3 * BLK * 2;  // halves per dK/dV buffer

template <int NW>
__device__ __forceinline__ void dkdv_block(const AttnArgs& a, _Float16* smem, float* red, int kb,
                                           int h, int b) {
  constexpr int NT = NW * 64, KB = NW * 16;
  constexpr int BUF = KV_BUF;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int S = a.S;
  const int kvh = h / (a.nq / a.nkv);
  const long long rowb = (long long)b * S;
  const int k0 = kb * KB + w * 16;  // first key of the wave
  const int key = k0 + c;
  const float sl2 = a.sm_scale * LOG2E;
  const float* lse_h = a.lse + ((long long)b * a.nq + h) * S;
  const float* del_h = a.delta + ((long long)b * a.nq + h) * S;
  const float* dsc_b = a.dsc + ((long long)b * a.nq + h) * S;
  const _Float16* qbase = a.q + rowb * a.ldq + h * HD;
  const _Float16* dbase = a.dO16 + rowb * a.ld16 + h * HD;
  const int qb0 = (kb * KB) / BLK;
  const int nqb = (S + BLK - 1) / BLK;
  TileDma<NW> dq_, dd_;
  dq_.init(a.ldq, w);
  dd_.init(a.ld16, w);
  auto issue = [&](int qb, _Float16* buf) {
    dq_.issue(qbase, a.ldq, qb * BLK, S, buf, w);
    dd_.issue(dbase, a.ld16, qb * BLK, S, buf + TILE, w);
    float* vec = reinterpret_cast<float*>(buf + 2 * TILE);
    if (w == 0) dma_vec64(lse_h, qb * BLK, S, vec);
    if (w == NW - 1) dma_vec64(del_h, qb * BLK, S, vec + BLK);
    if (w == NW / 2) dma_vec64(dsc_b, qb * BLK, S, vec + 2 * BLK);
  };
  issue(qb0, smem);
  const float gs = batch_do_scale<NT>(dsc_b, S, red);
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
    wait_vm<0>();
    tile_barrier();
    if (qb + 1 < nqb) issue(qb + 1, smem + ((qb + 1 - qb0) & 1) * BUF);
    const _Float16* buf = smem + ((qb - qb0) & 1) * BUF;
    if (qb * BLK + BLK - 1 < k0) continue;  // every query before every key of the wave
    const _Float16* Qs = buf;
    const _Float16* Ds = buf + TILE;
    const float* lse_s = reinterpret_cast<const float*>(buf + 2 * TILE);
    const float* del_s = lse_s + BLK;
    const float* dsc_s = lse_s + 2 * BLK;
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
    // every query of the tile >= every key of the wave and < S: no mask
    if (qb * BLK >= k0 + 15 && qb * BLK + BLK <= S)
      ds_tile_kv<false>(p, ds, lse_s, del_s, dsc_s, sl2, gs, qb * BLK, key, S, lane);
    else
      ds_tile_kv<true>(p, ds, lse_s, del_s, dsc_s, sl2, gs, qb * BLK, key, S, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const half8 pb = pair_frag(p[2 * j], p[2 * j + 1]);
      const half8 db = pair_frag(ds[2 * j], ds[2 * j + 1]);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        dvT[dt] = mfma16(frag_tr(Ds, dt * 16, j, lane), pb, dvT[dt]);
        dkT[dt] = mfma16(frag_tr(Qs, dt * 16, j, lane), db, dkT[dt]);
      }
    }
  }
  if (key < S) {
    const float inv = 1.0f / gs;
    const float fk = a.sm_scale * inv;
    const long long ldp = 2LL * a.nq * HD;
    float* dk = a.dkvp + (rowb + key) * ldp + h * HD;
    float* dv = a.dkvp + (rowb + key) * ldp + (a.nq + h) * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      *reinterpret_cast<float4*>(dk + dt * 16 + 4 * g) =
          make_float4(dkT[dt][0] * fk, dkT[dt][1] * fk, dkT[dt][2] * fk, dkT[dt][3] * fk);
      *reinterpret_cast<float4*>(dv + dt * 16 + 4 * g) =
          make_float4(dvT[dt][0] * inv, dvT[dt][1] * inv, dvT[dt][2] * inv, dvT[dt][3] * inv);
    }
  }
}

// The whole attention backward of a launch: blocks [0, nkvb) of x are dK/dV
// key blocks (most work first), the next nqb dQ query blocks (last, i.e.
// longest, first).  The two halves share no outputs, so one launch runs
// them side by side; a launch with nkvb or nqb = 0 runs one half.
constexpr int BWD_SMEM = 2 * KV_BUF > 4 * TILE ? 2 * KV_BUF : 4 * TILE;

// PART 0: both halves; 1: dK/dV only (nqb = 0); 2: dQ only (nkvb = 0) --
// the one-half forms keep their own (smaller) register and LDS budgets.
template <int NW, int RW, int PART>
__global__ __launch_bounds__(NW * 64) void attn_bwd_kernel(const AttnArgs a, int nkvb, int nqb) {
  constexpr int SMEM = PART == 1 ? 2 * KV_BUF : PART == 2 ? 4 * TILE : BWD_SMEM;
  __shared__ __attribute__((aligned(1024))) _Float16 smem[SMEM];
  __shared__ float red[NW];
  const int x = blockIdx.x;
  if constexpr (PART != 2) {
    if (PART == 1 || x < nkvb) {
      dkdv_block<NW>(a, smem, red, x, blockIdx.y, blockIdx.z);
      return;
    }
  }
  if constexpr (PART != 1) dq_block<NW, RW>(a, smem, nqb - 1 - (x - nkvb), blockIdx.y, blockIdx.z);
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

// Per token row, one wave per head: delta[b, h, s] = sum_d dO * O, and
// dO16 = fp16(dO * sc) with sc the power-of-two scale of the head's max |dO|,
// dsc[b, h, s] = 1 / sc (0 for an all-zero head row).
__global__ __launch_bounds__(256) void attn_delta_kernel(const float* __restrict__ dO, long long ldd,
                                                         const _Float16* __restrict__ o,
                                                         long long ldo, int nq, int S,
                                                         float* __restrict__ delta,
                                                         _Float16* __restrict__ dO16,
                                                         long long ld16, float* __restrict__ dsc) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = t / S, s = t - b * S;
  for (int h = w; h < nq; h += 4) {
    const float* d = dO + (long long)t * ldd + h * HD;
    const _Float16* oo = o + (long long)t * ldo + h * HD;
    const float d0 = d[lane], d1 = d[lane + 64];
    const float v = wave_sum(d0 * (float)oo[lane] + d1 * (float)oo[lane + 64]);
    const float amax = wave_max(fmaxf(fabsf(d0), fabsf(d1)));
    const float sc = pow2_scale_for(amax, kDoScaleExp);
    const long long bhs = ((long long)b * nq + h) * S + s;
    if (lane == 0) {
      delta[bhs] = v;
      dsc[bhs] = pow2_inv_scale_for(amax, kDoScaleExp);
    }
    _Float16* d16 = dO16 + (long long)t * ld16 + h * HD;
    d16[lane] = (_Float16)(d0 * sc);
    d16[lane + 64] = (_Float16)(d1 * sc);
  }
}

// Launch shape: NW waves of RW 16-row tiles.  Two tiles a wave halve the LDS
// operand reads per MFMA; fewer, smaller workgroups keep short sequences
// spread over the CUs.  LLMT_ATTN_CFG = "NW,RW" (NW 2 or 4, RW 1 or 2)
// overrides the forward / dQ shape for tuning.
struct AttnShape {
  int nw, rw;
};
AttnShape attn_shape(int B, int S, int nq) {
  const char* e = getenv("LLMT_ATTN_CFG");
  if (e && (e[0] == '2' || e[0] == '4') && e[1] == ',' && (e[2] == '1' || e[2] == '2') && !e[3])
    return {e[0] - '0', e[2] - '0'};
  const long long heads = (long long)B * nq;
  if (heads * ((S + 127) / 128) >= 512) return {4, 2};
  if (heads * ((S + 63) / 64) >= 256) return {4, 1};
  return {2, 1};
}
int dkdv_waves(int B, int S, int nq) {
  const char* e = getenv("LLMT_ATTN_DKDV_WAVES");
  if (e && (e[0] == '2' || e[0] == '4') && !e[1]) return e[0] - '0';
  return (long long)B * nq * ((S + 63) / 64) >= 256 ? 4 : 2;
}

template <int NW, int RW>
void launch_fwd(const AttnArgs& a, int B, hipStream_t st) {
  constexpr int QB = NW * RW * 16;
  hipLaunchKernelGGL((attn_fwd_kernel<NW, RW>), dim3((a.S + QB - 1) / QB, a.nq, B), dim3(NW * 64),
                     0, st, a);
}
template <int NW, int RW, int PART>
void launch_bwd(const AttnArgs& a, int B, int nkvb, int nqb, hipStream_t st) {
  hipLaunchKernelGGL((attn_bwd_kernel<NW, RW, PART>), dim3(nkvb + nqb, a.nq, B), dim3(NW * 64), 0,
                     st, a, nkvb, nqb);
}
// dK/dV key blocks of nwk waves and dQ query blocks of nwq waves x rw tiles:
// one launch when the wave counts agree and the halves are small (each
// under 2048 workgroups: the second launch would mostly wait on the first's
// tail), else one launch each (measured 5% faster at B4 x S2048).
void launch_attn_bwd(const AttnArgs& a, int B, int nwk, int nwq, int rw, hipStream_t st) {
  const int nkvb = (a.S + nwk * 16 - 1) / (nwk * 16);
  const int nqb = (a.S + nwq * rw * 16 - 1) / (nwq * rw * 16);
  const bool small = (long long)nkvb * a.nq * B < 2048;
  if (nwk == nwq && small) {
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

hipError_t attn_delta(const float* dO, long long ldd, const _Float16* o, long long ldo, int nq,
                      int S, int T, float* delta, _Float16* dO16, long long ld16, float* dsc,
                      hipStream_t st) {
  hipLaunchKernelGGL(attn_delta_kernel, dim3(T), dim3(256), 0, st, dO, ldd, o, ldo, nq, S, delta,
                     dO16, ld16, dsc);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t attn_fwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0) {
    set_error("attn_fwd: nq=%d nkv=%d S=%d", a.nq, a.nkv, a.S);
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

hipError_t attn_bwd(const AttnArgs& a, int B, hipStream_t st) {
  if (a.nq % a.nkv || a.S <= 0 || !a.dkvp || !a.dO16 || !a.dsc) {
    set_error("attn_bwd: nq=%d nkv=%d S=%d (dK/dV share, fp16 dO and its scales required)", a.nq,
              a.nkv, a.S);
    return hipErrorInvalidValue;
  }
  // dQ holds twice the accumulators of the forward: one 16-row tile a wave
  // keeps two waves per SIMD (two tiles spill to one), measured faster at
  // every S; LLMT_ATTN_CFG still selects any shape for tuning.
  AttnShape s = attn_shape(B, a.S, a.nq);
  if (!getenv("LLMT_ATTN_CFG")) s.rw = 1;
  launch_attn_bwd(a, B, dkdv_waves(B, a.S, a.nq), s.nw, s.rw, st);
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
