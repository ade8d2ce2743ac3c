// attn_common.h — shared pieces of the attention kernels (attn.hip: forward
// and the dO operand preparation; attn_bwd.hip: the backward): LDS tile
// layout, DMA of 64-row tiles, MFMA fragment reads and the launch shape.
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
// (buffer range check).
#pragma once

#include <stdlib.h>

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

// Per-head RMSNorm + half-split RoPE of one 128-wide row (the block API's
// QK-norm, src/kernels/rmsnorm.cu:36-41 and src/kernels/rope.cu:7-27) as an
// MFMA operand: lane (c, g) of the four lanes c + 16 g holding the row gets
// y = fp16(rope(x * r * w)) at halves 32 ks + 8 g .. + 7 in y[ks], r =
// rsqrt(mean x^2 + eps), position pos.  Every lane of the wave must call it
// (the row sum crosses lanes).
__device__ __forceinline__ void norm_rope_frag(half8 (&y)[4], const _Float16* x, const float* w,
                                               const float* cosT, const float* sinT, int pos,
                                               float eps, int g) {
  float a[4][8];
  float ss = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const half8 h = *reinterpret_cast<const half8*>(x + 32 * ks + 8 * g);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[ks][i] = (float)h[i];
      ss += a[ks][i] * a[ks][i];
    }
  }
  const float r = rsqrtf(xg_sum(ss) / HD + eps);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int i = 0; i < 8; ++i) a[ks][i] = a[ks][i] * r * w[32 * ks + 8 * g + i];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = 32 * ks + 8 * g + i;
      const float cs = cosT[pos * (HD / 2) + d], sn = sinT[pos * (HD / 2) + d];
      y[ks][i] = (_Float16)(a[ks][i] * cs - a[ks + 2][i] * sn);
      y[ks + 2][i] = (_Float16)(a[ks + 2][i] * cs + a[ks][i] * sn);
    }
}

// Backward of the same map for one row held as accumulator columns: lane
// (c, g) has dy at dims 16 d + 4 g + v in dy[d][v] (d < 8); on return dx of
// the raw input x there (src/kernels/rope.cu:57-89, then
// src/kernels/rmsnorm.cu:53-95 over 128-wide rows):
//   n = rope^T(dy); dx = r (n w - (r^2 / 128) sum(n w x) x).
// Every lane of the wave must call it.
__device__ __forceinline__ void norm_rope_bwd_row(float (&dy)[8][4], const _Float16* x,
                                                  const float* w, const float* cosT,
                                                  const float* sinT, int pos, float eps, int g) {
  float xv[8][4], wv[8][4], n[8][4];
  float ss = 0.f, dot = 0.f;
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const half4v h = *reinterpret_cast<const half4v*>(x + 16 * d + 4 * g);
    const float4 ww = *reinterpret_cast<const float4*>(w + 16 * d + 4 * g);
    wv[d][0] = ww.x; wv[d][1] = ww.y; wv[d][2] = ww.z; wv[d][3] = ww.w;
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[d][v] = (float)h[v];
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float4 c4 = *reinterpret_cast<const float4*>(cosT + pos * (HD / 2) + 16 * d + 4 * g);
    const float4 s4 = *reinterpret_cast<const float4*>(sinT + pos * (HD / 2) + 16 * d + 4 * g);
    const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      n[d][v] = dy[d][v] * cs[v] + dy[d + 4][v] * sn[v];
      n[d + 4][v] = dy[d + 4][v] * cs[v] - dy[d][v] * sn[v];
    }
  }
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      ss += xv[d][v] * xv[d][v];
      dot += n[d][v] * wv[d][v] * xv[d][v];
    }
  const float r = rsqrtf(xg_sum(ss) / HD + eps);
  const float coef = r * r / HD * xg_sum(dot);
#pragma unroll
  for (int d = 0; d < 8; ++d)
#pragma unroll
    for (int v = 0; v < 4; ++v) dy[d][v] = r * (n[d][v] * wv[d][v] - coef * xv[d][v]);
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

// Scheduling of a straight-line block of NR LDS reads feeding NM MFMAs (the
// gfx950 backend's sched_group_barrier): RA reads issued ahead, then groups
// of MP MFMAs each followed by the next DP reads, then the remaining MFMAs.
// The default schedule waits on each read right before its MFMA; running the
// reads ahead hides the LDS latency behind the MFMAs already issued.
constexpr int SG_MFMA = 0x008, SG_DSR = 0x100;
template <int NR, int NM, int RA, int MP, int DP, int ID>
__device__ __forceinline__ void sched_reads_ahead() {
  static_assert(RA <= NR && (NR - RA) % DP == 0 && (NR - RA) / DP * MP <= NM, "schedule shape");
  __builtin_amdgcn_sched_group_barrier(SG_DSR, RA, ID);
#pragma unroll
  for (int i = 0; i < (NR - RA) / DP; ++i) {
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, MP, ID);
    __builtin_amdgcn_sched_group_barrier(SG_DSR, DP, ID);
  }
  __builtin_amdgcn_sched_group_barrier(SG_MFMA, NM - (NR - RA) / DP * MP, ID);
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

}  // namespace

}  // namespace llmt
