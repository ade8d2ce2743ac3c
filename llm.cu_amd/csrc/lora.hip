// lora.hip — rank-16 adapter kernels: the dA/dB reductions over tokens, one
// multi-tensor AdamW over the whole fp32 adapter arena (which also refreshes
// the fp16 operand copies the GEMMs read), and the seeded initialiser.
//
// Reference: LoRA grads src/kernels/lora_backward.cu:50-90 (two TN GEMMs per
// adapter through matmul_tn_forward, src/kernels/matmul.cu:102-138, plus
// scale_add_inplace, src/kernels/lora.cu:10-18); AdamW
// src/kernels/lora.cu:206-246 (224 launches per step); init
// src/kernels/lora.cu:32-62 (cuRAND, not reproduced: this library draws its
// own seeded normals).
#include <algorithm>

#include "ops.h"

namespace llmt {

namespace {

constexpr int R = 16;
constexpr int NTH = 256;

// One adapter-gradient job: out = (acc ? out : 0) + lscale * X^T G over the T
// token rows, for the ncols columns of X and the 16 columns of G.
//   dA [16, d_in]:  X = adapter input (xn or o, fp16), G = dh  -> out[r][c]
//   dB [d_out, 16]: X = upstream grad dy,              G = h   -> out[c][r]
// (dy as the fp16 GEMM operand, row t scaled by the power of two 1 / xs[t],
// which the G row takes back exactly).  A workgroup owns GC columns of one
// job.
constexpr int GC = 256;

struct LoraGradGrid {
  int block_start[kLoraJobs + 1];  // column blocks of each job within a layer
};

// The reduction on the matrix cores in fp32 (v_mfma_f32_16x16x4_f32:
// out[r][c] = sum over 4 tokens k of G[k][r] X[k][c], so no operand needs a
// transposition): a workgroup of four waves owns GC columns, wave w the 64
// columns cb + 64 w .., every wave all T tokens (no cross-wave sum).  Lane
// l reads G[t + l / 16][l % 16] (times the row factor) as its A value and
// four consecutive fp16 columns cb + 64 w + 4 (l % 16) .. of X[t + l / 16]
// as its B values of the four MFMA column tiles (tile nb, MFMA column n
// stands for column 4 n + nb), so both loads are contiguous rows and each
// output lane ends up with four consecutive columns or ranks to store.
template <bool F16>
__device__ __forceinline__ float4 load_x4s(const void* X, long long off);
template <>
__device__ __forceinline__ float4 load_x4s<true>(const void* X, long long off) {
  const half4 h = *reinterpret_cast<const half4*>((const _Float16*)X + off);
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}
template <>
__device__ __forceinline__ float4 load_x4s<false>(const void* X, long long off) {
  return *reinterpret_cast<const float4*>((const float*)X + off);
}

constexpr int MG_U = 4;  // token quads a wave loads ahead

template <bool F16>
__device__ __forceinline__ void lora_grad_mfma_acc(const LoraGradJob& jb, int T, int col,
                                                   floatx4 (&acc)[4]) {
  const int lane = threadIdx.x & 63, kq = lane >> 4, r = lane & 15;
  float gv[MG_U];
  float4 xv[MG_U];
  auto load = [&](int t0) {
#pragma unroll
    for (int u = 0; u < MG_U; ++u) {
      const int t = t0 + 4 * u + kq;
      const int tc = min(t, T - 1);
      const float f = t < T ? (jb.xs ? jb.xs[tc] : 1.0f) : 0.f;
      gv[u] = jb.G[(long long)tc * jb.ldg + r] * f;
      xv[u] = load_x4s<F16>(jb.X, (long long)tc * jb.ldx + col);
    }
  };
  load(0);
  for (int t0 = 0; t0 < T; t0 += 4 * MG_U) {
    float g_c[MG_U];
    float4 x_c[MG_U];
#pragma unroll
    for (int u = 0; u < MG_U; ++u) {
      g_c[u] = gv[u];
      x_c[u] = xv[u];
    }
    if (t0 + 4 * MG_U < T) load(t0 + 4 * MG_U);
#pragma unroll
    for (int u = 0; u < MG_U; ++u) {
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u].x, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u].y, acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u].z, acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u].w, acc[3], 0, 0, 0);
    }
  }
}

__global__ __launch_bounds__(NTH) void lora_grad_mfma_kernel(const LoraGradJob* __restrict__ jobs,
                                                             const LoraGradGrid G, int T,
                                                             float lscale, int accumulate) {
  const int bpl = G.block_start[kLoraJobs];
  const int layer = (int)blockIdx.x / bpl, lb = (int)blockIdx.x - layer * bpl;
  int j = 0;
#pragma unroll
  for (int i = 1; i < kLoraJobs; ++i)
    if (lb >= G.block_start[i]) j = i;
  const LoraGradJob jb = jobs[layer * kLoraJobs + j];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = (lb - G.block_start[j]) * GC + 64 * w + 4 * (lane & 15);  // this lane's columns
  if ((lb - G.block_start[j]) * GC + 64 * w >= jb.ncols) return;           // wave-uniform
  const int cc = c < jb.ncols ? c : 0;
  floatx4 acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (jb.x_f16)
    lora_grad_mfma_acc<true>(jb, T, cc, acc);
  else
    lora_grad_mfma_acc<false>(jb, T, cc, acc);
  if (c >= jb.ncols) return;
  // lane: ranks 4 (l / 16) + i of MFMA column l % 16, i.e. columns c .. c + 3
  const int r0 = 4 * (lane >> 4);
  if (jb.out_is_B) {  // out[col][16]: four consecutive ranks of each column
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float4* o = reinterpret_cast<float4*>(jb.out + (long long)(c + nb) * R + r0);
      const float4 prev = accumulate ? *o : make_float4(0.f, 0.f, 0.f, 0.f);
      *o = make_float4(prev.x + lscale * acc[nb][0], prev.y + lscale * acc[nb][1],
                       prev.z + lscale * acc[nb][2], prev.w + lscale * acc[nb][3]);
    }
  } else {  // out[16][ncols]: four consecutive columns of each rank
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float4* o = reinterpret_cast<float4*>(jb.out + (long long)(r0 + i) * jb.ncols + c);
      const float4 prev = accumulate ? *o : make_float4(0.f, 0.f, 0.f, 0.f);
      *o = make_float4(prev.x + lscale * acc[0][i], prev.y + lscale * acc[1][i],
                       prev.z + lscale * acc[2][i], prev.w + lscale * acc[3][i]);
    }
  }
}

// Long token ranges: wave w of the four takes token quads w, w + 4, .. for
// all GC columns of the block (16 MFMA tiles: column group cg of 64, tile
// nb), loads MG2_U quads ahead, and the four partial 16 x GC blocks are added
// in LDS in wave order.
constexpr int MG2_U = 4;

template <bool F16>
__device__ __forceinline__ void lora_grad_mfma2_acc(const LoraGradJob& jb, int T, int cb, int w,
                                                    floatx4 (&acc)[4][4]) {
  const int lane = threadIdx.x & 63, kq = lane >> 4, r = lane & 15;
  const int nq = (T + 3) / 4;
  if (w >= nq) return;
  int colc[4];
#pragma unroll
  for (int cg = 0; cg < 4; ++cg) colc[cg] = min(cb + 64 * cg + 4 * r, jb.ncols - 4);
  float gv[MG2_U];
  float4 xv[MG2_U][4];
  auto load = [&](int q0) __attribute__((always_inline)) {  // quads q0, q0 + 4, ..
#pragma unroll
    for (int u = 0; u < MG2_U; ++u) {
      const int t = 4 * (q0 + 4 * u) + kq;
      const int tc = min(t, T - 1);
      const float f = t < T ? (jb.xs ? jb.xs[tc] : 1.0f) : 0.f;
      gv[u] = jb.G[(long long)tc * jb.ldg + r] * f;
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) xv[u][cg] = load_x4s<F16>(jb.X, (long long)tc * jb.ldx + colc[cg]);
    }
  };
  load(w);
  for (int q0 = w; q0 < nq; q0 += 4 * MG2_U) {
    float g_c[MG2_U];
    float4 x_c[MG2_U][4];
#pragma unroll
    for (int u = 0; u < MG2_U; ++u) {
      g_c[u] = gv[u];
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) x_c[u][cg] = xv[u][cg];
    }
    if (q0 + 4 * MG2_U < nq) load(q0 + 4 * MG2_U);
    // quads past nq carry a zero G value (t >= T), so they add nothing
#pragma unroll
    for (int u = 0; u < MG2_U; ++u)
#pragma unroll
      for (int cg = 0; cg < 4; ++cg) {
        acc[cg][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u][cg].x, acc[cg][0], 0, 0, 0);
        acc[cg][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u][cg].y, acc[cg][1], 0, 0, 0);
        acc[cg][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u][cg].z, acc[cg][2], 0, 0, 0);
        acc[cg][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(g_c[u], x_c[u][cg].w, acc[cg][3], 0, 0, 0);
      }
  }
}

__global__ __launch_bounds__(NTH) void lora_grad_mfma2_kernel(const LoraGradJob* __restrict__ jobs,
                                                              const LoraGradGrid G, int T,
                                                              float lscale, int accumulate) {
  const int bpl = G.block_start[kLoraJobs];
  const int layer = (int)blockIdx.x / bpl, lb = (int)blockIdx.x - layer * bpl;
  int j = 0;
#pragma unroll
  for (int i = 1; i < kLoraJobs; ++i)
    if (lb >= G.block_start[i]) j = i;
  const LoraGradJob jb = jobs[layer * kLoraJobs + j];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int cb = (lb - G.block_start[j]) * GC;
  floatx4 acc[4][4];
#pragma unroll
  for (int cg = 0; cg < 4; ++cg)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[cg][nb] = floatx4{0.f, 0.f, 0.f, 0.f};
  if (jb.x_f16)
    lora_grad_mfma2_acc<true>(jb, T, cb, w, acc);
  else
    lora_grad_mfma2_acc<false>(jb, T, cb, w, acc);
  // partial [16 ranks][GC columns] of each wave; column 4 n + nb of group cg
  __shared__ float red[4][R][GC];
  const int r0 = 4 * (lane >> 4), n = lane & 15;
#pragma unroll
  for (int cg = 0; cg < 4; ++cg)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<float4*>(&red[w][r0 + i][64 * cg + 4 * n]) =
          make_float4(acc[cg][0][i], acc[cg][1][i], acc[cg][2][i], acc[cg][3][i]);
  __syncthreads();
  // thread i finishes column cb + i (all 16 ranks), the waves in order
  const int col = cb + (int)threadIdx.x;
  if (col >= jb.ncols) return;
#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    float v = red[0][rr][threadIdx.x];
#pragma unroll
    for (int q = 1; q < 4; ++q) v += red[q][rr][threadIdx.x];
    float* o = jb.out_is_B ? jb.out + (long long)col * R + rr : jb.out + (long long)rr * jb.ncols + col;
    *o = (accumulate ? *o : 0.f) + lscale * v;
  }
}

// Arena element i -> (shadow block offset within the layer, row, column,
// row length) of its fp16 copies; the packed copy (a GEMM B operand) holds it
// at packed_index(row, col, len), the row-major twin at row * len + col.
struct ShadowPos {
  long long base;  // layer base + block offset
  long long row, col;
  int len;
};
__device__ __forceinline__ ShadowPos shadow_pos(const AdamShadow& sh, long long i) {
  const long long l = i / sh.per_layer;
  long long j = i - l * sh.per_layer;
  int s = 0;
#pragma unroll
  for (int k = 1; k < 8; ++k)
    if (j >= sh.seg_off[k]) s = k;
  j -= sh.seg_off[s];
  const int p = s >> 1;  // q, k, v, o
  const long long base = l * sh.shadow_per_layer;
  if ((s & 1) == 0) {  // A [16, d_in]: row r, column cc
    const int d_in = sh.d_in[p];
    const long long r = j / d_in, cc = j - r * d_in;
    if (p < 3) return {base + sh.a_qkv, p * R + r, cc, d_in};
    return {base + sh.a_o, r, cc, d_in};
  }
  // B [d_out, 16]: element (o, r) -> row r, column o of B^T
  const long long o = j / R, r = j - o * R;
  if (p < 3) return {base + sh.bt_qkv, p * R + r, sh.col_off[p] + o, sh.nt};
  return {base + sh.bt_o, r, o, sh.d_out[3]};
}
__device__ __forceinline__ void shadow_store(const AdamShadow& sh, long long i, float v) {
  const ShadowPos q = shadow_pos(sh, i);
  const _Float16 h = (_Float16)v;
  sh.shadow[q.base + packed_index(q.row, q.col, q.len)] = h;
  sh.rm[q.base + q.row * q.len + q.col] = h;
  if (sh.at) {  // A of q, k, v: also at (layer, column, row) of the transposed copy
    const long long l = i / sh.per_layer, j = i - l * sh.per_layer;
    if (j < sh.seg_off[5] && (j < sh.seg_off[1] || (j >= sh.seg_off[2] && j < sh.seg_off[3]) ||
                              j >= sh.seg_off[4]))
      sh.at[(l * sh.d_in[0] + q.col) * (3 * R) + q.row] = h;
  }
}

// The AdamW update of one element (src/kernels/lora.cu:206-220):
//   m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g^2;
//   p = p (1 - lr wd) - lr (m / bc1) / (sqrt(v / bc2) + eps).
// The bias corrections enter as reciprocals taken once (ib1 = 1 / bc1,
// ib2 = 1 / bc2), and the square root and the last reciprocal are the
// hardware v_sqrt_f32 / v_rcp_f32 (1 ulp each): the IEEE division and
// square-root sequences had made the kernel VALU-bound (about 200 VALU
// instructions a thread for four elements).  The update differs from the
// correctly rounded formula by a few ulp of itself.
struct AdamCoef {
  float b1, b2, c1, c2, ib1, ib2, decay, lr, eps;
};
__device__ __forceinline__ AdamCoef adam_coef(const AdamHp& hp) {
  return {hp.beta1, hp.beta2, 1.0f - hp.beta1, 1.0f - hp.beta2, 1.0f / hp.bc1, 1.0f / hp.bc2,
          1.0f - hp.lr * hp.wd, hp.lr, hp.eps};
}
__device__ __forceinline__ float adam_update(const AdamCoef& k, float p, float g, float& m,
                                             float& v) {
  m = k.b1 * m + k.c1 * g;
  v = k.b2 * v + k.c2 * g * g;
  const float denom = __builtin_amdgcn_sqrtf(v * k.ib2) + k.eps;
  return p * k.decay - k.lr * (m * k.ib1) * __builtin_amdgcn_rcpf(denom);
}

// One AdamW element update in place; returns the new parameter.
__device__ __forceinline__ float adamw_elem(float* __restrict__ p, const float* __restrict__ g,
                                            float* __restrict__ m, float* __restrict__ v,
                                            long long i, const AdamCoef& k) {
  float mi = m[i], vi = v[i];
  const float pi = adam_update(k, p[i], g[i], mi, vi);
  m[i] = mi;
  v[i] = vi;
  p[i] = pi;
  return pi;
}

// Any contiguous set of parameters, no shadows.
__global__ __launch_bounds__(NTH) void adamw_kernel(float* __restrict__ p,
                                                    const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v,
                                                    long long n,
                                                    const AdamHp* __restrict__ hpp) {
  const AdamCoef k = adam_coef(*hpp);
  for (long long i = (long long)blockIdx.x * NTH + threadIdx.x; i < n;
       i += (long long)gridDim.x * NTH)
    adamw_elem(p, g, m, v, i, k);
}

// The whole arena with its fp16 shadows, one launch: blockIdx.y = layer x 8
// + segment (q, k, v, o x A, B), blockIdx.x = a tile of kTile elements of
// that segment, so every block knows where its elements' shadow rows and
// columns are (32-bit index math only).  A thread moves four elements as
// 16-byte loads and stores of p, g, m, v (one 16-byte piece a thread over
// many blocks keeps the DRAM streams dense: a copy in this form measured
// 6.3 TB/s on MI355X against 4.6-5.6 TB/s grid-stride; here nontemporal
// loads and stores measured slower, 43 against 37 us).  Each tile covers
// the 16 shadow rows x 64 columns of two whole fragment-packed 16 x 32
// blocks, so a block writes complete 1 KB packed blocks and 128-byte pieces
// of the row-major twin (the same kernel over linear half-row tiles, whose
// packed stores leave partial lines, took 41 us):
// an A tile is rows r = 0..15 x columns c0 .. c0 + 63 of A (16 pieces of
// 256 bytes of the arena; thread = row t / 16, four columns); a B tile is
// the 64 rows o0 .. o0 + 63 of B [d_out, 16] (contiguous in the arena),
// transposed through LDS so that each thread stores four consecutive
// columns o of one row r of B^T.  update = 0 only refreshes the shadows
// from the parameters.
constexpr int kTile = 4 * NTH;
// Tiles a block (TPB): two where every segment is an even number of tiles
// (eight elements a thread, all 32 loads issued before the arithmetic:
// 37.3 against 37.9 us at one and 39 us at four), else one.

__device__ __forceinline__ floatx4 ld4v(const float* p) {
  return *reinterpret_cast<const floatx4*>(p);
}
__device__ __forceinline__ void st4v(float* p, floatx4 v) {
  *reinterpret_cast<floatx4*>(p) = v;
}

template <int TPB>
__global__ __launch_bounds__(NTH) void adamw_shadow_kernel(float* __restrict__ p,
                                                           const float* __restrict__ g,
                                                           float* __restrict__ m,
                                                           float* __restrict__ v,
                                                           const AdamHp* __restrict__ hpp,
                                                           int update, const AdamShadow sh) {
  __shared__ _Float16 bt[TPB][R][64 + 4];
  const int l = blockIdx.y >> 3, s = blockIdx.y & 7, q = s >> 1;
  const int n = (int)((s < 7 ? sh.seg_off[s + 1] : sh.per_layer) - sh.seg_off[s]);
  if (blockIdx.x * TPB * kTile >= n) return;
  const bool is_b = s & 1;
  // A: element (r, c0 + 4 (t % 16)) with r = t / 16; B: elements 4 t .. of the tile
  const int a_len = sh.d_in[q];
  const int ar = threadIdx.x >> 4;
  long long i[TPB];
  floatx4 pv[TPB];
#pragma unroll
  for (int u = 0; u < TPB; ++u) {
    const int tx = blockIdx.x * TPB + u;
    const int ac = tx * 64 + 4 * (threadIdx.x & 15);
    const int jt = is_b ? tx * kTile + 4 * threadIdx.x : ar * a_len + ac;
    i[u] = (long long)l * sh.per_layer + sh.seg_off[s] + jt;
    pv[u] = ld4v(p + i[u]);
  }
  if (update) {
    floatx4 gv[TPB], mv[TPB], vv[TPB];
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
      gv[u] = ld4v(g + i[u]);
      mv[u] = ld4v(m + i[u]);
      vv[u] = ld4v(v + i[u]);
    }
    const AdamCoef k = adam_coef(*hpp);
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float me = mv[u][e], ve = vv[u][e];
        pv[u][e] = adam_update(k, pv[u][e], gv[u][e], me, ve);
        mv[u][e] = me;
        vv[u][e] = ve;
      }
      st4v(p + i[u], pv[u]);
      st4v(m + i[u], mv[u]);
      st4v(v + i[u], vv[u]);
    }
  }
  const long long lb = (long long)l * sh.shadow_per_layer;
  if (!is_b) {
    // A [16, d_in]: element (r, c) -> row row0 + r, column c (row length d_in)
    const int row = (q < 3 ? q * R : 0) + ar;
    const long long base = lb + (q < 3 ? sh.a_qkv : sh.a_o);
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
      const int ac = (blockIdx.x * TPB + u) * 64 + 4 * (threadIdx.x & 15);
      const half4 h = {(_Float16)pv[u][0], (_Float16)pv[u][1], (_Float16)pv[u][2],
                       (_Float16)pv[u][3]};
      *reinterpret_cast<half4*>(sh.shadow + base + packed_index(row, ac, a_len)) = h;
      *reinterpret_cast<half4*>(sh.rm + base + (long long)row * a_len + ac) = h;
    }
    if (q == 3 || !sh.at) return;  // block-uniform
    // q, k, v: the transposed copy [column][3 R], through LDS: thread t then
    // stores ranks 4 (t % 4) .. of column t / 4 of the tile (8 bytes)
    __shared__ _Float16 at_t[TPB][64][R + 4];
#pragma unroll
    for (int u = 0; u < TPB; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) at_t[u][4 * (threadIdx.x & 15) + e][ar] = (_Float16)pv[u][e];
    __syncthreads();
    const int oc = threadIdx.x >> 2, orq = 4 * (threadIdx.x & 3);
#pragma unroll
    for (int u = 0; u < TPB; ++u) {
      const int col = (blockIdx.x * TPB + u) * 64 + oc;
      const half4 t = {at_t[u][oc][orq], at_t[u][oc][orq + 1], at_t[u][oc][orq + 2],
                       at_t[u][oc][orq + 3]};
      *reinterpret_cast<half4*>(sh.at + ((long long)l * a_len + col) * (3 * R) + q * R + orq) = t;
    }
    return;
  }
  // B [d_out, 16]: element j = (o, r) -> row row0 + r, column col0 + o of
  // B^T (row length len); tile u holds o in [64 tx, 64 tx + 64)
  {
    const int o = threadIdx.x >> 2, r = 4 * (threadIdx.x & 3);
#pragma unroll
    for (int u = 0; u < TPB; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) bt[u][r + e][o] = (_Float16)pv[u][e];
  }
  __syncthreads();
  const int len = q < 3 ? sh.nt : sh.d_out[3];
  const int r = threadIdx.x >> 4, c4 = 4 * (threadIdx.x & 15);
  const int row = (q < 3 ? q * R : 0) + r;
  const long long base = lb + (q < 3 ? sh.bt_qkv : sh.bt_o);
#pragma unroll
  for (int u = 0; u < TPB; ++u) {
    const int col = (q < 3 ? sh.col_off[q] : 0) + 64 * (blockIdx.x * TPB + u) + c4;
    const half4 t = *reinterpret_cast<const half4*>(&bt[u][r][c4]);
    *reinterpret_cast<half4*>(sh.shadow + base + packed_index(row, col, len)) = t;
    *reinterpret_cast<half4*>(sh.rm + base + (long long)row * len + col) = t;
  }
}

// Counter-based normal draws: SplitMix64 of (seed, index) -> two 24-bit
// uniforms -> Box-Muller.  Deterministic for a given seed regardless of the
// launch shape.
__device__ __forceinline__ unsigned long long splitmix64(unsigned long long x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__global__ __launch_bounds__(NTH) void lora_init_kernel(float* __restrict__ p,
                                                        float* __restrict__ m,
                                                        float* __restrict__ v, long long n,
                                                        unsigned long long seed, float a_std,
                                                        float b_std, const AdamShadow sh) {
  for (long long i = (long long)blockIdx.x * NTH + threadIdx.x; i < n;
       i += (long long)gridDim.x * NTH) {
    const unsigned long long z = splitmix64(seed * 0x100000001B3ull + (unsigned long long)i);
    const float u1 = ((float)(z >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    const float u2 = (float)((z >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
    const float nrm = sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
    const long long j = i % sh.per_layer;
    int s = 0;
#pragma unroll
    for (int k = 1; k < 8; ++k)
      if (j >= sh.seg_off[k]) s = k;
    const float val = nrm * ((s & 1) ? b_std : a_std);
    p[i] = val;
    m[i] = 0.f;
    v[i] = 0.f;
    if (sh.shadow) shadow_store(sh, i, val);
  }
}

inline unsigned grid_for(long long n) {
  long long g = (n + NTH - 1) / NTH;
  return (unsigned)(g > 8192 ? 8192 : (g < 1 ? 1 : g));
}

}  // namespace

hipError_t lora_grad(const LoraGradJob* jobs, const LoraGradPlan& plan, int layers, int T,
                     float lscale, int accumulate, hipStream_t st) {
  if (layers < 1 || T < 1) {
    set_error("lora_grad: %d layers, T=%d", layers, T);
    return hipErrorInvalidValue;
  }
  for (int i = 0; i < kLoraJobs; ++i)
    if (plan.ncols[i] % 4) {
      set_error("lora_grad: job %d has %d columns (a multiple of 4 is required)", i, plan.ncols[i]);
      return hipErrorInvalidValue;
    }
  LoraGradGrid G{};
  for (int i = 0; i < kLoraJobs; ++i)
    G.block_start[i + 1] = G.block_start[i] + (plan.ncols[i] + GC - 1) / GC;
  const dim3 grid(layers * G.block_start[kLoraJobs]);
  // short token ranges: one wave a 64-column slice over every token (more
  // waves in flight); long ones: four waves a block split the tokens
  // (C4: 0.98 -> 0.86 ms against the fp32 VALU form; C2 57 -> 46 us)
  if (T <= 512)
    hipLaunchKernelGGL(lora_grad_mfma_kernel, grid, dim3(NTH), 0, st, jobs, G, T, lscale, accumulate);
  else
    hipLaunchKernelGGL(lora_grad_mfma2_kernel, grid, dim3(NTH), 0, st, jobs, G, T, lscale, accumulate);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t adamw(float* p, const float* g, float* m, float* v, long long n, const AdamHp* hp,
                 int update, const AdamShadow& sh, hipStream_t st) {
  if (!sh.shadow) {
    if (!update) return hipSuccess;
    hipLaunchKernelGGL(adamw_kernel, dim3(grid_for(n)), dim3(NTH), 0, st, p, g, m, v, n, hp);
    LLMT_LAUNCH_CHECK();
    return hipSuccess;
  }
  if (sh.per_layer <= 0 || n % sh.per_layer || !sh.rm) {
    set_error("adamw: %lld parameters are not whole layers of %lld", n, sh.per_layer);
    return hipErrorInvalidValue;
  }
  // every segment is whole tiles (its A rows and B^T rows a multiple of 64
  // columns, 16-byte aligned), so the tiles never straddle segments
  long long seg = 0;
  bool pairs = true;  // every segment an even number of tiles
  for (int s = 0; s < 8; ++s) {
    const long long ns = (s < 7 ? sh.seg_off[s + 1] : sh.per_layer) - sh.seg_off[s];
    if (ns % kTile || sh.seg_off[s] % 4) {
      set_error("adamw: segment %d of %lld elements is not whole %d-element tiles", s, ns, kTile);
      return hipErrorInvalidValue;
    }
    pairs = pairs && ns % (2 * kTile) == 0;
    seg = std::max(seg, ns);
  }
  for (int q = 0; q < 4; ++q)
    if (sh.d_in[q] % 64 || sh.d_out[q] % 64) {
      set_error("adamw: adapter %d dims %d x %d not multiples of 64", q, sh.d_out[q], sh.d_in[q]);
      return hipErrorInvalidValue;
    }
  const dim3 grid((unsigned)(seg / (pairs ? 2 * kTile : kTile)), (unsigned)(n / sh.per_layer * 8));
  if (pairs)
    hipLaunchKernelGGL(adamw_shadow_kernel<2>, grid, dim3(NTH), 0, st, p, g, m, v, hp, update, sh);
  else
    hipLaunchKernelGGL(adamw_shadow_kernel<1>, grid, dim3(NTH), 0, st, p, g, m, v, hp, update, sh);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t lora_init(float* p, float* m, float* v, long long n, unsigned long long seed,
                     float a_std, float b_std, const AdamShadow& sh, hipStream_t st) {
  hipLaunchKernelGGL(lora_init_kernel, dim3(grid_for(n)), dim3(NTH), 0, st, p, m, v, n, seed,
                     a_std, b_std, sh);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
