// gemm.hip — skinny "NT" GEMM on fp16 MFMA (v_mfma_f32_16x16x32_f16) for
// gfx950, plus the layout kernels (transposes, conversions, the bit-exact
// int8 quantizer).
//
// Every frozen-weight product of the training step is expressed as
// C = A * B^T with both operands contiguous along the reduction dimension:
// the forward uses W [out, in] as B, the backward (dX = dY * W) uses the
// pre-transposed copy W^T [in, out] the library keeps next to W.  This is the
// MI355X-native replacement for the reference's three fp32 32x32-tiled
// kernels (src/kernels/matmul.cu:8-138): matmul_forward (NT), matmul_nn
// (dX) and, for LoRA, matmul_tn.
//
// Work decomposition.  The step's activations have few rows (T = 128 at the
// headline shape), so every weight element is used T times: the kernel is
// HBM-bound on the weight stream.  A workgroup of NW waves owns an
// (MF*16) x (NW*NF*16) output tile over a K range (split-K); the A tile
// [MF*16 x 64] is staged through LDS (double-buffered, padded rows: no bank
// conflicts for ds_read_b128) and shared by the waves; each wave streams its
// own NF*16 weight rows straight from HBM into MFMA operand registers with
// 16-byte loads, one 64-wide K chunk ahead.  Split partials go to an fp32
// workspace and are summed by the consuming epilogue kernel.
#include "ops.h"

namespace llmt {

namespace {

constexpr int BK = 64;
constexpr int LDA_S = BK + 8;  // padded LDS row, in halves (144 B)

// One MFMA B fragment (8 consecutive k of one row).  int8 rows are
// dequantised exactly to fp16 (|q| <= 127); a per-k scale (transposed int8
// weights, where the quantisation channel is the reduction index) is then
// applied as an fp16 multiply.
__device__ __forceinline__ half8 load_b_frag(const void* p, int is_i8, const _Float16* ks) {
  if (!is_i8) return *reinterpret_cast<const half8*>(p);
  const int8x8 q = *reinterpret_cast<const int8x8*>(p);
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (_Float16)(float)q[i];
  if (ks) h = h * *reinterpret_cast<const half8*>(ks);
  return h;
}

template <int MF, int NF, int NW>
__global__ __launch_bounds__(NW * 64) void gemm_nt_kernel(const GemmArgs g) {
  constexpr int MT = MF * 16;
  constexpr int PIECES = MT * (BK / 8);  // 16-byte pieces per A chunk
  constexpr int NT = NW * 64;
  constexpr int APT = (PIECES + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) _Float16 As[2][MT * LDA_S];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m0 = blockIdx.z * MT;
  const int nchunks = g.K / BK;
  const int kc0 = (int)((long long)blockIdx.y * nchunks / g.split);
  const int kc1 = (int)((long long)(blockIdx.y + 1) * nchunks / g.split);

  // Per-fragment B row pointers (a fragment's 16 rows lie in one segment).
  const char* bptr[NF];
  int bi8[NF];
  int ncol[NF];
  const _Float16* cscale[NF];
  const _Float16* kscale[NF];
  bool valid[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int n = (blockIdx.x * NW + wave) * NF * 16 + f * 16;
    ncol[f] = n;
    valid[f] = n < g.N;
    int s = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
      if (i < g.nseg && n >= g.seg_start[i]) s = i;
    const BSeg& sg = g.seg[s];
    const int row = n - g.seg_start[s] + (lane & 15);
    const int esz = sg.is_i8 ? 1 : 2;
    bptr[f] = (const char*)sg.ptr + ((long long)row * sg.ld + (lane >> 4) * 8) * esz;
    bi8[f] = sg.is_i8;
    cscale[f] = sg.colscale ? sg.colscale + (n - g.seg_start[s]) : nullptr;
    kscale[f] = sg.kscale ? sg.kscale + (lane >> 4) * 8 : nullptr;
    if (!valid[f]) bptr[f] = nullptr;
  }

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  half8 breg[NF][2], bnext[NF][2];
  uint4 astage[APT];

  auto load_a = [&](int kc) {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + i * NT;
      if (idx < PIECES) {
        const int r = idx >> 3, c = idx & 7;
        astage[i] = *reinterpret_cast<const uint4*>(g.A + (long long)(m0 + r) * g.lda + kc * BK + c * 8);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + i * NT;
      if (idx < PIECES) {
        const int r = idx >> 3, c = idx & 7;
        *reinterpret_cast<uint4*>(&As[buf][r * LDA_S + c * 8]) = astage[i];
      }
    }
  };
  auto load_b = [&](int kc, half8 (&dst)[NF][2]) {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (valid[f]) {
        const int esz = bi8[f] ? 1 : 2;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          dst[f][kk] = load_b_frag(bptr[f] + (long long)(kc * BK + kk * 32) * esz, bi8[f],
                                   kscale[f] ? kscale[f] + kc * BK + kk * 32 : nullptr);
      }
    }
  };

  if (kc0 < kc1) {
    load_a(kc0);
    store_a(0);
    load_b(kc0, breg);
  }
  int cur = 0;
  for (int kc = kc0; kc < kc1; ++kc) {
    __syncthreads();
    const bool more = kc + 1 < kc1;
    if (more) {
      load_a(kc + 1);
      load_b(kc + 1, bnext);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int mi = 0; mi < MF; ++mi) {
        const half8 a = *reinterpret_cast<const half8*>(
            &As[cur][(mi * 16 + (lane & 15)) * LDA_S + kk * 32 + (lane >> 4) * 8]);
#pragma unroll
        for (int f = 0; f < NF; ++f)
          if (valid[f]) acc[mi][f] = mfma16(a, breg[f][kk], acc[mi][f]);
      }
    }
    if (more) {
      store_a(cur ^ 1);
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        breg[f][0] = bnext[f][0];
        breg[f][1] = bnext[f][1];
      }
    }
    cur ^= 1;
  }

  float* C = g.C + (long long)blockIdx.y * g.split_stride;
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    if (!valid[f]) continue;
    const int col = ncol[f] + (lane & 15);
    const float cs = cscale[f] ? (float)cscale[f][lane & 15] : 1.0f;
#pragma unroll
    for (int mi = 0; mi < MF; ++mi) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + mi * 16 + (lane >> 4) * 4 + v;
        C[(long long)row * g.ldc + col] = acc[mi][f][v] * cs;
      }
    }
  }
}

template <int MF>
hipError_t launch_mf(const GemmArgs& g, hipStream_t st) {
  constexpr int NF = 2, NW = 4;
  const int ncols = NW * NF * 16;
  dim3 grid((g.N + ncols - 1) / ncols, g.split, g.M / (MF * 16));
  hipLaunchKernelGGL((gemm_nt_kernel<MF, NF, NW>), grid, dim3(NW * 64), 0, st, g);
  return hipGetLastError();
}

__global__ void sum_splits_kernel(const float* __restrict__ part, int split, long long sstride,
                                  int ldp, float* __restrict__ out, int ldo, int M, int N) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * N) return;
  const int m = (int)(i / N), n = (int)(i % N);
  float s = 0.f;
  for (int k = 0; k < split; ++k) s += part[k * sstride + (long long)m * ldp + n];
  out[(long long)m * ldo + n] = s;
}

// 64x64 tiles through LDS; 256 threads.
__global__ void transpose_f16_kernel(const _Float16* __restrict__ src, int rows, int cols, int lds,
                                     _Float16* __restrict__ dst, int ldd) {
  __shared__ _Float16 tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = src[(long long)gr * lds + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int gc = c0 + c, gr = r0 + tx;
    if (gc < cols && gr < rows) dst[(long long)gc * ldd + gr] = tile[tx][c];
  }
}

__global__ void transpose_i8_kernel(const int8_t* __restrict__ src, int rows, int cols, int lds,
                                    int8_t* __restrict__ dst, int ldd) {
  __shared__ int8_t tile[64][68];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = src[(long long)gr * lds + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int gc = c0 + c, gr = r0 + tx;
    if (gc < cols && gr < rows) dst[(long long)gc * ldd + gr] = tile[tx][c];
  }
}

__global__ void f32_to_f16_kernel(const float* __restrict__ s, _Float16* __restrict__ d, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    d[i] = (_Float16)s[i];
}

__global__ void copy_rows_f16_kernel(const _Float16* __restrict__ s, int rows, int cols, int lds,
                                     _Float16* __restrict__ d, int ldd) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)rows * cols) return;
  const int r = (int)(i / cols), c = (int)(i % cols);
  d[(long long)r * ldd + c] = s[(long long)r * lds + c];
}

__global__ void fill_f32_kernel(float* d, float v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    d[i] = v;
}

// src/kernels/quantize.cu:8-44, bit-exact: scale = max|w|/127 (IEEE fp32
// division), inv = 1/scale, q = rint(clamp(w*inv, -127, 127)) with
// round-half-to-even (v_rndne_f32).  One workgroup of 256 per row.
__global__ void quantize_rows_kernel(const float* __restrict__ w, int cols, int8_t* __restrict__ q,
                                     float* __restrict__ scale) {
  __shared__ float red[4];
  const long long base = (long long)blockIdx.x * cols;
  float m = 0.f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, fabsf(w[base + c]));
  m = block_max<4>(m, red);
  const float sc = m / 127.0f;
  if (threadIdx.x == 0) scale[blockIdx.x] = sc;
  const float inv = sc > 0.f ? 1.0f / sc : 0.f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    float v = w[base + c] * inv;
    v = fminf(fmaxf(v, -127.f), 127.f);
    q[base + c] = (int8_t)rintf(v);
  }
}

__global__ void f32_scale_to_f16_kernel(const float* s, _Float16* d, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) d[i] = (_Float16)s[i];
}

inline int grid1d(size_t n, int bs, int cap = 65536) {
  size_t g = (n + bs - 1) / bs;
  return (int)(g > (size_t)cap ? cap : (g == 0 ? 1 : g));
}

}  // namespace

void gemm_finalize_segments(GemmArgs& g) {
  int s = 0;
  for (int i = 0; i < g.nseg; ++i) {
    g.seg_start[i] = s;
    s += g.seg[i].rows;
  }
  for (int i = g.nseg; i <= 4; ++i) g.seg_start[i] = s;
  g.N = s;
}

int gemm_pick_split(int M, int N, int K, int max_split) {
  // Aim for >= 2 workgroups per CU on 256 CUs while keeping >= 4 K chunks
  // per split.
  const int mt = (M % 128 == 0) ? M / 128 : 1;
  const int ntiles = (N + 127) / 128 * mt;
  int split = (512 + ntiles - 1) / ntiles;
  const int kmax = (K / BK) / 4;
  if (split > kmax) split = kmax;
  if (split > max_split) split = max_split;
  if (split < 1) split = 1;
  return split;
}

hipError_t gemm_nt(const GemmArgs& g, hipStream_t st) {
  if (g.M <= 0 || g.N <= 0 || g.M % 16 || g.K % BK || g.split < 1 || g.nseg < 1 || g.nseg > 4) {
    set_error("gemm_nt: unsupported shape M=%d N=%d K=%d split=%d", g.M, g.N, g.K, g.split);
    return hipErrorInvalidValue;
  }
  for (int i = 0; i < g.nseg; ++i)
    if (g.seg[i].rows % 16) {
      set_error("gemm_nt: segment rows must be a multiple of 16 (%d)", g.seg[i].rows);
      return hipErrorInvalidValue;
    }
  hipError_t e;
  const int m16 = g.M / 16;
  if (m16 % 8 == 0) e = launch_mf<8>(g, st);
  else if (m16 % 4 == 0) e = launch_mf<4>(g, st);
  else if (m16 % 2 == 0) e = launch_mf<2>(g, st);
  else e = launch_mf<1>(g, st);
  if (e != hipSuccess) set_error("gemm_nt launch: %s", hipGetErrorString(e));
  return e;
}

hipError_t sum_splits(const float* part, int split, long long sstride, int ldp, float* out, int ldo,
                      int M, int N, hipStream_t st) {
  const long long n = (long long)M * N;
  hipLaunchKernelGGL(sum_splits_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part,
                     split, sstride, ldp, out, ldo, M, N);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t transpose_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st) {
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  hipLaunchKernelGGL(transpose_f16_kernel, grid, dim3(256), 0, st, src, rows, cols, lds, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t transpose_i8(const int8_t* src, int rows, int cols, int lds, int8_t* dst, int ldd,
                        hipStream_t st) {
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, st, src, rows, cols, lds, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t f32_to_f16(const float* src, _Float16* dst, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid1d(n, 256)), dim3(256), 0, st, src, dst, n);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t copy_rows_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st) {
  const long long n = (long long)rows * cols;
  hipLaunchKernelGGL(copy_rows_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src,
                     rows, cols, lds, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t fill_f32(float* dst, float v, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid1d(n, 256)), dim3(256), 0, st, dst, v, n);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t quantize_rows_i8(const float* w, int rows, int cols, int8_t* q, float* scale,
                            hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(rows), dim3(256), 0, st, w, cols, q, scale);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t f32_scale_to_f16(const float* s, _Float16* d, int n, hipStream_t st) {
  hipLaunchKernelGGL(f32_scale_to_f16_kernel, dim3((n + 255) / 256), dim3(256), 0, st, s, d, n);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
