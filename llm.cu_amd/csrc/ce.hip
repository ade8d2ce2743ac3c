// ce.hip — fused softmax + NLL + dlogits over the 151936-wide vocabulary.
//
// Restates src/kernels/loss.cu:13-91 (one block per row, three sweeps over
// the row, host-side sum) for gfx950: with only T = 128 rows and 256 CUs,
// each row is split into CE_CHUNK-wide chunks so the grid has T * chunks
// workgroups.
//   phase 1: per chunk, an online (max, sum exp(x - max)) pair -> stats.
//   phase 2: merge the row's pairs into lse = m + ln Z, then for every j
//            p = exp(x_j - lse), g = p - 1[j = t], and write the fp32 dlogits
//            g / n_valid and/or the fp16 operand g * 2^14 for the lm_head dX
//            GEMM (the scale keeps p ~ 1/V out of fp16 subnormals; the GEMM
//            epilogue divides it out exactly).  The chunk's second read hits
//            L2 / MALL (the 77.8 MB of logits fit in the 256 MB MALL).
//   phase 3: one workgroup sums the per-row losses in a fixed order.
// In the training step and the lm_head entry point the logits GEMM writes
// the (max, sum exp) pairs of its column tiles itself (GemmArgs::rowstats):
// phase 1 is then a merge of those pairs per row (ce_lse_kernel) and the
// logits are read once.
// Rows i with (i % seq_len) == seq_len - 1 have no target inside their
// window (loss.cu:18-21); their loss is 0 and their dlogits row is written
// as zeros (the reference leaves it uninitialised).
#include <algorithm>
#include <mutex>

#include "../../include/llmt.h"
#include "ops.h"

namespace llmt {

namespace {

constexpr int CE_THREADS = 256;
constexpr int CE_CHUNK = 8192;  // floats per workgroup chunk (32 KB)
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

__device__ __forceinline__ void merge(float& m, float& s, float m2, float s2) {
  softmax_merge(m, s, m2, s2);
}

// A thread's share of a chunk: CE_U float4 pieces, piece k at column
// j0 + 4 tid + 4 CE_THREADS k, all loaded before any use (pieces past the
// row end read as -inf).  exp2 is the hardware v_exp_f32 on fma-scaled
// arguments: the probabilities it cannot represent as fp32 normals
// (< 2^-126) vanish in the fp16 GEMM operand and leave the row sums unchanged.
constexpr int CE_U = CE_CHUNK / (4 * CE_THREADS);
static_assert(CE_U * 4 * CE_THREADS == CE_CHUNK, "chunk = whole float4 pieces a thread");
template <int U = CE_U, bool NT = false>
__device__ __forceinline__ void ce_load(const float* x, int j0, int j1, float4 (&v)[U]) {
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int j = j0 + 4 * (int)threadIdx.x + 4 * CE_THREADS * k;
    if (j < j1) {
      if constexpr (NT) {
        const floatx4 t = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(x + j));
        v[k] = make_float4(t[0], t[1], t[2], t[3]);
      } else {
        v[k] = *reinterpret_cast<const float4*>(x + j);
      }
    } else {
      v[k] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
  }
}

__global__ __launch_bounds__(CE_THREADS) void ce_phase1(const float* __restrict__ logits, int V,
                                                        int chunks, float2* __restrict__ stats) {
  const int row = blockIdx.y, ch = blockIdx.x;
  const int j0 = ch * CE_CHUNK;
  const int j1 = min(V, j0 + CE_CHUNK);
  // 16-byte loads; V is a multiple of 4 for every supported vocabulary.
  float4 v[CE_U];
  ce_load(logits + (long long)row * V, j0, j1, v);
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < CE_U; ++k) m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
  float s = 0.f;
  if (m != -INFINITY) {  // else every piece is past the row end
    const float m2 = m * LOG2E;
#pragma unroll
    for (int k = 0; k < CE_U; ++k)
      s += (__builtin_amdgcn_exp2f(fmaf(v[k].x, LOG2E, -m2)) +
            __builtin_amdgcn_exp2f(fmaf(v[k].y, LOG2E, -m2))) +
           (__builtin_amdgcn_exp2f(fmaf(v[k].z, LOG2E, -m2)) +
            __builtin_amdgcn_exp2f(fmaf(v[k].w, LOG2E, -m2)));
  }
  // wave then block merge of (m, s)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge(m, s, m2, s2);
  }
  __shared__ float rm[CE_THREADS / 64], rs[CE_THREADS / 64];
  if ((threadIdx.x & 63) == 0) {
    rm[threadIdx.x >> 6] = m;
    rs[threadIdx.x >> 6] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = rm[0], S = rs[0];
    for (int i = 1; i < CE_THREADS / 64; ++i) merge(M, S, rm[i], rs[i]);
    stats[(long long)row * chunks + ch] = make_float2(M, S);
  }
}

// NT: nontemporal stores (outputs far larger than the caches, which the
// next kernel cannot find there anyway).
template <bool NT = false>
__device__ __forceinline__ void ce_store(float* dlogits, _Float16* grad16, long long at, float4 g,
                                         float inv_valid) {
  if (dlogits) {
    const floatx4 d = {g.x * inv_valid, g.y * inv_valid, g.z * inv_valid, g.w * inv_valid};
    if constexpr (NT)
      __builtin_nontemporal_store(d, reinterpret_cast<floatx4*>(dlogits + at));
    else
      *reinterpret_cast<floatx4*>(dlogits + at) = d;
  }
  if (grad16) {
    half4 h = {(_Float16)(g.x * kGradLogitScale), (_Float16)(g.y * kGradLogitScale),
               (_Float16)(g.z * kGradLogitScale), (_Float16)(g.w * kGradLogitScale)};
    if constexpr (NT)
      __builtin_nontemporal_store(h, reinterpret_cast<half4*>(grad16 + at));
    else
      *reinterpret_cast<half4*>(grad16 + at) = h;
  }
}

// FROM_LSE: the row's lse comes from lse_rows (ce_lse_kernel, which also
// wrote the row loss), else from merging the row's `chunks` phase-1 pairs in
// stats.  A workgroup covers U float4 pieces a thread (U * 1024 columns):
// with the lse given, the row is cut finer (U = 2): one or two 16-byte loads
// a thread over many workgroups kept a copy-like kernel's DRAM streams at
// 6.2 TB/s on MI355X against 5.5 TB/s with eight a thread.  NT: logits
// larger than the 256 MB last-level cache are read, and the outputs
// written, nontemporal (C4: 702 -> 601 us); smaller ones come from and stay
// in that cache for the next kernel.
template <bool FROM_LSE, int U, bool NTS = false>
__global__ __launch_bounds__(CE_THREADS) void ce_phase2(const float* __restrict__ logits,
                                                        const int* __restrict__ targets, int V,
                                                        int seq_len, int chunks, float inv_valid,
                                                        const float2* __restrict__ stats,
                                                        const float* __restrict__ lse_rows,
                                                        float* __restrict__ dlogits,
                                                        _Float16* __restrict__ grad16,
                                                        float* __restrict__ loss_rows) {
  constexpr int CHUNK = U * 4 * CE_THREADS;
  const int row = blockIdx.y, ch = blockIdx.x;
  const bool valid = (row % seq_len) != seq_len - 1;
  const int j0 = ch * CHUNK;
  const int j1 = min(V, j0 + CHUNK);
  const long long base = (long long)row * V;
  if (!valid) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int j = j0 + 4 * (int)threadIdx.x + 4 * CE_THREADS * k;
      if (j < j1) ce_store<NTS>(dlogits, grad16, base + j, make_float4(0.f, 0.f, 0.f, 0.f), 0.f);
    }
    if (!FROM_LSE && ch == 0 && threadIdx.x == 0) loss_rows[row] = 0.f;
    return;
  }
  float4 v[U];
  ce_load<U, NTS>(logits + base, j0, j1, v);
  float lse;
  if constexpr (FROM_LSE) {
    lse = lse_rows[row];
  } else {
    float M = -INFINITY, S = 0.f;
    for (int c = 0; c < chunks; ++c) {
      const float2 p = stats[(long long)row * chunks + c];
      merge(M, S, p.x, p.y);
    }
    lse = M + __logf(S);
  }
  const float l2 = lse * LOG2E;
  // Out-of-range ids are clamped (never read out of bounds); the reference
  // does not check them.
  const int t = min(max(targets[row], 0), V - 1);
  if (!FROM_LSE && ch == 0 && threadIdx.x == 0) loss_rows[row] = lse - logits[base + t];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int j = j0 + 4 * (int)threadIdx.x + 4 * CE_THREADS * k;
    if (j < j1)
      ce_store<NTS>(dlogits, grad16, base + j,
               make_float4(__builtin_amdgcn_exp2f(fmaf(v[k].x, LOG2E, -l2)),
                           __builtin_amdgcn_exp2f(fmaf(v[k].y, LOG2E, -l2)),
                           __builtin_amdgcn_exp2f(fmaf(v[k].z, LOG2E, -l2)),
                           __builtin_amdgcn_exp2f(fmaf(v[k].w, LOG2E, -l2))),
               inv_valid);
  }
  // p - 1 at the target, stored again by the thread whose piece holds it
  // (program order puts it after that thread's first store)
  if (t >= j0 && t < j1 && (((t - j0) >> 2) & (CE_THREADS - 1)) == (int)threadIdx.x) {
    const float gt = __builtin_amdgcn_exp2f(fmaf(logits[base + t], LOG2E, -l2)) - 1.0f;
    // (the same store path as the piece's first store: same-address order)
    if constexpr (NTS) {
      if (dlogits) __builtin_nontemporal_store(gt * inv_valid, dlogits + base + t);
      if (grad16) __builtin_nontemporal_store((_Float16)(gt * kGradLogitScale), grad16 + base + t);
    } else {
      if (dlogits) dlogits[base + t] = gt * inv_valid;
      if (grad16) grad16[base + t] = (_Float16)(gt * kGradLogitScale);
    }
  }
}

// A row's lse from the ntiles (max, sum exp) pairs the logits GEMM wrote:
// thread i merges tiles i, i + CE_THREADS, .. in order, then the threads'
// pairs meet in a fixed butterfly and the waves' in wave order; also the
// row's loss lse - x_t (0 for rows without a target).
__global__ __launch_bounds__(CE_THREADS) void ce_lse_kernel(const float2* __restrict__ stats,
                                                            int ntiles,
                                                            const float* __restrict__ logits,
                                                            const int* __restrict__ targets, int V,
                                                            int seq_len,
                                                            float* __restrict__ lse_rows,
                                                            float* __restrict__ loss_rows) {
  const int row = blockIdx.x;
  float m = -INFINITY, s = 0.f;
  for (int i = threadIdx.x; i < ntiles; i += CE_THREADS) {
    const float2 p = stats[(long long)row * ntiles + i];
    merge(m, s, p.x, p.y);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    merge(m, s, m2, s2);
  }
  __shared__ float rm[CE_THREADS / 64], rs[CE_THREADS / 64];
  if ((threadIdx.x & 63) == 0) {
    rm[threadIdx.x >> 6] = m;
    rs[threadIdx.x >> 6] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = rm[0], S = rs[0];
    for (int i = 1; i < CE_THREADS / 64; ++i) merge(M, S, rm[i], rs[i]);
    const float lse = M + __logf(S);
    lse_rows[row] = lse;
    const bool valid = (row % seq_len) != seq_len - 1;
    const int t = min(max(targets[row], 0), V - 1);
    loss_rows[row] = valid ? lse - logits[(long long)row * V + t] : 0.f;
  }
}

// Deterministic mean over valid rows (fixed summation order).
__global__ __launch_bounds__(CE_THREADS) void ce_mean(const float* __restrict__ loss_rows, int rows,
                                                      float inv_valid, float* __restrict__ out) {
  __shared__ float red[CE_THREADS / 64];
  float s = 0.f;
  for (int i = threadIdx.x; i < rows; i += CE_THREADS) s += loss_rows[i];
  s = block_sum<CE_THREADS / 64>(s, red);
  if (threadIdx.x == 0) *out = s * inv_valid;
}

}  // namespace

int ce_chunks(int V) { return (V + CE_CHUNK - 1) / CE_CHUNK; }
int ce_stats_per_row(int V) { return std::max(ce_chunks(V), (V + 127) / 128); }

hipError_t cross_entropy(const float* logits, const int* targets, int rows, int V, int seq_len,
                         float2* stats, float* dlogits, _Float16* grad16, float* loss_rows,
                         float* loss_mean, hipStream_t st) {
  if (V % 4 || seq_len < 2 || rows % seq_len) {
    set_error("cross_entropy: unsupported V=%d seq_len=%d rows=%d", V, seq_len, rows);
    return hipErrorInvalidValue;
  }
  const int chunks = ce_chunks(V);
  const int n_valid = rows / seq_len * (seq_len - 1);
  const float inv_valid = 1.0f / (float)n_valid;
  hipLaunchKernelGGL(ce_phase1, dim3(chunks, rows), dim3(CE_THREADS), 0, st, logits, V, chunks,
                     stats);
  LLMT_LAUNCH_CHECK();
  hipLaunchKernelGGL((ce_phase2<false, CE_U>), dim3(chunks, rows), dim3(CE_THREADS), 0, st, logits,
                     targets, V, seq_len, chunks, inv_valid, stats, nullptr, dlogits, grad16,
                     loss_rows);
  LLMT_LAUNCH_CHECK();
  if (loss_mean) {
    hipLaunchKernelGGL(ce_mean, dim3(1), dim3(CE_THREADS), 0, st, loss_rows, rows, inv_valid,
                       loss_mean);
    LLMT_LAUNCH_CHECK();
  }
  return hipSuccess;
}

hipError_t cross_entropy_from_stats(const float* logits, const float2* stats, int ntiles,
                                    const int* targets, int rows, int V, int seq_len, float* lse,
                                    float* dlogits, _Float16* grad16, float* loss_rows,
                                    float* loss_mean, hipStream_t st) {
  if (V % 4 || seq_len < 2 || rows % seq_len || ntiles < 1 || !stats || !lse) {
    set_error("cross_entropy_from_stats: unsupported V=%d seq_len=%d rows=%d ntiles=%d", V,
              seq_len, rows, ntiles);
    return hipErrorInvalidValue;
  }
  const int chunks = ce_chunks(V);
  const int n_valid = rows / seq_len * (seq_len - 1);
  const float inv_valid = 1.0f / (float)n_valid;
  hipLaunchKernelGGL(ce_lse_kernel, dim3(rows), dim3(CE_THREADS), 0, st, stats, ntiles, logits,
                     targets, V, seq_len, lse, loss_rows);
  LLMT_LAUNCH_CHECK();
  constexpr int U2 = 2;
  const dim3 g2((V + U2 * 4 * CE_THREADS - 1) / (U2 * 4 * CE_THREADS), rows);
  // logits beyond the 256 MB last-level cache: nontemporal reads and writes
  if ((double)rows * V * 4 > 256.0 * (1 << 20))
    hipLaunchKernelGGL((ce_phase2<true, U2, true>), g2, dim3(CE_THREADS), 0, st, logits, targets,
                       V, seq_len, chunks, inv_valid, nullptr, lse, dlogits, grad16, loss_rows);
  else
    hipLaunchKernelGGL((ce_phase2<true, U2, false>), g2, dim3(CE_THREADS), 0, st, logits, targets,
                       V, seq_len, chunks, inv_valid, nullptr, lse, dlogits, grad16, loss_rows);
  LLMT_LAUNCH_CHECK();
  if (loss_mean) {
    hipLaunchKernelGGL(ce_mean, dim3(1), dim3(CE_THREADS), 0, st, loss_rows, rows, inv_valid,
                       loss_mean);
    LLMT_LAUNCH_CHECK();
  }
  return hipSuccess;
}

// ------------------------------------------------------------------ no-alloc variant
// llmt_cross_entropy_noalloc keeps the per-(row, chunk) softmax statistics
// in a file-scope device array instead of a workspace allocated per call:
// kNoAllocStats float2 entries (2 MiB), enough for rows * ce_chunks(V) of
// 13,797 rows at V = 151936.  Each GPU holds its own copy for the life of the
// process; its address is looked up once per device with
// hipGetSymbolAddress (the array's name is a host-side stand-in and is never
// passed to a kernel).  Phase 1 writes every entry phase 2 reads, so nothing
// needs clearing between calls.  Calls that overlap on one GPU share the
// array and race.
constexpr long long kNoAllocStats = 262144;
static __device__ __align__(256) float2 scratch[kNoAllocStats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float2* g_scratch[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on first use).
hipError_t scratch_address(float2** out) {
  int dev = 0;
  LLMT_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("llmt_cross_entropy_noalloc: device %d outside the %d supported", dev, kMaxDevices);
    return hipErrorInvalidDevice;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    // The first call may come under a caller's stream capture: the lookup
    // (no stream work) runs in relaxed capture mode for this thread, so a
    // global-mode capture does not reject it, and the mode is restored.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    LLMT_HIP_TRY(hipThreadExchangeStreamCaptureMode(&mode));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    LLMT_HIP_TRY(hipThreadExchangeStreamCaptureMode(&mode));
    LLMT_HIP_TRY(e);
    g_scratch[dev] = static_cast<float2*>(p);
  }
  *out = g_scratch[dev];
  return hipSuccess;
}
}  // namespace

}  // namespace llmt

extern "C" int llmt_cross_entropy_noalloc(const float* logits, const int* targets, int rows, int V,
                                          int seq_len, float* dlogits, float* loss_rows,
                                          float* loss_mean, void* stream) {
  using namespace llmt;
  set_error("");
  if (!logits || !targets || !loss_rows || rows <= 0 || V <= 0 || V % 4 || seq_len < 2 ||
      rows % seq_len) {
    set_error("llmt_cross_entropy_noalloc: bad arguments (V%%4 == 0, rows %% seq_len == 0, "
              "seq_len >= 2)");
    return LLMT_ERR_ARG;
  }
  const long long need = (long long)rows * ce_chunks(V);
  if (need > kNoAllocStats) {
    set_error("llmt_cross_entropy_noalloc: rows x chunks = %d x %d = %lld statistics exceed the "
              "%lld of the built-in scratch (at most %lld rows at V = %d)",
              rows, ce_chunks(V), need, kNoAllocStats, kNoAllocStats / ce_chunks(V), V);
    return LLMT_ERR_ARG;
  }
  float2* stats = nullptr;
  hipError_t e = scratch_address(&stats);
  if (e == hipSuccess)
    e = cross_entropy(logits, targets, rows, V, seq_len, stats, dlogits, nullptr, loss_rows,
                      loss_mean, (hipStream_t)stream);
  return e == hipSuccess ? LLMT_OK : (e == hipErrorInvalidValue ? LLMT_ERR_ARG : LLMT_ERR_HIP);
}
