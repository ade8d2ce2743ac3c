// api_ops.cpp — C ABI: error reporting and the standalone operators of
// include/llmt.h (GEMM, int8 quantizer, cross-entropy, fused lm_head + CE,
// attention).  Each validates shapes on the host before any launch.
#include <stdarg.h>
#include <string.h>

#include "../../include/llmt.h"
#include "ops.h"

namespace llmt {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

}  // namespace llmt

using namespace llmt;

#define API_TRY(expr)                    \
  do {                                   \
    hipError_t e__ = (expr);             \
    if (e__ != hipSuccess) {             \
      if (!g_err[0] || e__ != hipErrorInvalidValue) \
        set_error("%s: %s", #expr, hipGetErrorString(e__)); \
      return e__ == hipErrorInvalidValue ? LLMT_ERR_ARG : LLMT_ERR_HIP; \
    }                                    \
  } while (0)

extern "C" {

const char* llmt_last_error(void) { return g_err; }

void llmt_dims_qwen3_1_7b(llmt_dims* d) {
  d->hidden = LLMT_HIDDEN_SIZE;
  d->n_layers = LLMT_NUM_LAYERS;
  d->n_heads = LLMT_NUM_HEADS;
  d->n_kv_heads = LLMT_NUM_KV_HEADS;
  d->head_dim = LLMT_HEAD_DIM;
  d->intermediate = LLMT_INTERMEDIATE_SIZE;
  d->vocab = LLMT_VOCAB_SIZE;
  d->rank = LLMT_LORA_RANK;
  d->alpha = (float)LLMT_LORA_ALPHA;
  d->eps = LLMT_RMS_NORM_EPS;
  d->theta = LLMT_ROPE_THETA;
}

// The standalone GEMMs take a row-major B; it is packed into a temporary
// fragment-packed copy first (the training step packs its frozen weights once).
static int gemm_common(const void* A, int lda, const void* B, int ldb, int is_i8,
                       const void* scale, float* C, int ldc, int M, int N, int K, void* stream) {
  g_err[0] = 0;
  if (!A || !B || !C || M <= 0 || N <= 0 || K <= 0 || M % 16 || K % 32 || N % 16 ||
      lda < K || ldb < K || ldc < N || lda % 8 || ldc % 4) {
    set_error("llmt_gemm: unsupported shape M=%d N=%d K=%d (M%%16, N%%16, K%%32, lda%%8, ldc%%4 "
              "must be 0)", M, N, K);
    return LLMT_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  void* packed = nullptr;
  const size_t esz = is_i8 ? 1 : 2;
  API_TRY(hipMallocAsync(&packed, (size_t)N * K * esz, st));
  if (is_i8)
    API_TRY(pack_i8((const int8_t*)B, ldb, 0, N, K, (int8_t*)packed, K, 0, 0, st));
  else
    API_TRY(pack_f16((const _Float16*)B, ldb, 0, N, K, (_Float16*)packed, K, 0, 0, st));
  GemmArgs g{};
  g.A = (const _Float16*)A;
  g.lda = lda;
  g.nseg = 1;
  g.seg[0] = BSeg{packed, (const _Float16*)scale, nullptr, N, K, is_i8};
  gemm_finalize_segments(g);
  g.M = M;
  g.K = K;
  g.split = gemm_pick_split(M, N, K, 64);
  float* part = nullptr;
  if (g.split > 1) {
    API_TRY(hipMallocAsync((void**)&part, (size_t)g.split * M * N * sizeof(float), st));
    g.C = part;
    g.ldc = N;
    g.split_stride = (long long)M * N;
  } else {
    g.C = C;
    g.ldc = ldc;
    g.split_stride = 0;
  }
  API_TRY(gemm_nt(g, st));
  if (part) {
    ReduceArgs ra{};
    ra.part = part;
    ra.split = g.split;
    ra.ss = (long long)M * N;
    ra.ldp = N;
    ra.out = C;
    ra.ldo = ldc;
    ra.M = M;
    ra.N = N;
    API_TRY(reduce_lora(ra, st));
    API_TRY(hipFreeAsync(part, st));
  }
  API_TRY(hipFreeAsync(packed, st));
  return LLMT_OK;
}

int llmt_gemm_f16(const void* A, int lda, const void* B, int ldb, float* C, int ldc, int M, int N,
                  int K, void* stream) {
  return gemm_common(A, lda, B, ldb, 0, nullptr, C, ldc, M, N, K, stream);
}

int llmt_gemm_i8(const void* A, int lda, const int8_t* q, int ldq, const void* scale, float* C,
                 int ldc, int M, int N, int K, void* stream) {
  return gemm_common(A, lda, q, ldq, 1, scale, C, ldc, M, N, K, stream);
}

int llmt_quantize_rows_i8(const float* w, int rows, int cols, int8_t* q, float* scale,
                          void* stream) {
  g_err[0] = 0;
  if (!w || !q || !scale || rows <= 0 || cols <= 0) {
    set_error("llmt_quantize_rows_i8: bad arguments");
    return LLMT_ERR_ARG;
  }
  API_TRY(quantize_rows_i8(w, rows, cols, q, scale, (hipStream_t)stream));
  return LLMT_OK;
}

int llmt_cross_entropy(const float* logits, const int* targets, int rows, int V, int seq_len,
                       float* dlogits, float* loss_rows, float* loss_mean, void* stream) {
  g_err[0] = 0;
  if (!logits || !targets || !loss_rows || rows <= 0 || V <= 0 || V % 4 || seq_len < 2 ||
      rows % seq_len) {
    set_error("llmt_cross_entropy: bad arguments (V%%4 == 0, rows %% seq_len == 0, seq_len >= 2)");
    return LLMT_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  float2* stats = nullptr;
  API_TRY(hipMallocAsync((void**)&stats, sizeof(float2) * rows * ce_chunks(V), st));
  API_TRY(cross_entropy(logits, targets, rows, V, seq_len, stats, dlogits, nullptr, loss_rows,
                        loss_mean, st));
  API_TRY(hipFreeAsync(stats, st));
  return LLMT_OK;
}

}  // extern "C"
