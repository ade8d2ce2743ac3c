// ops.h — internal launchers shared by the native step, the compat layer and
// the standalone operator exports.  All take an explicit stream and return
// hipError_t (hipSuccess or the launch error, recorded via set_error).
#pragma once

#include "common.h"

namespace llmt {

// ---------------------------------------------------------------- GEMM
// C[split][m][n] = sum_{k in split's K range} A[m][k] * B[n][k], with the B
// operand given as up to four row segments concatenated along n (frozen
// weights plus LoRA rows).  A: fp16 [M, lda]; a segment is fp16 or int8
// [rows, ld] (int8 rows are dequantised exactly to fp16 in registers; the
// optional fp16 colscale[rows] multiplies the result columns).
struct BSeg {
  const void* ptr;
  const _Float16* colscale;
  int rows;
  int ld;
  int is_i8;
};

struct GemmArgs {
  const _Float16* A;
  int lda;
  BSeg seg[4];
  int seg_start[5];
  int nseg;
  float* C;
  int ldc;
  long long split_stride;  // elements between split partials
  int M, N, K, split;
};

// Fills seg_start/N from seg[0..nseg).
void gemm_finalize_segments(GemmArgs& g);
// Split factor for a GEMM of this shape on this device (>=1, bounded by K).
int gemm_pick_split(int M, int N, int K, int max_split);
hipError_t gemm_nt(const GemmArgs& g, hipStream_t st);
// out[m][n] = sum_s part[s][m][n] (ld = ldp for parts, ldo for out).
hipError_t sum_splits(const float* part, int split, long long split_stride, int ldp, float* out,
                      int ldo, int M, int N, hipStream_t st);

// ---------------------------------------------------------------- layout
hipError_t transpose_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st);
hipError_t transpose_i8(const int8_t* src, int rows, int cols, int8_t* dst, hipStream_t st);
hipError_t f32_to_f16(const float* src, _Float16* dst, size_t n, hipStream_t st);
hipError_t copy_rows_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st);
hipError_t fill_f32(float* dst, float v, size_t n, hipStream_t st);
hipError_t quantize_rows_i8(const float* w, int rows, int cols, int8_t* q, float* scale,
                            hipStream_t st);
hipError_t f32_scale_to_f16(const float* s, _Float16* d, int n, hipStream_t st);

// ---------------------------------------------------------------- cross entropy
// Two-phase fused softmax + NLL + dlogits over rows of width V.
// stats: float2 [rows * chunks] workspace.  grad16 (may be NULL) receives
// fp16 (p - 1[j=t]) * 2^14; dlogits (may be NULL) receives fp32
// (p - 1[j=t]) / n_valid.  loss_rows[r] = lse - x_t (0 for invalid rows).
int ce_chunks(int V);
hipError_t cross_entropy(const float* logits, const int* targets, int rows, int V, int seq_len,
                         float2* stats, float* dlogits, _Float16* grad16, float* loss_rows,
                         float* loss_mean, hipStream_t st);
constexpr float kGradLogitScale = 16384.0f;  // 2^14

}  // namespace llmt
