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
  const _Float16* colscale;  // int8 [out, in] layout: per output row n
  const _Float16* kscale;    // int8 [in, out] layout: per reduction index k
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
  // split_col > 0 (large tiles, split 2): only the column tiles at or past
  // split_col are split over K; the others write their whole sum to partial
  // 0 and leave partial 1 untouched (gemm_split_col).
  int split_col;
  // glu > 0: fused SwiGLU epilogue (split 1, N = 2 glu, one segment whose
  // rows [0, glu) are the gate and [glu, 2 glu) the up projection): gu16
  // gets [gate | up] in fp16 ([M, 2 glu], the backward's stash; C unused)
  // and glu16[m][n] = fp16(silu(gate) * up), both from the fp32 sums.
  int glu;
  _Float16* glu16;
  int ldglu;
  _Float16* gu16;
  // rowstats (split 1, one segment, no SwiGLU): the epilogue also writes,
  // for every row m and column tile t of the launch, the online-softmax pair
  // (max, sum exp(C - max)) of the row's stored values in the tile:
  // rowstats[m * gemm_rowstats_tiles(g) + t] (the fused cross entropy's
  // statistics of the lm_head logits, so the logits are read only once).
  float2* rowstats;
};
// The fused SwiGLU epilogue exists for this GEMM shape and weight type.
bool gemm_glu_ok(int M, int I, int K, bool i8);
// Column tiles per row whose statistics gemm_nt writes for g.rowstats (the
// row width of the rowstats array), 0 if this GEMM cannot write them.
int gemm_rowstats_tiles(const GemmArgs& g);

// Every B segment is fragment-packed (packed_index, common.h) with row
// length K; rows a multiple of 16.  A is row-major fp16 [M, lda], K % 32 == 0.
// Fills seg_start/N from seg[0..nseg).
void gemm_finalize_segments(GemmArgs& g);
// Split factor for a GEMM of this shape on this device (>=1, bounded by K).
int gemm_pick_split(int M, int N, int K, int max_split);
// For a large-tile GEMM planned unsplit whose 256 x 256 tiles end in a
// partial wave of the CUs: the column where tiles start to be split in two
// so that the last wave is full (GemmArgs::split_col, with split 2); 0 when
// the tiles fill whole waves or the shape does not allow it.
int gemm_split_col(int M, int N, int K);
hipError_t gemm_nt(const GemmArgs& g, hipStream_t st);
// Name of the kernel gemm_nt launches for g ("gemm_skinny", "gemm_dma", ...).
const char* gemm_kernel_name(const GemmArgs& g);
// out[m][n] = sum_s part[s][m][n] in split order, plus for output columns
// [c0, c0 + n) of each LoRA adapter lscale * sum_r part-sum[m][hcol + r] *
// M(r, n') (M = B [n, 16] if is_B, else A [16, n]).  out != part; M % 16 == 0.
struct LoraUp {
  const float* M;
  int c0, n, hcol, is_B;
};
struct ReduceArgs {
  const float* part;
  int split;
  long long ss;
  int ldp;
  float* out;
  int ldo;
  int M, N;
  int nlora;
  LoraUp up[3];
  float lscale;
  float out_scale;  // 0 is read as 1
};
hipError_t reduce_lora(const ReduceArgs& a, hipStream_t st);
// Pack a row-major block into rows [row0, row0 + R) x k [k0, k0 + C) of a
// fragment-packed operand with row length K (transpose: the block is src^T).
hipError_t pack_f16(const _Float16* src, long long lds, int transpose, int R, int C, _Float16* dst,
                    long long K, int row0, int k0, hipStream_t st);
// pack_i8 stores each int8 x biased, as the byte x + 128 (x ^ 0x80), which
// the GEMMs' int8 -> fp16 conversion expects; zs (NULL: none) is the fp16
// scale of each source row (the block's rows, or its columns when
// transposed), and rows whose scale is 0 are stored as zeros.
hipError_t pack_i8(const int8_t* src, long long lds, int transpose, int R, int C, int8_t* dst,
                   long long K, int row0, int k0, hipStream_t st, const _Float16* zs = nullptr);

// ---------------------------------------------------------------- layout
hipError_t transpose_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st);
hipError_t transpose_i8(const int8_t* src, int rows, int cols, int lds, int8_t* dst, int ldd,
                        hipStream_t st);
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
// float2 pairs a row that hold either the CE's chunk pairs or a logits
// GEMM's tile pairs (every tile width gemm_nt uses is >= 128 columns).
int ce_stats_per_row(int V);
hipError_t cross_entropy(const float* logits, const int* targets, int rows, int V, int seq_len,
                         float2* stats, float* dlogits, _Float16* grad16, float* loss_rows,
                         float* loss_mean, hipStream_t st);
// The same from statistics the logits GEMM wrote (GemmArgs::rowstats, ntiles
// pairs a row): one pass over the logits.  lse: float [rows] workspace.
hipError_t cross_entropy_from_stats(const float* logits, const float2* stats, int ntiles,
                                    const int* targets, int rows, int V, int seq_len, float* lse,
                                    float* dlogits, _Float16* grad16, float* loss_rows,
                                    float* loss_mean, hipStream_t st);
constexpr float kGradLogitScale = 16384.0f;  // 2^14

// ---------------------------------------------------------------- row kernels
// A token row of a split-K GEMM output as the input of a row epilogue: the
// fp32 partials (summed in split order by the consumer) plus the LoRA
// up-projection terms, taken from the row-major fp16 twin of an adapter
// shadow block ([rows, kp], the same values as the fragment-packed block the
// GEMMs read; a row's columns are contiguous, so a wave's loads coalesce):
//   y[c] += lscale * sum_r h[hidx + r] * shadow(row0 + r, c)   for c in [c0, c0 + n)
// where h are the raw extra columns [hcol, hcol + nh) of the same GEMM.
struct LoraTerm {
  const _Float16* shr;  // element (row0 + r, c) at shr[(row0 + r) * kp + c]
  int row0, kp;
  int c0, n;            // multiples of 8
  int hidx;
};
struct RowIn {
  const float* part;
  int split;
  long long ss;
  int ldp;
  int split_col;  // > 0: columns below it have only partial 0 (GemmArgs::split_col)
  int hcol, nh;  // nh % 4 == 0, nh <= 64 (0: none)
  int nterm;     // <= 3
  LoraTerm term[3];
  float lscale;
};

struct QkvPostArgs {
  RowIn in;
  const float* qn;
  const float* kn;
  const float* cosT;
  const float* sinT;  // [S, 64]
  int S, nq, nkv;
  float eps;
  _Float16* qkraw;   // [T, Q + KV] fp16
  _Float16* qkv16;   // [T, Q + 2 KV]
  float* hbuf;       // [T, 64]: h columns 0..47
};

struct NormBwdArgs {
  RowIn in;
  const float* rinv_in;  // per-row, may be NULL
  float gscale;
  float* dh_out;         // [T, 64]: the in.nh raw h columns times the row scale
  int dh_col;
  const float* x;        // RMSNorm input [T, H]
  const float* w;
  float eps;
  int H;
  const float* dres_in;  // may be NULL (= 0); may alias dres_out
  float* dres_out;
  float* dmid_out;       // may be NULL
  _Float16* g16;
  float* rinv_out;
  // NULL, or a per-column factor [H] folded into g16 (the consuming int8
  // GEMM's per-k weight scale, which that GEMM then leaves out)
  const _Float16* g16_ks;
  // NULL, or the layer's A_q | A_k | A_v transposed [H][3 R] fp16: with the
  // three full-width q/k/v terms, the LoRA dx term then runs on MFMA
  const _Float16* lora_at;
};

struct QkBwdArgs {
  const float* dqkv;  // attention grads [T, ld] (dq | dk | dv)
  int ld_dqkv;
  const _Float16* qkraw;  // [T, Q + KV] q, k before the QK-norm (fp16)
  const float* qn;
  const float* kn;
  const float* cosT;
  const float* sinT;
  int S, nq, nkv;
  float eps;
  float* dy32;        // [T, NT], may be NULL
  _Float16* g16;      // [T, NT], row t scaled by 1 / rinv_out[t]
  float* rinv_out;
};

hipError_t embed_norm(const int* tok, const _Float16* E, int V, int H, const float* w, float eps,
                      int T, float* x, _Float16* xn, hipStream_t st);
hipError_t qkv_post(const QkvPostArgs& a, int T, hipStream_t st);
hipError_t o_post(const RowIn& in, const float* x_in, const float* w, float eps, int H, int T,
                  float* hbuf, float* x_mid, _Float16* xn2, hipStream_t st);
hipError_t gu_post(const RowIn& in, int I, int T, _Float16* gu, _Float16* a16, hipStream_t st);
hipError_t resid_norm(const RowIn& in, const float* x_res, const float* w, float eps, int H, int T,
                      float* x_out, _Float16* xn, hipStream_t st);
// cos / sin tables of the half-split RoPE, [S, 64] fp32 each, on the device.
hipError_t rope_tables(int S, double theta, float* cosT, float* sinT, hipStream_t st);
// Per-head QK-RMSNorm + RoPE of [T, nh, 128] fp16 rows (weights w [128]).
// Up to two tensors in one launch.  (The backward runs inside the attention
// backward's epilogues, AttnArgs::qn / kn.)
struct HeadRows {
  const _Float16* x;  // raw rows
  const float* w;     // norm weights [128]
  _Float16* out;      // normed, rotated rows
  int nh;
};
hipError_t head_norm_rope(const HeadRows* segs, int nseg, const float* cosT, const float* sinT,
                          int S, int T, float eps, hipStream_t st);
hipError_t norm_bwd(const NormBwdArgs& a, int T, hipStream_t st);
// ks: NULL, or a per-column factor [2 I] folded into dgu16 (as g16_ks).
hipError_t swiglu_bwd(const RowIn& in, const float* rinv_in, const _Float16* gu, int I, int T,
                      _Float16* dgu16, float* rinv_out, const _Float16* ks, hipStream_t st);
// dX of the O projection -> the attention's dO operand: dO16 (row t, head h)
// = fp16(dO * 2^k) with 2^k the power-of-two scale of that head row,
// dsc[b, h, s] = 2^-k (0 for an all-zero head row), delta[b, h, s] =
// sum_d dO * O.
hipError_t o_dx_post(const RowIn& in, const float* rinv_in, const _Float16* o16, int nq, int S,
                     int T, float* dh_out, _Float16* dO16, float* delta, float* dsc,
                     hipStream_t st);
hipError_t qk_bwd(const QkBwdArgs& a, int T, hipStream_t st);
// x_out = x (may alias), xn = fp16(rmsnorm(x) * w): a layer input from fp32.
hipError_t copy_norm(const float* x, const float* w, float eps, int H, int T, float* x_out,
                     _Float16* xn, hipStream_t st);
// A gradient row as the fp16 GEMM operand: dres = dy (may alias), g16 =
// fp16(dy * ks * sc), rinv = 1 / sc with sc the row's power-of-two scale and
// ks a per-column factor (1 when NULL).
hipError_t grad_rows(const float* dy, int H, int T, float* dres, _Float16* g16, float* rinv,
                     const _Float16* ks, hipStream_t st);
// dst[r][c] = (float) src[r][c] for a [rows, cols] block (lds, ldd).
hipError_t f16_to_f32_rows(const _Float16* src, long long lds, int rows, int cols, float* dst,
                           long long ldd, hipStream_t st);
// dst = fp16(src * scale) elementwise.
hipError_t f32_to_f16_scaled(const float* src, _Float16* dst, size_t n, float scale,
                             hipStream_t st);

// ---------------------------------------------------------------- attention
struct AttnArgs {
  const _Float16* q;    // [T, ldq] (head h at column h * 128)
  long long ldq;
  const _Float16* k;    // [T, ldk]
  long long ldk;
  const _Float16* v;    // [T, ldv]
  long long ldv;
  int nq, nkv, S;
  float sm_scale;
  _Float16* o;          // forward output [T, ldo]
  long long ldo;
  float* lse;           // [B, nq, S] natural-log LSE of the scaled scores
  const _Float16* dO16;  // backward: fp16 [T, ld16], head h of row t = dO / dsc[b, h, s]
  long long ld16;
  const float* dsc;     // [B, nq, S] inverse power-of-two scale of each dO16 head row (0: zero)
  const float* delta;   // [B, nq, S] rowsum(dO * O)
  float* dq;            // fp32 [T, ldgq]
  long long ldgq;
  float* dk;            // dK, dV (summed over each GQA group) fp32 [T, ldgkv]
  float* dv;
  long long ldgkv;
  // The attention block API's fusions (all null in the training step, whose
  // row epilogues do this work).  qn: q is per-head RMSNorm (weights qn,
  // eps) + RoPE (cosT / sinT [S, 64]) of qraw [T, ldqr]: the forward applies
  // both to its Q fragments and writes the fp16 result to q16w (the
  // backward's q); the dQ blocks apply their backward to dQ (dq then holds
  // d qraw).  kn: the same backward for k on the dK blocks (kraw [T, ldkr];
  // dk then holds d kraw).  dout: the forward also writes the backward's dO
  // operand from dout fp16 [T, lddo] into dO16w, deltaw and dscw (as
  // attn_delta does).
  const _Float16* qraw;
  long long ldqr;
  const _Float16* kraw;
  long long ldkr;
  const float* qn;
  const float* kn;
  const float* cosT;
  const float* sinT;
  float eps;
  _Float16* q16w;
  const _Float16* dout;
  long long lddo;
  _Float16* dO16w;
  float* deltaw;
  float* dscw;
};
hipError_t attn_fwd(const AttnArgs& a, int B, hipStream_t st);
hipError_t attn_bwd(const AttnArgs& a, int B, hipStream_t st);
// Operands of a standalone attention backward from dO [T, ldd] (fp32, or
// fp16 with dO_is_f16) and O fp16 [T, ldo]: delta[b, h, s] = sum_d dO * O,
// dO16 [T, ld16] and dsc as o_dx_post writes them.
hipError_t attn_delta(const void* dO, int dO_is_f16, long long ldd, const _Float16* o,
                      long long ldo, int nq, int S, int T, float* delta, _Float16* dO16,
                      long long ld16, float* dsc, hipStream_t st);

// ---------------------------------------------------------------- LoRA / AdamW
struct LoraGradJob {
  const void* X;     // [T, ldx] fp16 or fp32
  int x_f16;
  long long ldx;
  const float* xs;   // NULL, or row t of X stands for X[t] * xs[t]
  int ncols;
  const float* G;    // [T, ldg] (16 columns used)
  long long ldg;
  float* out;
  int out_is_B;      // 0: out[16][ncols] (dA), 1: out[ncols][16] (dB)
};
// The adapter-gradient jobs of `layers` consecutive layers (kLoraJobs per
// layer, same order and column counts in every layer) in one launch; `jobs`
// is a device table [layer][kLoraJobs], starting at the first layer.
constexpr int kLoraJobs = 8;
struct LoraGradPlan {
  int ncols[kLoraJobs];  // columns of each job (identical across layers)
};
hipError_t lora_grad(const LoraGradJob* jobs, const LoraGradPlan& plan, int layers, int T,
                     float lscale, int accumulate, hipStream_t st);

struct AdamHp {
  float lr, beta1, beta2, eps, wd, bc1, bc2;
};
// Where the fp16 operand copies of an arena element live.  Arena layout per
// layer: q A, q B, k A, k B, v A, v B, o A, o B (seg_off = start of each).
// Shadow layout per layer (halves): A_qkv [48][H] at a_qkv, A_o [16][Q] at
// a_o, B^T_qkv [48][nt] at bt_qkv (block-diagonal, zero elsewhere), B^T_o
// [16][H] at bt_o.
struct AdamShadow {
  _Float16* shadow;  // NULL: no shadow writes
  _Float16* rm;      // row-major twin (same block offsets), written with shadow
  _Float16* at;      // NULL, or A_q | A_k | A_v transposed: [layer][d_in[0]][3 R]
  long long per_layer;
  long long seg_off[8];
  int d_in[4];
  int d_out[4];
  int col_off[3];
  int nt;
  long long shadow_per_layer;
  long long a_qkv, a_o, bt_qkv, bt_o;
};
// hp is a device pointer (so a captured graph picks up new step counts).
hipError_t adamw(float* p, const float* g, float* m, float* v, long long n, const AdamHp* hp,
                 int update, const AdamShadow& sh, hipStream_t st);
hipError_t lora_init(float* p, float* m, float* v, long long n, unsigned long long seed,
                     float a_std, float b_std, const AdamShadow& sh, hipStream_t st);

}  // namespace llmt
