// step.cpp — the native layer of include/llmt.h: one context owns every
// device buffer of the LoRA training step (frozen weights with their
// pre-transposed copies, the fp32 adapter arenas and their fp16 operand
// shadows, the per-layer stashes, the workspaces), sequences the kernels of
// one step on one stream, optionally captures the step into a HIP graph, and
// reads the loss back with the step's single host synchronisation.
//
// Step order follows src/train.cu:251-288: forward
// (src/kernels/lora_forward.cu:169-305), fused cross-entropy
// (src/kernels/loss.cu:74-91), backward (src/kernels/lora_backward.cu:212-408),
// AdamW (src/kernels/lora.cu:235-246).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <vector>

#include "../../include/llmt.h"
#include "ctx.h"

using namespace llmt;

namespace llmt {

// ------------------------------------------------------------------ memory

void* Ctx::alloc(size_t bytes) {
  bytes = (bytes + 255) & ~(size_t)255;
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    set_error("hipMalloc(%zu) failed", bytes);
    return nullptr;
  }
  // Every buffer starts zeroed: rows the step never writes (the pad rows of
  // a batch, see Ctx::rows) then hold finite values from the start.
  if (hipMemset(p, 0, bytes) != hipSuccess) {
    hipFree(p);
    set_error("hipMemset(%zu) failed", bytes);
    return nullptr;
  }
  blocks.push_back(p);
  device_bytes += bytes;
  return p;
}

// Rows B * S .. rows(B) - 1 of the buffers the step writes only at real
// token rows (the layer-0 input rows the token gather fills, the attention
// output and gradients, the CE's fp16 dlogits) are zeroed once per batch
// size, outside any captured graph; with them zero, every other kernel of
// the step keeps the pad rows at exactly zero.
hipError_t Ctx::clear_pad_rows(int B) {
  if (B == pad_batch) return hipSuccess;
  const size_t r0 = (size_t)B * S, n = (size_t)rows(B) - r0;
  if (n) {
    LLMT_HIP_TRY(hipMemsetAsync(stash[0].x_in + r0 * H, 0, n * H * sizeof(float), st));
    LLMT_HIP_TRY(hipMemsetAsync(stash[0].xn + r0 * H, 0, n * H * sizeof(_Float16), st));
    for (int l = 0; l < L; ++l)
      LLMT_HIP_TRY(hipMemsetAsync(stash[l].o16 + r0 * Q, 0, n * Q * sizeof(_Float16), st));
    LLMT_HIP_TRY(hipMemsetAsync(dqkv32 + r0 * NT, 0, n * NT * sizeof(float), st));
    LLMT_HIP_TRY(hipMemsetAsync(grad16 + r0 * V, 0, n * V * sizeof(_Float16), st));
  }
  pad_batch = B;
  return hipSuccess;
}

Ctx::~Ctx() {
  if (graph_exec) hipGraphExecDestroy(graph_exec);
  for (void* p : blocks) hipFree(p);
  if (host_loss) hipHostFree(host_loss);
  if (host_hp) hipHostFree(host_hp);
  if (own_stream) hipStreamDestroy(st);
}

// ------------------------------------------------------------------ launches

hipError_t Ctx::gemm(int cat, const _Float16* A, int lda, const BSeg* segs, int nseg, int M, int K,
                     float* direct, int ldc, GemmOut* out, _Float16* glu16, _Float16* gu16,
                     float2* rowstats, int* tiles, bool last_wave_split) {
  GemmArgs g{};
  g.A = A;
  g.lda = lda;
  g.nseg = nseg;
  for (int i = 0; i < nseg; ++i) g.seg[i] = segs[i];
  gemm_finalize_segments(g);
  g.M = M;
  g.K = K;
  if (glu16) {
    g.split = 1;
    g.C = nullptr;
    g.ldc = 0;
    g.split_stride = 0;
    g.glu = g.N / 2;
    g.glu16 = glu16;
    g.ldglu = g.N / 2;
    g.gu16 = gu16;
  } else if (direct) {
    g.split = 1;
    g.C = direct;
    g.ldc = ldc;
    g.split_stride = 0;
    if (rowstats) {
      const int nt = gemm_rowstats_tiles(g);
      if (nt <= 0 || (size_t)M * nt > (size_t)Tmax * ce_stats_per_row(V)) {
        set_error("gemm: row statistics unavailable for this shape (%d tiles)", nt);
        return hipErrorInvalidValue;
      }
      g.rowstats = rowstats;
      if (tiles) *tiles = nt;
    }
  } else {
    g.split = gemm_pick_split(M, g.N, K, 64);
    if (last_wave_split && nseg == 1 && g.split == 1) {
      g.split_col = gemm_split_col(M, g.N, K);
      if (g.split_col) g.split = 2;
    }
    g.C = part;
    g.ldc = g.N;
    g.split_stride = (long long)M * g.N;
    if ((size_t)g.split * M * g.N > part_elems) {
      set_error("gemm: workspace too small (%d x %d x %d > %zu)", g.split, M, g.N, part_elems);
      return hipErrorInvalidValue;
    }
  }
  if (recording) {
    double wbytes = 0;
    for (int i = 0; i < nseg; ++i) wbytes += (double)segs[i].rows * K * (segs[i].is_i8 ? 1 : 2);
    // the backward's dX GEMMs are kinds of their own (the O projection's dX
    // has the forward's shape)
    const bool dx = cat == CAT_GEMM_BWD || (cat == CAT_GEMM_HEAD && !direct);
    char kind[128];
    snprintf(kind, sizeof kind, "%s M%d N%d K%d split%d%s%s", gemm_kernel_name(g), M, g.N, K,
             g.split, segs[0].is_i8 ? " int8" : "", dx ? " dX" : "");
    launches.push_back({cat, kind, [g](hipStream_t s) { return gemm_nt(g, s); },
                        2.0 * M * g.N * K, wbytes});
  }
  LLMT_HIP_TRY(gemm_nt(g, st));
  if (!out) return hipSuccess;
  out->part = g.C;
  out->split = g.split;
  out->ss = g.split_stride;
  out->ldp = g.ldc;
  out->split_col = g.split_col;
  return hipSuccess;
}

RowIn Ctx::row_in(const GemmOut& go, int hcol, int nh, int nterm, const LoraTerm* terms) const {
  RowIn r{};
  r.part = go.part;
  r.split = go.split;
  r.ss = go.ss;
  r.ldp = go.ldp;
  r.split_col = go.split_col;
  r.hcol = hcol;
  r.nh = nh;
  r.nterm = nterm;
  for (int i = 0; i < nterm; ++i) r.term[i] = terms[i];
  r.lscale = lscale;
  return r;
}

// Bytes a row epilogue reads from a GEMM's split partials: split x T rows of
// n columns plus the raw h columns.
static double part_bytes(const RowIn& r, int T, int n) {
  if (r.split_col > 0) return 4.0 * (double)T * (n + (n - r.split_col) + r.nh);
  return 4.0 * r.split * (double)T * (n + r.nh);
}

// ------------------------------------------------------------------ layout helpers

BSeg Ctx::wseg(const WMat& w) const {
  BSeg s{};
  s.ptr = w.p;
  s.colscale = w.colscale;
  s.kscale = w.kscale;
  s.rows = w.rows;
  s.ld = w.ld;
  s.is_i8 = w.i8;
  return s;
}

BSeg Ctx::hseg(const _Float16* p, int rows, int ld) const {
  BSeg s{};
  s.ptr = p;
  s.rows = rows;
  s.ld = ld;
  return s;
}

float* Ctx::lora_ptr(float* arena, int l, int proj, int is_b) const {
  return arena + (size_t)l * lora_per_layer + seg_off[2 * proj + is_b];
}

_Float16* Ctx::shadow_ptr(int l, long long off) const {
  return shadow + (size_t)l * shadow_per_layer + off;
}

AdamShadow Ctx::shadow_desc() const {
  AdamShadow sh{};
  sh.shadow = shadow;
  sh.rm = shadow_rm;
  sh.at = shadow_at;
  sh.per_layer = lora_per_layer;
  for (int i = 0; i < 8; ++i) sh.seg_off[i] = seg_off[i];
  sh.d_in[0] = sh.d_in[1] = sh.d_in[2] = H;
  sh.d_in[3] = Q;
  sh.d_out[0] = Q;
  sh.d_out[1] = sh.d_out[2] = KV;
  sh.d_out[3] = H;
  sh.col_off[0] = 0;
  sh.col_off[1] = Q;
  sh.col_off[2] = Q + KV;
  sh.nt = NT;
  sh.shadow_per_layer = shadow_per_layer;
  sh.a_qkv = sh_a_qkv;
  sh.a_o = sh_a_o;
  sh.bt_qkv = sh_bt_qkv;
  sh.bt_o = sh_bt_o;
  return sh;
}

// ------------------------------------------------------------------ forward

// One decoder layer's forward (src/kernels/lora_forward.cu:198-298) from
// stash[l].x_in / stash[l].xn; writes the layer output to x_out and its
// RMSNorm with next_w (the next layer's attention norm, or the final norm)
// to xn_out.
hipError_t Ctx::layer_fwd(int l, int B, const float* next_w, float* x_out, _Float16* xn_out) {
  const int T = rows(B);
  const float eps = dims.eps;
  Layer& w = layers[l];
  Stash& s = stash[l];
  GemmOut go;
  // Q/K/V (+ the three LoRA A) projections in one GEMM; the epilogue adds
  // s (x A^T) B^T per projection from the h columns.
  BSeg sq[2] = {wseg(w.wqkv), hseg(shadow_ptr(l, sh_a_qkv), 3 * kRank, H)};
  const _Float16* bt_qkv = shadow_rm + (size_t)l * shadow_per_layer + sh_bt_qkv;
  const LoraTerm tq[3] = {{bt_qkv, 0, NT, 0, Q, 0},
                          {bt_qkv, kRank, NT, Q, KV, kRank},
                          {bt_qkv, 2 * kRank, NT, Q + KV, KV, 2 * kRank}};
  LLMT_HIP_TRY(gemm(CAT_GEMM_FWD, s.xn, H, sq, 2, T, H, nullptr, 0, &go));
  QkvPostArgs qa{};
  qa.in = row_in(go, NT, 3 * kRank, 3, tq);
  qa.qn = w.q_norm; qa.kn = w.k_norm;
  qa.cosT = cosT; qa.sinT = sinT;
  qa.S = S; qa.nq = nq; qa.nkv = nkv; qa.eps = eps;
  qa.qkraw = s.qkraw; qa.qkv16 = s.qkv16; qa.hbuf = s.h;
  // partials in; q/k raw (fp16), q/k/v (fp16) and the 48 h columns out
  LLMT_HIP_TRY(run(CAT_ROWS, "qkv_post", [=](hipStream_t q) { return qkv_post(qa, T, q); }, 0,
                   part_bytes(qa.in, T, NT) + (double)T * ((Q + KV) * 2 + NT * 2 + 48 * 4)));
  const AttnArgs aa = attn_args(s);
  // QK^T and PV: two causal S x S x 128 products per (sequence, query head)
  const double attn_prod = 2.0 * B * nq * (S * (S + 1.0) / 2.0) * kHeadDim;
  LLMT_HIP_TRY(run(CAT_ATTN, "attn_fwd", [=](hipStream_t q) { return attn_fwd(aa, B, q); },
                   2 * attn_prod));
  // O (+ LoRA A) projection, residual, FFN norm
  BSeg so[2] = {wseg(w.wo), hseg(shadow_ptr(l, sh_a_o), kRank, Q)};
  const LoraTerm to[1] = {{shadow_rm + (size_t)l * shadow_per_layer + sh_bt_o, 0, H, 0, H, 0}};
  LLMT_HIP_TRY(gemm(CAT_GEMM_FWD, s.o16, Q, so, 2, T, Q, nullptr, 0, &go));
  {
    const RowIn ri = row_in(go, H, kRank, 1, to);
    const float *x_in = s.x_in, *fw = w.ffn_norm;
    float *hb = s.h, *x_mid = s.x_mid;
    _Float16* xn2 = s.xn2;
    const int Hh = H;
    // partials and x_in in; x_mid (fp32), its norm (fp16) and h_o out
    LLMT_HIP_TRY(run(CAT_ROWS, "o_post", [=](hipStream_t q) {
      return o_post(ri, x_in, fw, eps, Hh, T, hb, x_mid, xn2, q);
    }, 0, part_bytes(ri, T, H) + (double)T * (H * 4 + H * 4 + H * 2 + 16 * 4)));
  }
  // gate/up, SwiGLU (in the GEMM epilogue where the large-tile kernel runs)
  BSeg sg[1] = {wseg(w.wgu)};
  if (gemm_glu_ok(T, I, H, sg[0].is_i8)) {
    LLMT_HIP_TRY(gemm(CAT_GEMM_FWD, s.xn2, H, sg, 1, T, H, nullptr, 0, nullptr, a16, s.gu));
  } else {
    LLMT_HIP_TRY(gemm(CAT_GEMM_FWD, s.xn2, H, sg, 1, T, H, nullptr, 0, &go));
    const RowIn ri = row_in(go);
    _Float16* gu = s.gu;
    _Float16* a = a16;
    const int Ii = I;
    LLMT_HIP_TRY(run(CAT_ROWS, "gu_post", [=](hipStream_t q) { return gu_post(ri, Ii, T, gu, a, q); },
                     0, part_bytes(ri, T, 2 * I) + (double)T * (2 * I * 2 + I * 2)));
  }
  // down, residual, next norm
  BSeg sd[1] = {wseg(w.wd)};
  LLMT_HIP_TRY(gemm(CAT_GEMM_FWD, a16, I, sd, 1, T, I, nullptr, 0, &go));
  {
    const RowIn ri = row_in(go);
    const float* x_mid = s.x_mid;
    const int Hh = H;
    LLMT_HIP_TRY(run(CAT_ROWS, "resid_norm", [=](hipStream_t q) {
      return resid_norm(ri, x_mid, next_w, eps, Hh, T, x_out, xn_out, q);
    }, 0, part_bytes(ri, T, H) + (double)T * (H * 4 + H * 4 + H * 2)));
  }
  return hipSuccess;
}

hipError_t Ctx::forward(const int* tok, int B, float* logits_out) {
  const int T = rows(B);
  {
    // the token gather fills the B * S real rows (the pad rows stay zero)
    const int nt = B * S;
    const _Float16* e = E;
    const int Vv = V, Hh = H;
    const float *w0 = layers[0].attn_norm, eps = dims.eps;
    float* x0 = stash[0].x_in;
    _Float16* xn0 = stash[0].xn;
    LLMT_HIP_TRY(run(CAT_ROWS, "embed_norm", [=](hipStream_t q) {
      return embed_norm(tok, e, Vv, Hh, w0, eps, nt, x0, xn0, q);
    }, 0, (double)nt * (4 + H * 2 + H * 4 + H * 2)));
  }
  for (int l = 0; l < L; ++l) {
    const bool last = l + 1 == L;
    LLMT_HIP_TRY(layer_fwd(l, B, last ? final_norm : layers[l + 1].attn_norm,
                           last ? x_final : stash[l + 1].x_in, last ? xf16 : stash[l + 1].xn));
  }
  // lm_head logits (tied embedding); into the context's logits with the
  // softmax pairs of the GEMM's column tiles for the fused cross entropy.
  // logits_out receives rows(B) rows.
  BSeg se[1] = {hseg(Eh, V, H)};
  if (logits_out) {
    head_tiles = 0;
    LLMT_HIP_TRY(gemm(CAT_GEMM_HEAD, xf16, H, se, 1, T, H, logits_out, V, nullptr));
  } else {
    LLMT_HIP_TRY(gemm(CAT_GEMM_HEAD, xf16, H, se, 1, T, H, logits, V, nullptr, nullptr, nullptr,
                      ce_stats, &head_tiles));
  }
  return hipSuccess;
}

hipError_t Ctx::ce(const float* lg, const int* tgt, int B, float* dlogits_out) {
  const float* x = lg ? lg : logits;
  const int rows = B * S, Vv = V, Ss = S;
  float2* stats = ce_stats;
  _Float16* g16c = grad16;
  float *lr = loss_rows, *lm = loss_dev, *lse = lse_rows;
  // the logits (fp32) in, the fp16 operand and optionally fp32 dlogits out
  const double out_bytes = (double)rows * V * (2 + (dlogits_out ? 4 : 0));
  if (!lg && head_tiles > 0) {  // the forward's logits with their tile pairs
    const int nt = head_tiles;
    LLMT_HIP_TRY(run(CAT_CE, "cross_entropy", [=](hipStream_t q) {
      return cross_entropy_from_stats(x, stats, nt, tgt, rows, Vv, Ss, lse, dlogits_out, g16c, lr,
                                      lm, q);
    }, 0, (double)rows * (V * 4.0 + nt * 8.0) + out_bytes));
    return hipSuccess;
  }
  // two reads of the logits (statistics, then the gradient)
  LLMT_HIP_TRY(run(CAT_CE, "cross_entropy", [=](hipStream_t q) {
    return cross_entropy(x, tgt, rows, Vv, Ss, stats, dlogits_out, g16c, lr, lm, q);
  }, 0, (double)rows * V * 8.0 + out_bytes));
  return hipSuccess;
}

AttnArgs Ctx::attn_args(const Stash& s) const {
  AttnArgs a{};
  a.q = s.qkv16;
  a.ldq = NT;
  a.k = s.qkv16 + Q;
  a.ldk = NT;
  a.v = s.qkv16 + Q + KV;
  a.ldv = NT;
  a.nq = nq;
  a.nkv = nkv;
  a.S = S;
  a.sm_scale = 1.0f / sqrtf((float)kHeadDim);
  a.o = s.o16;
  a.ldo = Q;
  a.lse = s.lse;
  a.dO16 = dO16;
  a.ld16 = Q;
  a.dsc = dsc;
  a.delta = delta;
  a.dq = dqkv32;
  a.ldgq = NT;
  a.dk = dqkv32 + Q;
  a.dv = dqkv32 + Q + KV;
  a.ldgkv = NT;
  return a;
}

// ------------------------------------------------------------------ backward

// lm_head dX over the vocabulary (from the fp16 grad16 = (p - onehot) * 2^14)
// and the final RMSNorm backward: leaves the residual-stream gradient in
// d_res and its fp16 operand in g16 / rinv.
hipError_t Ctx::head_bwd(int B) {
  const int T = rows(B);
  const float eps = dims.eps;
  const int n_valid = B * (S - 1);
  GemmOut go;
  // lm_head dX over the vocabulary, then the final RMSNorm backward.
  BSeg sh_[1] = {hseg(EhT, H, V)};
  LLMT_HIP_TRY(gemm(CAT_GEMM_HEAD, grad16, V, sh_, 1, T, V, nullptr, 0, &go));
  NormBwdArgs nb{};
  nb.in = row_in(go);
  nb.rinv_in = nullptr;
  nb.gscale = 1.0f / (kGradLogitScale * (float)n_valid);
  nb.dh_out = nullptr;
  nb.x = x_final;
  nb.w = final_norm;
  nb.eps = eps;
  nb.H = H;
  nb.dres_in = nullptr;
  nb.dres_out = d_res;
  nb.dmid_out = nullptr;
  nb.g16 = g16;
  nb.rinv_out = rinv;
  nb.g16_ks = layers[L - 1].wdT.kscale;  // g16 feeds the last layer's down dX
  // partials and x in; the residual gradient (fp32) and its fp16 operand out
  LLMT_HIP_TRY(run(CAT_ROWS, "norm_bwd_final", [=](hipStream_t q) { return norm_bwd(nb, T, q); },
                   0, part_bytes(nb.in, T, H) + (double)T * H * (4 + 4 + 2)));
  return hipSuccess;
}

// One decoder layer's backward (src/kernels/lora_backward.cu:271-406) from
// d_res / g16 / rinv (the gradient at the layer output); leaves the gradient
// at the layer input there and the layer's adapter-gradient inputs (dh, and
// the projections' upstream gradients as the fp16 GEMM operands with their
// row factors) in its per-layer slots for lora_grads.
hipError_t Ctx::layer_bwd(int l, int B) {
  const int T = rows(B);
  const float eps = dims.eps;
  GemmOut go_;
  NormBwdArgs nb{};

  Layer& w = layers[l];
  Stash& s = stash[l];
  float* const dh = this->dh(l);
  _Float16* const og16 = go16(l);  // o projection upstream gradient (fp16, row factor ro)
  _Float16* const qg16 = gq16(l);  // q/k/v projections upstream gradient (row factor rq)
  // MLP: down dX -> SwiGLU bwd -> gate/up dX -> FFN norm bwd (+ residual).
  // With int8 weights both dX GEMMs reduce over the weights' output channel,
  // whose scale their fp16 operands (g16, dgu16) already carry: the writers
  // fold it in per column, so these GEMMs dequantise without it.
  BSeg sd[1] = {wseg(w.wdT)};
  sd[0].kscale = nullptr;
  LLMT_HIP_TRY(gemm(CAT_GEMM_BWD, g16, H, sd, 1, T, H, nullptr, 0, &go_, nullptr, nullptr, nullptr,
                    nullptr, true));
  {
    const RowIn ri = row_in(go_);
    const float* ri_in = rinv;
    const _Float16* gu = s.gu;
    _Float16* d16 = dgu16;
    float* r2 = rinv2;
    const int Ii = I;
    const _Float16* ks = w.wguT.kscale;
    // partials and gate|up (fp16) in, dgate|dup (fp16) out
    LLMT_HIP_TRY(run(CAT_ROWS, "swiglu_bwd", [=](hipStream_t q) {
      return swiglu_bwd(ri, ri_in, gu, Ii, T, d16, r2, ks, q);
    }, 0, part_bytes(ri, T, I) + (double)T * (2 * I * 2 + 2 * I * 2)));
  }
  BSeg sg[1] = {wseg(w.wguT)};
  sg[0].kscale = nullptr;
  LLMT_HIP_TRY(gemm(CAT_GEMM_BWD, dgu16, 2 * I, sg, 1, T, 2 * I, nullptr, 0, &go_));
  nb = NormBwdArgs{};
  nb.in = row_in(go_);
  nb.rinv_in = rinv2;
  nb.gscale = 1.0f;
  nb.dh_out = nullptr;
  nb.x = s.x_mid;
  nb.w = w.ffn_norm;
  nb.eps = eps;
  nb.H = H;
  nb.dres_in = d_res;
  nb.dres_out = d_res;
  nb.dmid_out = nullptr;
  nb.g16 = og16;
  nb.rinv_out = ro(l);
  // partials, x and the residual gradient in; the residual gradient and its
  // fp16 operand out
  LLMT_HIP_TRY(run(CAT_ROWS, "norm_bwd", [=](hipStream_t q) { return norm_bwd(nb, T, q); }, 0,
                   part_bytes(nb.in, T, H) + (double)T * H * (4 + 4 + 4 + 2)));
  // O projection dX (+ dh_o through the B_o^T rows)
  // (int8: this GEMM and the Q/K/V dX apply the per-k weight scale in the
  // kernel; folded into their operands, the LoRA B^T rows riding in the same
  // A stream would need B^T / s, and dh, in the operands' units, would grow
  // by ~1 / s past the fp16 range of the LoRA norm backward's MFMA operand)
  BSeg so[2] = {wseg(w.woT), hseg(shadow_ptr(l, sh_bt_o), kRank, H)};
  const LoraTerm tbo[1] = {{shadow_rm + (size_t)l * shadow_per_layer + sh_a_o, 0, Q, 0, Q, 0}};
  LLMT_HIP_TRY(gemm(CAT_GEMM_BWD, og16, H, so, 2, T, H, nullptr, 0, &go_));
  {
    const RowIn ri = row_in(go_, Q, kRank, 1, tbo);
    const float* r = ro(l);
    const _Float16* o16 = s.o16;
    _Float16* d16 = dO16;
    float *de = delta, *ds = dsc;
    const int nqh = nq, Ss = S;
    // partials and O (fp16) in; dO (fp16), dh_o and delta / dsc out
    LLMT_HIP_TRY(run(CAT_ROWS, "o_dx_post", [=](hipStream_t q) {
      return o_dx_post(ri, r, o16, nqh, Ss, T, dh, d16, de, ds, q);
    }, 0, part_bytes(ri, T, Q) + (double)T * (Q * 2 + Q * 2 + 16 * 4 + nq * 8)));
  }
  // attention backward
  const AttnArgs aa = attn_args(s);
  // recomputed QK^T, dO V^T, P^T dO, dS^T Q, dS K: five causal products
  const double attn_prod = 2.0 * B * nq * (S * (S + 1.0) / 2.0) * kHeadDim;
  LLMT_HIP_TRY(run(CAT_ATTN, "attn_bwd", [=](hipStream_t q) { return attn_bwd(aa, B, q); },
                   5 * attn_prod));
  // RoPE + QK-norm backward
  QkBwdArgs qb{};
  qb.dqkv = dqkv32; qb.ld_dqkv = NT;
  qb.qkraw = s.qkraw;
  qb.qn = w.q_norm; qb.kn = w.k_norm;
  qb.cosT = cosT; qb.sinT = sinT;
  qb.S = S; qb.nq = nq; qb.nkv = nkv; qb.eps = eps;
  qb.dy32 = nullptr; qb.g16 = qg16; qb.rinv_out = rq(l);
  // dq/dk/dv (fp32) and q/k raw (fp16) in, the fp16 operand out
  LLMT_HIP_TRY(run(CAT_ROWS, "qk_bwd", [=](hipStream_t q) { return qk_bwd(qb, T, q); }, 0,
                   (double)T * (NT * 4 + (Q + KV) * 2 + NT * 2)));
  // Q/K/V dX (+ dh_q, dh_k, dh_v through the B^T rows), attention norm bwd
  BSeg sq[2] = {wseg(w.wqkvT), hseg(shadow_ptr(l, sh_bt_qkv), 3 * kRank, NT)};
  const _Float16* a_qkv = shadow_rm + (size_t)l * shadow_per_layer + sh_a_qkv;
  const LoraTerm tbq[3] = {{a_qkv, 0, H, 0, H, 0},
                           {a_qkv, kRank, H, 0, H, kRank},
                           {a_qkv, 2 * kRank, H, 0, H, 2 * kRank}};
  LLMT_HIP_TRY(gemm(CAT_GEMM_BWD, qg16, NT, sq, 2, T, NT, nullptr, 0, &go_));
  nb = NormBwdArgs{};
  nb.in = row_in(go_, H, 3 * kRank, 3, tbq);
  nb.rinv_in = rq(l);
  nb.gscale = 1.0f;
  nb.dh_out = dh;
  nb.dh_col = 0;
  nb.x = s.x_in;
  nb.w = w.attn_norm;
  nb.eps = eps;
  nb.H = H;
  nb.dres_in = d_res;
  nb.dres_out = d_res;
  nb.dmid_out = nullptr;
  nb.g16 = g16;
  nb.rinv_out = rinv;
  nb.g16_ks = l > 0 ? layers[l - 1].wdT.kscale : nullptr;  // g16 feeds layer l - 1's down dX
  nb.lora_at = shadow_at + (size_t)l * H * 3 * kRank;
  LLMT_HIP_TRY(run(CAT_ROWS, "norm_bwd_lora", [=](hipStream_t q) { return norm_bwd(nb, T, q); },
                   0, part_bytes(nb.in, T, H) + (double)T * (H * (4 + 4 + 4 + 2) + 48 * 4)));
  return hipSuccess;
}

hipError_t Ctx::lora_grads(int l0, int nl, int B, int accumulate) {
  const LoraGradJob* jobs = lora_jobs + (size_t)l0 * kLoraJobs;
  const LoraGradPlan plan = lora_plan;
  const float ls = lscale;
  const int T = rows(B);
  // per layer: the dA inputs (xn three times, o; fp16) and the dB inputs
  // (the two fp16 gradient operands) with the h / dh columns (fp32), the
  // gradients out (fp32)
  const double per_layer = (double)T * ((3.0 * H + Q) * 2 + (NT + H) * 2 + 2 * 64 * 4) +
                           (double)lora_per_layer * 4 * (accumulate ? 2 : 1);
  return run(CAT_LORA, "lora_grad", [=](hipStream_t q) {
    return lora_grad(jobs, plan, nl, T, ls, accumulate, q);
  }, 0, per_layer * nl);
}

hipError_t Ctx::backward(int B, int accumulate) {
  LLMT_HIP_TRY(head_bwd(B));
  for (int l = L - 1; l >= 0; --l) LLMT_HIP_TRY(layer_bwd(l, B));
  // every layer's adapter gradients in one launch
  LLMT_HIP_TRY(lora_grads(0, L, B, accumulate));
  return hipSuccess;
}

hipError_t Ctx::optimizer() {
  float *p = lora_p, *g = lora_g, *m = lora_m, *v = lora_v;
  const long long n = (long long)lora_numel;
  const AdamHp* hp = hp_dev;
  const AdamShadow sh = shadow_desc();
  // p, g, m, v in; p, m, v and the two fp16 copies of p out
  LLMT_HIP_TRY(run(CAT_ADAM, "adamw", [=](hipStream_t q) { return adamw(p, g, m, v, n, hp, 1, sh, q); },
                   0, (double)n * (7 * 4 + 2 * 2)));
  return hipSuccess;
}

hipError_t Ctx::refresh_shadows() {
  LLMT_HIP_TRY(adamw(lora_p, nullptr, nullptr, nullptr, (long long)lora_numel, hp_dev, 0,
                     shadow_desc(), st));
  return hipSuccess;
}

hipError_t Ctx::device_step(int B, int with_adam, const int* tok, const int* tgt) {
  LLMT_HIP_TRY(forward(tok ? tok : tok_buf, B, nullptr));
  LLMT_HIP_TRY(ce(nullptr, tgt ? tgt : tgt_buf, B, nullptr));
  LLMT_HIP_TRY(backward(B, 0));
  if (with_adam) LLMT_HIP_TRY(optimizer());
  return hipSuccess;
}

}  // namespace llmt

// ====================================================================== C ABI

#define TRY_ARG(cond, ...)          \
  do {                              \
    if (!(cond)) {                  \
      set_error(__VA_ARGS__);       \
      return LLMT_ERR_ARG;          \
    }                               \
  } while (0)

#define TRY_HIP(expr)                                                         \
  do {                                                                        \
    hipError_t e__ = (expr);                                                  \
    if (e__ != hipSuccess) {                                                  \
      if (e__ != hipErrorInvalidValue || !llmt_last_error()[0])               \
        set_error("%s: %s", #expr, hipGetErrorString(e__));                   \
      return e__ == hipErrorInvalidValue ? LLMT_ERR_ARG : LLMT_ERR_HIP;       \
    }                                                                         \
  } while (0)

static Ctx* C_(llmt_ctx* c) { return reinterpret_cast<Ctx*>(c); }
static const Ctx* C_(const llmt_ctx* c) { return reinterpret_cast<const Ctx*>(c); }

extern "C" {

int llmt_ctx_create(const llmt_dims* dims, int max_batch, int seq_len, int weight_format,
                    void* stream, llmt_ctx** out) {
  set_error("");
  TRY_ARG(dims && out, "llmt_ctx_create: NULL argument");
  TRY_ARG(dims->head_dim == kHeadDim, "head_dim must be %d (got %d)", kHeadDim, dims->head_dim);
  TRY_ARG(dims->rank == kRank, "LoRA rank must be %d (got %d)", kRank, dims->rank);
  TRY_ARG(dims->n_heads > 0 && dims->n_kv_heads > 0 && dims->n_heads % dims->n_kv_heads == 0,
          "n_heads must be a multiple of n_kv_heads");
  TRY_ARG(dims->hidden % 64 == 0 && dims->intermediate % 64 == 0 && dims->vocab % 64 == 0,
          "hidden, intermediate and vocab must be multiples of 64");
  TRY_ARG(dims->n_layers >= 1, "n_layers >= 1");
  TRY_ARG(max_batch >= 1 && seq_len >= 2, "max_batch >= 1 and seq_len >= 2");
  TRY_ARG(weight_format == LLMT_WEIGHTS_F16 || weight_format == LLMT_WEIGHTS_I8,
          "weight_format");
  Ctx* c = new Ctx();
  c->dims = *dims;
  c->maxB = max_batch;
  c->S = seq_len;
  c->wfmt = weight_format;
  c->st = (hipStream_t)stream;
  if (!c->st) {
    // A stream of its own (graph capture needs one); created blocking, so it
    // stays ordered with work on the legacy default stream.
    if (hipStreamCreate(&c->st) != hipSuccess) {
      delete c;
      set_error("llmt_ctx_create: hipStreamCreate failed");
      return LLMT_ERR_HIP;
    }
    c->own_stream = true;
  }
  int rc = c->init();
  if (rc != LLMT_OK) {
    delete c;
    return rc;
  }
  *out = reinterpret_cast<llmt_ctx*>(c);
  return LLMT_OK;
}

int llmt_ctx_destroy(llmt_ctx* ctx) {
  if (ctx) {
    hipStreamSynchronize(C_(ctx)->st);
    delete C_(ctx);
  }
  return LLMT_OK;
}

size_t llmt_ctx_device_bytes(const llmt_ctx* ctx) { return ctx ? C_(ctx)->device_bytes : 0; }

size_t llmt_lora_numel(const llmt_ctx* ctx) { return ctx ? C_(ctx)->lora_numel : 0; }

size_t llmt_lora_offset(const llmt_ctx* ctx, int layer, int proj, int is_b) {
  const Ctx* c = C_(ctx);
  if (!c || layer < 0 || layer >= c->L || proj < 0 || proj > 3) return (size_t)-1;
  return (size_t)layer * c->lora_per_layer + c->seg_off[2 * proj + (is_b ? 1 : 0)];
}

int llmt_lora_copy(llmt_ctx* ctx, int kind, float* buf, int to_ctx) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && buf && kind >= 0 && kind <= 3, "llmt_lora_copy: bad arguments");
  float* arena[4] = {c->lora_p, c->lora_g, c->lora_m, c->lora_v};
  const size_t bytes = c->lora_numel * sizeof(float);
  if (to_ctx) {
    TRY_HIP(hipMemcpyAsync(arena[kind], buf, bytes, hipMemcpyDefault, c->st));
    if (kind == LLMT_LORA_PARAM) TRY_HIP(c->refresh_shadows());
  } else {
    TRY_HIP(hipMemcpyAsync(buf, arena[kind], bytes, hipMemcpyDefault, c->st));
  }
  TRY_HIP(hipStreamSynchronize(c->st));
  return LLMT_OK;
}

int llmt_lora_init(llmt_ctx* ctx, uint64_t seed, float a_std, float b_std) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c, "llmt_lora_init: NULL ctx");
  TRY_HIP(lora_init(c->lora_p, c->lora_m, c->lora_v, (long long)c->lora_numel, seed, a_std, b_std,
                    c->shadow_desc(), c->st));
  TRY_HIP(hipMemsetAsync(c->lora_g, 0, c->lora_numel * sizeof(float), c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  return LLMT_OK;
}

static int check_tokens(Ctx* c, const int* tokens, const int* targets, int batch) {
  TRY_ARG(c && tokens && targets, "NULL argument");
  TRY_ARG(batch >= 1 && batch <= c->maxB, "batch %d outside [1, %d]", batch, c->maxB);
  TRY_ARG(c->weights_ready(), "frozen weights not set (llmt_set_layer_* / llmt_set_embed_f16)");
  return LLMT_OK;
}

static int stage_inputs(Ctx* c, const int* tokens, const int* targets, int batch) {
  const size_t n = (size_t)batch * c->S * sizeof(int);
  TRY_HIP(hipMemcpyAsync(c->tok_buf, tokens, n, hipMemcpyDefault, c->st));
  TRY_HIP(hipMemcpyAsync(c->tgt_buf, targets, n, hipMemcpyDefault, c->st));
  return LLMT_OK;
}

// AdamW hyper-parameters of `step` into the pinned staging slot (copied to
// the device by set_hp, or by the step graph's own copy node).
static int set_hp_host(Ctx* c, const llmt_hparams* hp, int step) {
  TRY_ARG(hp && step >= 1, "llmt_step: hparams NULL or step < 1");
  AdamHp h{};
  h.lr = hp->lr;
  h.beta1 = hp->beta1;
  h.beta2 = hp->beta2;
  h.eps = hp->eps;
  h.wd = hp->wd;
  // src/kernels/lora.cu:238-239: bias corrections in fp32 with powf.
  h.bc1 = 1.0f - powf(hp->beta1, (float)step);
  h.bc2 = 1.0f - powf(hp->beta2, (float)step);
  // The pinned staging slot may still be read by an in-flight copy of the
  // previous step; the stream is idle here (every step ends synchronised).
  *c->host_hp = h;
  return LLMT_OK;
}

static int set_hp(Ctx* c, const llmt_hparams* hp, int step) {
  int rc = set_hp_host(c, hp, step);
  if (rc) return rc;
  TRY_HIP(hipMemcpyAsync(c->hp_dev, c->host_hp, sizeof(AdamHp), hipMemcpyHostToDevice, c->st));
  return LLMT_OK;
}

// Graph replays take the input copies (tokens, targets, and the staged
// hyper-parameters when the step has AdamW) as nodes of the step graph, so a
// step is one launch; the graph is keyed by the token/target pointers.  A
// caller whose pointers change between steps would rebuild it every step, so
// the first change switches the context to copies outside the graph (one
// rebuild, then the graph is reused whatever the pointers).
static bool graph_inputs(Ctx* c, const int* tokens, const int* targets) {
  if (!c->use_graph || c->recording || c->inputs_move) return false;
  if (c->graph_exec && c->graph_tok && (c->graph_tok != tokens || c->graph_tgt != targets)) {
    c->inputs_move = true;
    return false;
  }
  return true;
}

// tokens/targets non-NULL: the graph's kernels read the caller's token and
// target buffers in place (the graph is keyed by those pointers), the staged
// hyper-parameters (with AdamW) are copied inside the graph, and so is the
// loss read-back, so a step is one graph launch and one wait.
static int run_step(Ctx* c, int batch, int with_adam, float* loss_host,
                    const int* tokens = nullptr, const int* targets = nullptr) {
  TRY_HIP(c->clear_pad_rows(batch));
  if (c->use_graph && !c->recording) {
    if (!c->graph_exec || c->graph_batch != batch || c->graph_adam != with_adam ||
        c->graph_tok != tokens || c->graph_tgt != targets) {
      if (c->graph_exec) {
        hipGraphExecDestroy(c->graph_exec);
        c->graph_exec = nullptr;
      }
      hipGraph_t g = nullptr;
      TRY_HIP(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
      hipError_t e = hipSuccess;
      if (tokens && with_adam)
        e = hipMemcpyAsync(c->hp_dev, c->host_hp, sizeof(AdamHp), hipMemcpyHostToDevice, c->st);
      if (e == hipSuccess) e = c->device_step(batch, with_adam, tokens, targets);
      if (e == hipSuccess)
        e = hipMemcpyAsync(c->host_loss, c->loss_dev, sizeof(float), hipMemcpyDeviceToHost, c->st);
      hipError_t e2 = hipStreamEndCapture(c->st, &g);
      if ((e != hipSuccess || e2 != hipSuccess) && g) hipGraphDestroy(g);
      TRY_HIP(e);
      TRY_HIP(e2);
      e = hipGraphInstantiate(&c->graph_exec, g, nullptr, nullptr, 0);
      hipGraphDestroy(g);
      TRY_HIP(e);
      c->graph_batch = batch;
      c->graph_adam = with_adam;
      c->graph_tok = tokens;
      c->graph_tgt = targets;
    }
    TRY_HIP(hipGraphLaunch(c->graph_exec, c->st));
  } else {
    TRY_HIP(c->device_step(batch, with_adam));
    TRY_HIP(hipMemcpyAsync(c->host_loss, c->loss_dev, sizeof(float), hipMemcpyDeviceToHost, c->st));
  }
  TRY_HIP(hipStreamSynchronize(c->st));
  if (loss_host) *loss_host = *c->host_loss;
  return LLMT_OK;
}

int llmt_step(llmt_ctx* ctx, const int* tokens, const int* targets, int batch,
              const llmt_hparams* hp, int step, float* loss_host) {
  set_error("");
  Ctx* c = C_(ctx);
  int rc = check_tokens(c, tokens, targets, batch);
  if (rc) return rc;
  if (graph_inputs(c, tokens, targets)) {
    if ((rc = set_hp_host(c, hp, step))) return rc;
    return run_step(c, batch, 1, loss_host, tokens, targets);
  }
  if ((rc = set_hp(c, hp, step))) return rc;
  if ((rc = stage_inputs(c, tokens, targets, batch))) return rc;
  return run_step(c, batch, 1, loss_host);
}

int llmt_forward_backward(llmt_ctx* ctx, const int* tokens, const int* targets, int batch,
                          float* loss_host) {
  set_error("");
  Ctx* c = C_(ctx);
  int rc = check_tokens(c, tokens, targets, batch);
  if (rc) return rc;
  if (graph_inputs(c, tokens, targets)) return run_step(c, batch, 0, loss_host, tokens, targets);
  if ((rc = stage_inputs(c, tokens, targets, batch))) return rc;
  return run_step(c, batch, 0, loss_host);
}

int llmt_adamw(llmt_ctx* ctx, const llmt_hparams* hp, int step) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c, "NULL ctx");
  int rc = set_hp(c, hp, step);
  if (rc) return rc;
  TRY_HIP(c->optimizer());
  TRY_HIP(hipStreamSynchronize(c->st));
  return LLMT_OK;
}

int llmt_set_graph(llmt_ctx* ctx, int enable) {
  Ctx* c = C_(ctx);
  if (!c) return LLMT_ERR_ARG;
  c->use_graph = enable != 0;
  if (!c->use_graph && c->graph_exec) {
    hipGraphExecDestroy(c->graph_exec);
    c->graph_exec = nullptr;
  }
  return LLMT_OK;
}

const float* llmt_logits(const llmt_ctx* ctx) { return ctx ? C_(ctx)->logits : nullptr; }

const float* llmt_layer_in(const llmt_ctx* ctx, int layer) {
  const Ctx* c = C_(ctx);
  return c && layer >= 0 && layer < c->L ? c->stash[layer].x_in : nullptr;
}

// Times `fns` replayed back to back `reps` times as one captured graph
// (after one warm-up launch): the average duration of one of them in us.
static int replay_us(Ctx* c, const std::vector<const Launch*>& fns, int reps, float* us) {
  hipGraph_t gph = nullptr;
  hipGraphExec_t ex = nullptr;
  TRY_HIP(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
  hipError_t e = hipSuccess;
  for (const Launch* l : fns)
    if (e == hipSuccess) e = l->fn(c->st);
  hipError_t e2 = hipStreamEndCapture(c->st, &gph);
  if ((e != hipSuccess || e2 != hipSuccess) && gph) hipGraphDestroy(gph);
  TRY_HIP(e);
  TRY_HIP(e2);
  e = hipGraphInstantiate(&ex, gph, nullptr, nullptr, 0);
  hipGraphDestroy(gph);
  TRY_HIP(e);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipGraphLaunch(ex, c->st);  // warm
  if (e == hipSuccess) e = hipEventRecord(e0, c->st);
  for (int r = 0; r < reps && e == hipSuccess; ++r) e = hipGraphLaunch(ex, c->st);
  if (e == hipSuccess) e = hipEventRecord(e1, c->st);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  hipGraphExecDestroy(ex);
  TRY_HIP(e);
  *us = ms * 1e3f / (float)(reps * fns.size());
  return LLMT_OK;
}

int llmt_profile_kernels(llmt_ctx* ctx, const int* tokens, const int* targets, int batch,
                         const llmt_hparams* hp, int step, int reps, int max_kinds, int* nkinds,
                         const char** names, int* cats, int* launches, float* us, double* flops,
                         double* bytes) {
  set_error("");
  Ctx* c = C_(ctx);
  int rc = check_tokens(c, tokens, targets, batch);
  if (rc) return rc;
  TRY_ARG(nkinds && names && cats && launches && us && flops && bytes && reps >= 1 &&
              max_kinds >= 1,
          "llmt_profile_kernels: outputs, reps, max_kinds");
  if ((rc = set_hp(c, hp, step))) return rc;
  if ((rc = stage_inputs(c, tokens, targets, batch))) return rc;
  // 1. one eager step, every launch recorded
  c->recording = true;
  c->launches.clear();
  rc = run_step(c, batch, 1, nullptr);
  c->recording = false;
  if (rc) return rc;
  // 2. group by kind, in first-seen order
  std::vector<std::vector<const Launch*>> groups;
  std::vector<std::string> keys;
  for (const Launch& l : c->launches) {
    size_t j = 0;
    while (j < keys.size() && keys[j] != l.kind) ++j;
    if (j == keys.size()) {
      keys.push_back(l.kind);
      groups.emplace_back();
    }
    groups[j].push_back(&l);
  }
  // 3. replay each kind on its own.  AdamW replays would step the adapters
  // again: the arenas are saved first and restored after.
  const size_t nb = c->lora_numel * sizeof(float);
  float* saved = nullptr;
  TRY_HIP(hipMalloc(&saved, 3 * nb));
  float* arena[3] = {c->lora_p, c->lora_m, c->lora_v};
  hipError_t e = hipSuccess;
  for (int i = 0; i < 3 && e == hipSuccess; ++i)
    e = hipMemcpyAsync((char*)saved + i * nb, arena[i], nb, hipMemcpyDeviceToDevice, c->st);
  const int nk = (int)std::min<size_t>(groups.size(), (size_t)max_kinds);
  c->prof_names = keys;
  for (int k = 0; k < nk && rc == LLMT_OK && e == hipSuccess; ++k) {
    rc = replay_us(c, groups[k], reps, &us[k]);
    const Launch& l0 = *groups[k][0];
    names[k] = c->prof_names[k].c_str();
    cats[k] = l0.cat;
    launches[k] = (int)groups[k].size();
    flops[k] = l0.flops;
    bytes[k] = l0.bytes;
  }
  for (int i = 0; i < 3 && e == hipSuccess; ++i)
    e = hipMemcpyAsync(arena[i], (char*)saved + i * nb, nb, hipMemcpyDeviceToDevice, c->st);
  if (e == hipSuccess) e = c->refresh_shadows();
  if (e == hipSuccess) e = hipStreamSynchronize(c->st);
  hipFree(saved);
  c->launches.clear();
  if (rc) return rc;
  TRY_HIP(e);
  *nkinds = nk;
  return LLMT_OK;
}

}  // extern "C"
