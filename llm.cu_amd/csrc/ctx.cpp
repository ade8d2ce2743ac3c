// ctx.cpp — context set-up: buffer layout, frozen-weight upload (with the
// pre-transposed copies the backward GEMMs stream), the reference's on-disk
// weight and adapter formats, and the single-layer entry points of config C0.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "ctx.h"

using namespace llmt;

#define TRY_ARG(cond, ...)    \
  do {                        \
    if (!(cond)) {            \
      set_error(__VA_ARGS__); \
      return LLMT_ERR_ARG;    \
    }                         \
  } while (0)

#define TRY_HIP(expr)                                                   \
  do {                                                                  \
    hipError_t e__ = (expr);                                            \
    if (e__ != hipSuccess) {                                            \
      if (e__ != hipErrorInvalidValue || !llmt_last_error()[0])         \
        set_error("%s: %s", #expr, hipGetErrorString(e__));             \
      return e__ == hipErrorInvalidValue ? LLMT_ERR_ARG : LLMT_ERR_HIP; \
    }                                                                   \
  } while (0)

#define TRY_PTR(p)                 \
  do {                             \
    if (!(p)) return LLMT_ERR_HIP; \
  } while (0)

namespace llmt {

int Ctx::init() {
  H = dims.hidden;
  nq = dims.n_heads;
  nkv = dims.n_kv_heads;
  Q = nq * kHeadDim;
  KV = nkv * kHeadDim;
  NT = Q + 2 * KV;
  I = dims.intermediate;
  V = dims.vocab;
  L = dims.n_layers;
  Tmax = rows(maxB);
  lscale = dims.alpha / (float)dims.rank;
  const long long R = kRank;

  // adapter arena, per layer: q A, q B, k A, k B, v A, v B, o A, o B
  const long long sz[8] = {R * H, (long long)Q * R, R * H, (long long)KV * R,
                           R * H, (long long)KV * R, R * Q, (long long)H * R};
  long long off = 0;
  for (int i = 0; i < 8; ++i) {
    seg_off[i] = off;
    off += sz[i];
  }
  lora_per_layer = (size_t)off;
  lora_numel = lora_per_layer * L;
  sh_a_qkv = 0;
  sh_a_o = 3 * R * H;
  sh_bt_qkv = sh_a_o + R * Q;
  sh_bt_o = sh_bt_qkv + 3 * R * NT;
  shadow_per_layer = sh_bt_o + R * H;

  TRY_PTR(lora_p = alloc_n<float>(lora_numel));
  TRY_PTR(lora_g = alloc_n<float>(lora_numel));
  TRY_PTR(lora_m = alloc_n<float>(lora_numel));
  TRY_PTR(lora_v = alloc_n<float>(lora_numel));
  TRY_PTR(shadow = alloc_n<_Float16>(shadow_per_layer * L));
  TRY_PTR(shadow_rm = alloc_n<_Float16>(shadow_per_layer * L));
  TRY_PTR(shadow_at = alloc_n<_Float16>((size_t)L * H * 3 * R));
  TRY_PTR(hp_dev = alloc_n<AdamHp>(1));
  TRY_HIP(hipMemset(lora_p, 0, lora_numel * sizeof(float)));
  TRY_HIP(hipMemset(lora_g, 0, lora_numel * sizeof(float)));
  TRY_HIP(hipMemset(lora_m, 0, lora_numel * sizeof(float)));
  TRY_HIP(hipMemset(lora_v, 0, lora_numel * sizeof(float)));
  TRY_HIP(hipMemset(shadow, 0, shadow_per_layer * L * sizeof(_Float16)));
  TRY_HIP(hipMemset(shadow_rm, 0, shadow_per_layer * L * sizeof(_Float16)));
  TRY_HIP(hipMemset(shadow_at, 0, (size_t)L * H * 3 * R * sizeof(_Float16)));

  // RoPE tables: angles in double, rounded once to fp32 (src/kernels/rope.cu:15-18).
  {
    std::vector<float> c((size_t)S * 64), s((size_t)S * 64);
    for (int p = 0; p < S; ++p)
      for (int d = 0; d < 64; ++d) {
        const double freq = 1.0 / pow((double)dims.theta, 2.0 * d / kHeadDim);
        const double ang = (double)p * freq;
        c[(size_t)p * 64 + d] = (float)cos(ang);
        s[(size_t)p * 64 + d] = (float)sin(ang);
      }
    TRY_PTR(cosT = alloc_n<float>(c.size()));
    TRY_PTR(sinT = alloc_n<float>(s.size()));
    TRY_HIP(hipMemcpy(cosT, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice));
    TRY_HIP(hipMemcpy(sinT, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice));
  }

  // frozen weights
  layers.resize(L);
  const size_t mats[4][2] = {{(size_t)NT, (size_t)H}, {(size_t)H, (size_t)Q},
                             {(size_t)2 * I, (size_t)H}, {(size_t)H, (size_t)I}};
  const int esz = wfmt == LLMT_WEIGHTS_I8 ? 1 : 2;
  for (int l = 0; l < L; ++l) {
    Layer& w = layers[l];
    WMat* fw[4] = {&w.wqkv, &w.wo, &w.wgu, &w.wd};
    WMat* bw[4] = {&w.wqkvT, &w.woT, &w.wguT, &w.wdT};
    for (int m = 0; m < 4; ++m) {
      const size_t rows = mats[m][0], cols = mats[m][1];
      void* f = alloc(rows * cols * esz);
      void* b = alloc(rows * cols * esz);
      TRY_PTR(f);
      TRY_PTR(b);
      fw[m]->p = f;
      fw[m]->rows = (int)rows;
      fw[m]->ld = (int)cols;
      fw[m]->i8 = esz == 1;
      bw[m]->p = b;
      bw[m]->rows = (int)cols;
      bw[m]->ld = (int)rows;
      bw[m]->i8 = esz == 1;
      if (esz == 1) {
        _Float16* sc = alloc_n<_Float16>(rows);
        TRY_PTR(sc);
        fw[m]->colscale = sc;
        bw[m]->kscale = sc;
      }
    }
    float* nw = alloc_n<float>(2 * H + 2 * kHeadDim);
    TRY_PTR(nw);
    w.attn_norm = nw;
    w.ffn_norm = nw + H;
    w.q_norm = nw + 2 * H;
    w.k_norm = nw + 2 * H + kHeadDim;
  }
  TRY_PTR(E = alloc_n<_Float16>((size_t)V * H));
  TRY_PTR(ET = alloc_n<_Float16>((size_t)V * H));
  Eh = E;
  EhT = ET;
  TRY_PTR(final_norm = alloc_n<float>(H));

  // per-layer stashes
  const size_t T = Tmax;
  stash.resize(L);
  for (int l = 0; l < L; ++l) {
    Stash& s = stash[l];
    TRY_PTR(s.x_in = alloc_n<float>(T * H));
    TRY_PTR(s.xn = alloc_n<_Float16>(T * H));
    TRY_PTR(s.qkraw = alloc_n<_Float16>(T * (Q + KV)));
    TRY_PTR(s.qkv16 = alloc_n<_Float16>(T * NT));
    TRY_PTR(s.h = alloc_n<float>(T * 64));
    TRY_PTR(s.o16 = alloc_n<_Float16>(T * Q));
    TRY_PTR(s.lse = alloc_n<float>((size_t)maxB * nq * S));
    TRY_PTR(s.x_mid = alloc_n<float>(T * H));
    TRY_PTR(s.xn2 = alloc_n<_Float16>(T * H));
    TRY_PTR(s.gu = alloc_n<_Float16>(T * 2 * I));
  }
  TRY_PTR(x_final = alloc_n<float>(T * H));
  TRY_PTR(xf16 = alloc_n<_Float16>(T * H));
  TRY_PTR(logits = alloc_n<float>(T * V));
  TRY_PTR(grad16 = alloc_n<_Float16>(T * V));
  TRY_PTR(ce_stats = alloc_n<float2>((size_t)T * ce_stats_per_row(V)));
  TRY_PTR(lse_rows = alloc_n<float>(T));
  TRY_PTR(loss_rows = alloc_n<float>(T));
  TRY_PTR(loss_dev = alloc_n<float>(1));
  TRY_PTR(tok_buf = alloc_n<int>(T));
  TRY_PTR(tgt_buf = alloc_n<int>(T));
  TRY_HIP(hipMemset(tok_buf, 0, T * sizeof(int)));
  TRY_HIP(hipMemset(tgt_buf, 0, T * sizeof(int)));

  // split-K partials: the largest split * M * N over every GEMM of the step
  const int shapes[9][2] = {{NT + 3 * kRank, H}, {H + kRank, Q}, {2 * I, H}, {H, I},
                            {H, V},              {I, H},         {H, 2 * I}, {Q + kRank, H},
                            {H + 3 * kRank, NT}};
  part_elems = 0;
  for (int b = 1; b <= maxB; ++b) {
    const int M = rows(b);
    for (auto& sh : shapes) {
      const int split = gemm_split_col(M, sh[0], sh[1]) ? 2 : gemm_pick_split(M, sh[0], sh[1], 64);
      const size_t e = (size_t)split * M * sh[0];
      if (e > part_elems) part_elems = e;
    }
  }
  if (part_elems == 0) part_elems = 1;
  TRY_PTR(part = alloc_n<float>(part_elems));
  TRY_PTR(a16 = alloc_n<_Float16>(T * I));
  TRY_PTR(d_res = alloc_n<float>(T * H));
  TRY_PTR(go16_all = alloc_n<_Float16>((size_t)L * T * H));
  TRY_PTR(ro_all = alloc_n<float>((size_t)L * T));
  TRY_PTR(g16 = alloc_n<_Float16>(T * (H > NT ? H : NT)));
  TRY_PTR(rinv = alloc_n<float>(T));
  TRY_PTR(rinv2 = alloc_n<float>(T));
  TRY_PTR(dgu16 = alloc_n<_Float16>(T * 2 * I));
  // [B, nq, S] per sequence; the O-projection epilogue also writes the pad
  // rows (row t at sequence t / S, position t % S), so whole sequences up to
  // row Tmax - 1 are allocated.
  const size_t nseq_pad = ((size_t)Tmax + S - 1) / S;
  TRY_PTR(delta = alloc_n<float>(nseq_pad * nq * S));
  TRY_PTR(dsc = alloc_n<float>(nseq_pad * nq * S));
  TRY_PTR(dqkv32 = alloc_n<float>(T * NT));
  TRY_PTR(dO16 = alloc_n<_Float16>((size_t)T * Q));
  TRY_PTR(gq16_all = alloc_n<_Float16>((size_t)L * T * NT));
  TRY_PTR(rq_all = alloc_n<float>((size_t)L * T));
  TRY_PTR(dh_all = alloc_n<float>((size_t)L * T * 64));
  // adapter-gradient jobs (src/kernels/lora_backward.cu:50-90): per layer
  // dA_p = s dh_p^T x_p and dB_p = s dy_p^T h_p for p = q, k, v, o
  {
    std::vector<LoraGradJob> jobs((size_t)L * kLoraJobs);
    for (int l = 0; l < L; ++l) {
      const Stash& s = stash[l];
      float* dhl = dh(l);
      const _Float16* gql = gq16(l);
      auto g = [&](int proj, int is_b) {
        return lora_g + (size_t)l * lora_per_layer + seg_off[2 * proj + is_b];
      };
      const LoraGradJob js[kLoraJobs] = {
          {s.xn, 1, H, nullptr, H, dhl + 0, 64, g(0, 0), 0},
          {s.xn, 1, H, nullptr, H, dhl + 16, 64, g(1, 0), 0},
          {s.xn, 1, H, nullptr, H, dhl + 32, 64, g(2, 0), 0},
          {s.o16, 1, Q, nullptr, Q, dhl + 48, 64, g(3, 0), 0},
          {gql, 1, NT, rq(l), Q, s.h + 0, 64, g(0, 1), 1},
          {gql + Q, 1, NT, rq(l), KV, s.h + 16, 64, g(1, 1), 1},
          {gql + Q + KV, 1, NT, rq(l), KV, s.h + 32, 64, g(2, 1), 1},
          {go16(l), 1, H, ro(l), H, s.h + 48, 64, g(3, 1), 1},
      };
      for (int j = 0; j < kLoraJobs; ++j) jobs[(size_t)l * kLoraJobs + j] = js[j];
      if (l == 0)
        for (int j = 0; j < kLoraJobs; ++j) lora_plan.ncols[j] = js[j].ncols;
    }
    TRY_PTR(lora_jobs = alloc_n<LoraGradJob>(jobs.size()));
    if (hipMemcpy(lora_jobs, jobs.data(), jobs.size() * sizeof(LoraGradJob),
                  hipMemcpyHostToDevice) != hipSuccess) {
      set_error("init: job table upload failed");
      return LLMT_ERR_HIP;
    }
  }

  TRY_HIP(hipHostMalloc((void**)&host_loss, sizeof(float), hipHostMallocDefault));
  TRY_HIP(hipHostMalloc((void**)&host_hp, sizeof(AdamHp), hipHostMallocDefault));
  *host_loss = 0.f;
  TRY_HIP(hipDeviceSynchronize());
  return LLMT_OK;
}

}  // namespace llmt

static Ctx* C_(llmt_ctx* c) { return reinterpret_cast<Ctx*>(c); }

// Pack a row-major [rows, cols] matrix into rows [r0, r0 + rows) of the
// forward operand f (row length cols) and, transposed, into k range
// [r0, r0 + rows) of the backward operand b (row length = f's row count).
static hipError_t put_f16(Ctx* c, const void* src, int rows, int cols, const WMat& f, int r0,
                          const WMat& b) {
  LLMT_HIP_TRY(pack_f16((const _Float16*)src, cols, 0, rows, cols, (_Float16*)f.p, f.ld, r0, 0,
                        c->st));
  return pack_f16((const _Float16*)src, cols, 1, cols, rows, (_Float16*)b.p, b.ld, 0, r0, c->st);
}

// Rows whose fp16 scale is 0 are packed as zeros (both copies).
static hipError_t put_i8(Ctx* c, const int8_t* src, const void* scale, int rows, int cols,
                         const WMat& f, int r0, const WMat& b) {
  const _Float16* sc = f.colscale + r0;
  LLMT_HIP_TRY(hipMemcpyAsync((_Float16*)sc, scale, (size_t)rows * 2, hipMemcpyDefault, c->st));
  LLMT_HIP_TRY(pack_i8(src, cols, 0, rows, cols, (int8_t*)f.p, f.ld, r0, 0, c->st, sc));
  return pack_i8(src, cols, 1, cols, rows, (int8_t*)b.p, b.ld, 0, r0, c->st, sc);
}

static int put_norms(Ctx* c, Layer& w, const float* attn_norm, const float* ffn_norm,
                     const float* q_norm, const float* k_norm) {
  TRY_ARG(attn_norm && ffn_norm && q_norm && k_norm, "norm weights must be given");
  TRY_HIP(hipMemcpyAsync(w.attn_norm, attn_norm, c->H * 4, hipMemcpyDefault, c->st));
  TRY_HIP(hipMemcpyAsync(w.ffn_norm, ffn_norm, c->H * 4, hipMemcpyDefault, c->st));
  TRY_HIP(hipMemcpyAsync(w.q_norm, q_norm, kHeadDim * 4, hipMemcpyDefault, c->st));
  TRY_HIP(hipMemcpyAsync(w.k_norm, k_norm, kHeadDim * 4, hipMemcpyDefault, c->st));
  return LLMT_OK;
}

extern "C" {

int llmt_set_layer_f16(llmt_ctx* ctx, int layer, const void* wq, const void* wk, const void* wv,
                       const void* wo, const void* w_gate, const void* w_up, const void* w_down,
                       const float* attn_norm, const float* ffn_norm, const float* q_norm,
                       const float* k_norm) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && layer >= 0 && layer < c->L, "llmt_set_layer_f16: bad ctx/layer");
  TRY_ARG(c->wfmt == LLMT_WEIGHTS_F16, "context was created for int8 weights");
  TRY_ARG(wq && wk && wv && wo && w_gate && w_up && w_down, "NULL weight");
  Layer& w = c->layers[layer];
  const int H = c->H, Q = c->Q, KV = c->KV, I = c->I;
  TRY_HIP(put_f16(c, wq, Q, H, w.wqkv, 0, w.wqkvT));
  TRY_HIP(put_f16(c, wk, KV, H, w.wqkv, Q, w.wqkvT));
  TRY_HIP(put_f16(c, wv, KV, H, w.wqkv, Q + KV, w.wqkvT));
  TRY_HIP(put_f16(c, wo, H, Q, w.wo, 0, w.woT));
  TRY_HIP(put_f16(c, w_gate, I, H, w.wgu, 0, w.wguT));
  TRY_HIP(put_f16(c, w_up, I, H, w.wgu, I, w.wguT));
  TRY_HIP(put_f16(c, w_down, H, I, w.wd, 0, w.wdT));
  int rc = put_norms(c, w, attn_norm, ffn_norm, q_norm, k_norm);
  if (rc) return rc;
  TRY_HIP(hipStreamSynchronize(c->st));
  w.ready = true;
  return LLMT_OK;
}

int llmt_set_layer_i8(llmt_ctx* ctx, int layer, const int8_t* const q[7],
                      const void* const scale[7], const float* attn_norm, const float* ffn_norm,
                      const float* q_norm, const float* k_norm) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && layer >= 0 && layer < c->L, "llmt_set_layer_i8: bad ctx/layer");
  TRY_ARG(c->wfmt == LLMT_WEIGHTS_I8, "context was created for fp16 weights");
  TRY_ARG(q && scale, "NULL weight array");
  for (int i = 0; i < 7; ++i) TRY_ARG(q[i] && scale[i], "NULL weight %d", i);
  Layer& w = c->layers[layer];
  const int H = c->H, Q = c->Q, KV = c->KV, I = c->I;
  TRY_HIP(put_i8(c, q[0], scale[0], Q, H, w.wqkv, 0, w.wqkvT));
  TRY_HIP(put_i8(c, q[1], scale[1], KV, H, w.wqkv, Q, w.wqkvT));
  TRY_HIP(put_i8(c, q[2], scale[2], KV, H, w.wqkv, Q + KV, w.wqkvT));
  TRY_HIP(put_i8(c, q[3], scale[3], H, Q, w.wo, 0, w.woT));
  TRY_HIP(put_i8(c, q[4], scale[4], I, H, w.wgu, 0, w.wguT));
  TRY_HIP(put_i8(c, q[5], scale[5], I, H, w.wgu, I, w.wguT));
  TRY_HIP(put_i8(c, q[6], scale[6], H, I, w.wd, 0, w.wdT));
  int rc = put_norms(c, w, attn_norm, ffn_norm, q_norm, k_norm);
  if (rc) return rc;
  TRY_HIP(hipStreamSynchronize(c->st));
  w.ready = true;
  return LLMT_OK;
}

int llmt_set_embed_f16(llmt_ctx* ctx, const void* embed_lm_head, const float* final_norm) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && embed_lm_head && final_norm, "llmt_set_embed_f16: NULL argument");
  const _Float16* e = (const _Float16*)embed_lm_head;
  TRY_HIP(pack_f16(e, c->H, 0, c->V, c->H, c->E, c->H, 0, 0, c->st));
  TRY_HIP(pack_f16(e, c->H, 1, c->H, c->V, c->ET, c->V, 0, 0, c->st));
  TRY_HIP(hipMemcpyAsync(c->final_norm, final_norm, c->H * 4, hipMemcpyDefault, c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  // The tied embedding is the lm_head again (an earlier untied head keeps
  // its buffers for a later llmt_set_lm_head_f16); a captured step that
  // read the untied head is rebuilt.
  if (c->Eh != c->E && c->graph_exec) {
    (void)hipGraphExecDestroy(c->graph_exec);
    c->graph_exec = nullptr;
  }
  c->Eh = c->E;
  c->EhT = c->ET;
  c->embed_ready = true;
  return LLMT_OK;
}

int llmt_set_lm_head_f16(llmt_ctx* ctx, const void* lm_head) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && lm_head, "llmt_set_lm_head_f16: NULL argument");
  if (!c->head_own) {
    _Float16* eh = c->alloc_n<_Float16>((size_t)c->V * c->H);
    _Float16* eht = eh ? c->alloc_n<_Float16>((size_t)c->V * c->H) : nullptr;
    if (!eh || !eht) return LLMT_ERR_HIP;
    c->head_own = eh;
    c->headT_own = eht;
  }
  c->Eh = c->head_own;
  c->EhT = c->headT_own;
  const _Float16* w = (const _Float16*)lm_head;
  TRY_HIP(pack_f16(w, c->H, 0, c->V, c->H, c->Eh, c->H, 0, 0, c->st));
  TRY_HIP(pack_f16(w, c->H, 1, c->H, c->V, c->EhT, c->V, 0, 0, c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  if (c->graph_exec) {  // a captured step would keep the old operands
    (void)hipGraphExecDestroy(c->graph_exec);
    c->graph_exec = nullptr;
  }
  return LLMT_OK;
}

// ---------------------------------------------------------------- file formats

// Raw little-endian fp32, no header (python/export_weights.py:19-26); the
// size must match exactly (the reference only checks for short reads,
// src/train.cu:42-54).
static int read_f32(const char* path, size_t n, std::vector<float>& buf) {
  FILE* f = fopen(path, "rb");
  if (!f) {
    set_error("cannot open %s", path);
    return LLMT_ERR_IO;
  }
  fseek(f, 0, SEEK_END);
  const long sz = ftell(f);
  fseek(f, 0, SEEK_SET);
  if (sz != (long)(n * sizeof(float))) {
    fclose(f);
    set_error("%s: %ld bytes, expected %zu", path, sz, n * sizeof(float));
    return LLMT_ERR_IO;
  }
  buf.resize(n);
  const size_t got = fread(buf.data(), sizeof(float), n, f);
  fclose(f);
  if (got != n) {
    set_error("short read %s", path);
    return LLMT_ERR_IO;
  }
  return LLMT_OK;
}

int llmt_load_weights_dir(llmt_ctx* ctx, const char* dir) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && dir, "llmt_load_weights_dir: NULL argument");
  const int H = c->H, Q = c->Q, KV = c->KV, I = c->I, V = c->V;
  // staging: the embedding, or one layer's seven matrices and four norms
  const size_t layer_elems = (size_t)H * (2 * Q + 2 * KV + 3 * (size_t)I);
  const size_t big = std::max((size_t)V * H, layer_elems + 2 * (size_t)H + 2 * kHeadDim);
  float* f32 = nullptr;
  _Float16* f16 = nullptr;
  int8_t* q8 = nullptr;
  float* s32 = nullptr;
  _Float16* s16 = nullptr;
  TRY_HIP(hipMalloc((void**)&f32, big * 4));
  int rc = LLMT_OK;
  std::vector<float> host;
  char path[1024];
  auto fail = [&](int r) {
    hipFree(f32);
    hipFree(f16);
    hipFree(q8);
    hipFree(s32);
    hipFree(s16);
    return r;
  };
  if (hipMalloc((void**)&f16, big * 2) != hipSuccess ||
      hipMalloc((void**)&q8, layer_elems) != hipSuccess ||
      hipMalloc((void**)&s32, (size_t)(I * 2 + Q + 2 * KV + 2 * H) * 4) != hipSuccess ||
      hipMalloc((void**)&s16, (size_t)(I * 2 + Q + 2 * KV + 2 * H) * 2) != hipSuccess) {
    set_error("llmt_load_weights_dir: out of device memory");
    return fail(LLMT_ERR_HIP);
  }
  // Upload one fp32 file into f32 at element offset off.
  auto up = [&](const char* name, size_t n, size_t off) -> int {
    snprintf(path, sizeof(path), "%s/%s", dir, name);
    int r = read_f32(path, n, host);
    if (r) return r;
    if (hipMemcpy(f32 + off, host.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess) {
      set_error("upload %s failed", path);
      return LLMT_ERR_HIP;
    }
    return LLMT_OK;
  };
  const char* names[7] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                          "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                          "mlp.down_proj"};
  const size_t rows[7] = {(size_t)Q, (size_t)KV, (size_t)KV, (size_t)H,
                          (size_t)I, (size_t)I,  (size_t)H};
  const size_t cols[7] = {(size_t)H, (size_t)H, (size_t)H, (size_t)Q,
                          (size_t)H, (size_t)H, (size_t)I};
  for (int l = 0; l < c->L && rc == LLMT_OK; ++l) {
    size_t off[7], o = 0;
    for (int m = 0; m < 7; ++m) {
      off[m] = o;
      o += rows[m] * cols[m];
      char nm[256];
      snprintf(nm, sizeof(nm), "model.layers.%d.%s.weight.bin", l, names[m]);
      if ((rc = up(nm, rows[m] * cols[m], off[m]))) return fail(rc);
    }
    const size_t nrm = o;
    char nm[256];
    const char* nn[4] = {"input_layernorm", "post_attention_layernorm", "self_attn.q_norm",
                         "self_attn.k_norm"};
    const size_t nsz[4] = {(size_t)H, (size_t)H, (size_t)kHeadDim, (size_t)kHeadDim};
    size_t noff[4], no = nrm;
    for (int k = 0; k < 4; ++k) {
      noff[k] = no;
      snprintf(nm, sizeof(nm), "model.layers.%d.%s.weight.bin", l, nn[k]);
      if ((rc = up(nm, nsz[k], no))) return fail(rc);
      no += nsz[k];
    }
    if (c->wfmt == LLMT_WEIGHTS_F16) {
      if (f32_to_f16(f32, f16, nrm, c->st) != hipSuccess) return fail(LLMT_ERR_HIP);
      rc = llmt_set_layer_f16(ctx, l, f16 + off[0], f16 + off[1], f16 + off[2], f16 + off[3],
                              f16 + off[4], f16 + off[5], f16 + off[6], f32 + noff[0],
                              f32 + noff[1], f32 + noff[2], f32 + noff[3]);
    } else {
      // src/kernels/quantize.cu:8-44 on the device, scales kept as fp16.
      const int8_t* qp[7];
      const void* sp[7];
      size_t so = 0;
      for (int m = 0; m < 7; ++m) {
        if (quantize_rows_i8(f32 + off[m], (int)rows[m], (int)cols[m], q8 + off[m], s32 + so,
                             c->st) != hipSuccess ||
            f32_scale_to_f16(s32 + so, s16 + so, (int)rows[m], c->st) != hipSuccess)
          return fail(LLMT_ERR_HIP);
        qp[m] = q8 + off[m];
        sp[m] = s16 + so;
        so += rows[m];
      }
      rc = llmt_set_layer_i8(ctx, l, qp, sp, f32 + noff[0], f32 + noff[1], f32 + noff[2],
                             f32 + noff[3]);
    }
    if (rc) return fail(rc);
  }
  std::vector<float> fn;
  snprintf(path, sizeof(path), "%s/model.norm.weight.bin", dir);
  if ((rc = read_f32(path, H, fn))) return fail(rc);
  if ((rc = up("model.embed_tokens.weight.bin", (size_t)V * H, 0))) return fail(rc);
  if (f32_to_f16(f32, f16, (size_t)V * H, c->st) != hipSuccess || hipStreamSynchronize(c->st) != hipSuccess ||
      hipMemcpy(f32, fn.data(), H * 4, hipMemcpyHostToDevice) != hipSuccess)
    return fail(LLMT_ERR_HIP);
  if ((rc = llmt_set_embed_f16(ctx, f16, f32))) return fail(rc);
  // The reference loads lm_head.weight.bin on its own (src/train.cu:87-88);
  // its scripts write it as a copy of the embedding (scripts/run.sh:19).  A
  // head file equal to the embedding keeps the tied buffers; a different one
  // becomes an untied head; no file means tied.
  snprintf(path, sizeof(path), "%s/lm_head.weight.bin", dir);
  if (FILE* hf = fopen(path, "rb")) {
    fclose(hf);
    std::vector<float> head;
    if ((rc = read_f32(path, (size_t)V * H, head))) return fail(rc);
    if (memcmp(head.data(), host.data(), head.size() * sizeof(float)) != 0) {
      if (hipMemcpy(f32, head.data(), head.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
          f32_to_f16(f32, f16, (size_t)V * H, c->st) != hipSuccess ||
          hipStreamSynchronize(c->st) != hipSuccess)
        return fail(LLMT_ERR_HIP);
      rc = llmt_set_lm_head_f16(ctx, f16);
    }
  }
  return fail(rc);
}

// src/train.cu:146-170: <dir>/lora_step{N}_layer{L}_{wq|wk|wv|wo}_{A|B}.bin,
// raw fp32, A [16, d_in], B [d_out, 16].
static const char* kProjNames[4] = {"wq", "wk", "wv", "wo"};

int llmt_lora_save(llmt_ctx* ctx, const char* dir, int step) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && dir, "llmt_lora_save: NULL argument");
  std::vector<float> host(c->lora_numel);
  TRY_HIP(hipMemcpyAsync(host.data(), c->lora_p, c->lora_numel * 4, hipMemcpyDeviceToHost, c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  char path[1024];
  for (int l = 0; l < c->L; ++l)
    for (int p = 0; p < 4; ++p)
      for (int b = 0; b < 2; ++b) {
        const int s = 2 * p + b;
        const size_t n = (size_t)(s + 1 < 8 ? c->seg_off[s + 1] : (long long)c->lora_per_layer) -
                         (size_t)c->seg_off[s];
        snprintf(path, sizeof(path), "%s/lora_step%d_layer%d_%s_%c.bin", dir, step, l,
                 kProjNames[p], b ? 'B' : 'A');
        FILE* f = fopen(path, "wb");
        if (!f) {
          set_error("cannot write %s", path);
          return LLMT_ERR_IO;
        }
        const size_t w = fwrite(host.data() + (size_t)l * c->lora_per_layer + c->seg_off[s], 4, n, f);
        fclose(f);
        if (w != n) {
          set_error("short write %s", path);
          return LLMT_ERR_IO;
        }
      }
  return LLMT_OK;
}

int llmt_lora_load(llmt_ctx* ctx, const char* dir, int step) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && dir, "llmt_lora_load: NULL argument");
  std::vector<float> host(c->lora_numel), tmp;
  char path[1024];
  for (int l = 0; l < c->L; ++l)
    for (int p = 0; p < 4; ++p)
      for (int b = 0; b < 2; ++b) {
        const int s = 2 * p + b;
        const size_t n = (size_t)(s + 1 < 8 ? c->seg_off[s + 1] : (long long)c->lora_per_layer) -
                         (size_t)c->seg_off[s];
        snprintf(path, sizeof(path), "%s/lora_step%d_layer%d_%s_%c.bin", dir, step, l,
                 kProjNames[p], b ? 'B' : 'A');
        int rc = read_f32(path, n, tmp);
        if (rc) return rc;
        memcpy(host.data() + (size_t)l * c->lora_per_layer + c->seg_off[s], tmp.data(), n * 4);
      }
  return llmt_lora_copy(ctx, LLMT_LORA_PARAM, host.data(), 1);
}

// AdamW state next to the adapter files: <dir>/lora_step{N}_adamw.bin =
// "LLMTADAM", int32 version 1, int32 step, int64 numel, fp32 m[numel],
// fp32 v[numel] (little-endian).  The reference has no resume; this is the
// state a restart at step N + 1 needs besides the adapters themselves.
static const char kAdamMagic[8] = {'L', 'L', 'M', 'T', 'A', 'D', 'A', 'M'};

int llmt_lora_save_state(llmt_ctx* ctx, const char* dir, int step) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && dir, "llmt_lora_save_state: NULL argument");
  const size_t n = c->lora_numel;
  std::vector<float> mv(2 * n);
  TRY_HIP(hipMemcpyAsync(mv.data(), c->lora_m, n * 4, hipMemcpyDeviceToHost, c->st));
  TRY_HIP(hipMemcpyAsync(mv.data() + n, c->lora_v, n * 4, hipMemcpyDeviceToHost, c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  char path[1024];
  snprintf(path, sizeof(path), "%s/lora_step%d_adamw.bin", dir, step);
  FILE* f = fopen(path, "wb");
  if (!f) {
    set_error("cannot write %s", path);
    return LLMT_ERR_IO;
  }
  const int32_t hdr[2] = {1, step};
  const int64_t numel = (int64_t)n;
  bool ok = fwrite(kAdamMagic, 1, 8, f) == 8 && fwrite(hdr, 4, 2, f) == 2 &&
            fwrite(&numel, 8, 1, f) == 1 && fwrite(mv.data(), 4, 2 * n, f) == 2 * n;
  ok = (fclose(f) == 0) && ok;
  if (!ok) {
    set_error("short write %s", path);
    return LLMT_ERR_IO;
  }
  return LLMT_OK;
}

int llmt_lora_load_state(llmt_ctx* ctx, const char* dir, int step) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && dir, "llmt_lora_load_state: NULL argument");
  const size_t n = c->lora_numel;
  char path[1024];
  snprintf(path, sizeof(path), "%s/lora_step%d_adamw.bin", dir, step);
  FILE* f = fopen(path, "rb");
  if (!f) {
    set_error("cannot open %s", path);
    return LLMT_ERR_IO;
  }
  char magic[8];
  int32_t hdr[2];
  int64_t numel = 0;
  std::vector<float> mv(2 * n);
  const bool ok = fread(magic, 1, 8, f) == 8 && fread(hdr, 4, 2, f) == 2 &&
                  fread(&numel, 8, 1, f) == 1 && memcmp(magic, kAdamMagic, 8) == 0 &&
                  hdr[0] == 1 && hdr[1] == step && numel == (int64_t)n &&
                  fread(mv.data(), 4, 2 * n, f) == 2 * n;
  fclose(f);
  if (!ok) {
    set_error("%s: not an AdamW state of step %d with %zu parameters", path, step, n);
    return LLMT_ERR_IO;
  }
  int rc = llmt_lora_copy(ctx, LLMT_LORA_M, mv.data(), 1);
  if (rc) return rc;
  return llmt_lora_copy(ctx, LLMT_LORA_V, mv.data() + n, 1);
}

}  // extern "C"
