// api_blocks.cpp — C ABI for the benchmark configurations that exercise one
// block of the step in isolation:
//   C0  one decoder layer forward / backward through a context
//       (llmt_layer_forward / llmt_layer_backward);
//   C1  lm_head logits + fused cross-entropy + lm_head dX
//       (llmt_head_ce on a context's packed tied embedding, llmt_lm_head_ce
//       standalone);
//   C3  causal GQA flash attention forward / backward and the whole
//       QK-norm + RoPE + attention backward block
//       (llmt_attention_fwd / _bwd / _block_bwd).
// Every entry point validates shapes on the host before launching.
#include <math.h>
#include <string.h>

#include <mutex>
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

static Ctx* C_(llmt_ctx* c) { return reinterpret_cast<Ctx*>(c); }

// Temporary device buffers released (stream-ordered) on scope exit.
struct Temps {
  hipStream_t st;
  std::vector<void*> ptrs;
  explicit Temps(hipStream_t s) : st(s) {}
  template <class T>
  T* get(size_t n) {
    void* p = nullptr;
    if (hipMallocAsync(&p, n * sizeof(T) + 256, st) != hipSuccess) return nullptr;
    ptrs.push_back(p);
    return static_cast<T*>(p);
  }
  ~Temps() {
    for (void* p : ptrs) (void)hipFreeAsync(p, st);
  }
};

// Device workspace of llmt_attention_block_bwd, one per (device, stream),
// kept across calls and grown on demand: a new size waits for the stream to
// finish with the old buffer, frees it and allocates the new one (hipMalloc),
// so a steady caller allocates nothing per call and leaves the GPU no idle
// gap between calls.  Calls on one stream are ordered by the stream; calls
// on different streams use different workspaces.  At most kMaxBlockWs
// workspaces live per device: a stream beyond that takes over the least
// recently used one after a device synchronisation (its stream may be gone,
// so the whole device is drained before the buffer is reused).  The RoPE
// tables of the last (S, theta) stay at its start and are rebuilt only when
// either changes.  Host threads must not issue calls on one stream at once.
constexpr int kMaxBlockWs = 4;
struct BlockWs {
  int dev = -1;
  hipStream_t st = nullptr;
  char* base = nullptr;
  size_t cap = 0, used = 0;
  unsigned long long last_use = 0;
  int rope_S = 0;
  double rope_theta = 0.0;
  // sub-buffer of n elements, 256-byte aligned (nullptr past the capacity)
  template <class T>
  T* get(size_t n) {
    const size_t off = (used + 255) & ~(size_t)255;
    if (off + n * sizeof(T) > cap) return nullptr;
    used = off + n * sizeof(T);
    return reinterpret_cast<T*>(base + off);
  }
};
static std::mutex g_ws_mu;
static std::vector<BlockWs*> g_ws;
static unsigned long long g_ws_clock = 0;

static hipError_t block_ws(hipStream_t st, size_t bytes, BlockWs** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  BlockWs* w = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    int on_dev = 0;
    BlockWs* lru = nullptr;
    for (BlockWs* x : g_ws) {
      if (x->dev != dev) continue;
      ++on_dev;
      if (x->st == st) w = x;
      if (!lru || x->last_use < lru->last_use) lru = x;
    }
    if (!w && on_dev >= kMaxBlockWs) {  // reuse the least recently used one
      if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
      w = lru;
      w->st = st;
    }
    if (!w) {
      w = new BlockWs;
      w->dev = dev;
      w->st = st;
      g_ws.push_back(w);
    }
    w->last_use = ++g_ws_clock;
  }
  if (bytes > w->cap) {
    if (w->base) {
      if ((e = hipStreamSynchronize(st)) != hipSuccess) return e;
      if ((e = hipFree(w->base)) != hipSuccess) return e;
      w->base = nullptr;
      w->cap = 0;
    }
    if ((e = hipMalloc((void**)&w->base, bytes)) != hipSuccess) return e;
    w->cap = bytes;
    w->rope_S = 0;
  }
  w->used = 0;
  *out = w;
  return hipSuccess;
}

extern "C" {

// ------------------------------------------------------------------ C0

int llmt_layer_forward(llmt_ctx* ctx, int layer, const float* x, float* y, int batch) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && x && y && layer >= 0 && layer < c->L, "llmt_layer_forward: bad arguments");
  TRY_ARG(batch >= 1 && batch <= c->maxB && (batch * c->S) % 16 == 0, "batch");
  TRY_ARG(c->layers[layer].ready, "layer %d weights not set", layer);
  const int T = batch * c->S;
  Stash& s = c->stash[layer];
  Layer& w = c->layers[layer];
  c->pad_batch = 0;  // rows a later step may pad are written here
  TRY_HIP(copy_norm(x, w.attn_norm, c->dims.eps, c->H, T, s.x_in, s.xn, c->st));
  TRY_HIP(c->layer_fwd(layer, batch, w.attn_norm, y, c->xf16));
  TRY_HIP(hipStreamSynchronize(c->st));
  return LLMT_OK;
}

int llmt_layer_backward(llmt_ctx* ctx, int layer, const float* dy, float* dx, int batch) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && dy && dx && layer >= 0 && layer < c->L, "llmt_layer_backward: bad arguments");
  TRY_ARG(batch >= 1 && batch <= c->maxB && (batch * c->S) % 16 == 0, "batch");
  const int T = batch * c->S;
  c->pad_batch = 0;
  // g16 feeds the layer's down dX, which takes int8 weights' scale from it
  TRY_HIP(grad_rows(dy, c->H, T, c->d_res, c->g16, c->rinv, c->layers[layer].wdT.kscale, c->st));
  TRY_HIP(c->layer_bwd(layer, batch));
  TRY_HIP(c->lora_grads(layer, 1, batch, 0));
  TRY_HIP(hipMemcpyAsync(dx, c->d_res, (size_t)T * c->H * 4, hipMemcpyDeviceToDevice, c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  return LLMT_OK;
}

// ------------------------------------------------------------------ C1

// lm_head GEMMs on packed operands E (K = H) and ET (K = V), fused CE between:
// the logits GEMM also writes the softmax pairs of its column tiles (stats:
// T * ce_stats_per_row(V) pairs; lse: T floats), so the CE reads the logits
// once.
static int head_ce_packed(hipStream_t st, const _Float16* hidden, const _Float16* E,
                          const _Float16* ET, const int* targets, int T, int seq_len, int H,
                          int V, float* logits, _Float16* grad16, float2* stats, float* lse,
                          float* loss_rows, float* loss_mean, float* dlogits, float* dhidden,
                          float* part, size_t part_elems) {
  GemmArgs g{};
  g.A = hidden;
  g.lda = H;
  g.nseg = 1;
  g.seg[0] = BSeg{E, nullptr, nullptr, V, H, 0};
  gemm_finalize_segments(g);
  g.M = T;
  g.K = H;
  g.split = 1;
  g.C = logits;
  g.ldc = V;
  const int nt = gemm_rowstats_tiles(g);
  TRY_ARG(nt > 0 && nt <= ce_stats_per_row(V), "head_ce: logits tile statistics");
  g.rowstats = stats;
  TRY_HIP(gemm_nt(g, st));
  TRY_HIP(cross_entropy_from_stats(logits, stats, nt, targets, T, V, seq_len, lse, dlogits, grad16,
                                   loss_rows, loss_mean, st));
  GemmArgs d{};
  d.A = grad16;
  d.lda = V;
  d.nseg = 1;
  d.seg[0] = BSeg{ET, nullptr, nullptr, H, V, 0};
  gemm_finalize_segments(d);
  d.M = T;
  d.K = V;
  d.split = gemm_pick_split(T, H, V, 64);
  TRY_ARG((size_t)d.split * T * H <= part_elems, "head_ce: partial workspace");
  d.C = part;
  d.ldc = H;
  d.split_stride = (long long)T * H;
  TRY_HIP(gemm_nt(d, st));
  ReduceArgs ra{};
  ra.part = part;
  ra.split = d.split;
  ra.ss = d.split_stride;
  ra.ldp = H;
  ra.out = dhidden;
  ra.ldo = H;
  ra.M = T;
  ra.N = H;
  const int n_valid = T / seq_len * (seq_len - 1);
  ra.out_scale = 1.0f / (kGradLogitScale * (float)n_valid);
  TRY_HIP(reduce_lora(ra, st));
  return LLMT_OK;
}

int llmt_head_ce(llmt_ctx* ctx, const void* hidden16, const int* targets, int batch,
                 float* loss_host, float* dlogits, float* dhidden) {
  set_error("");
  Ctx* c = C_(ctx);
  TRY_ARG(c && hidden16 && targets && dhidden, "llmt_head_ce: NULL argument");
  TRY_ARG(c->embed_ready, "embedding not set");
  TRY_ARG(batch >= 1 && batch <= c->maxB && (batch * c->S) % 16 == 0, "batch");
  const int T = batch * c->S;
  c->pad_batch = 0;
  int rc = head_ce_packed(c->st, (const _Float16*)hidden16, c->Eh, c->EhT, targets, T, c->S, c->H,
                          c->V, c->logits, c->grad16, c->ce_stats, c->lse_rows, c->loss_rows,
                          c->loss_dev, dlogits, dhidden, c->part, c->part_elems);
  if (rc) return rc;
  TRY_HIP(hipMemcpyAsync(c->host_loss, c->loss_dev, 4, hipMemcpyDeviceToHost, c->st));
  TRY_HIP(hipStreamSynchronize(c->st));
  if (loss_host) *loss_host = *c->host_loss;
  return LLMT_OK;
}

int llmt_lm_head_ce(const void* hidden, const void* W, const int* targets, int T, int seq_len,
                    int H, int V, float* loss_mean, float* dlogits, float* dhidden, void* stream) {
  set_error("");
  TRY_ARG(hidden && W && targets && loss_mean && dhidden, "llmt_lm_head_ce: NULL argument");
  TRY_ARG(T > 0 && T % 16 == 0 && seq_len >= 2 && T % seq_len == 0 && H % 32 == 0 &&
              V % 32 == 0 && H % 8 == 0,
          "llmt_lm_head_ce: T %% 16, T %% seq_len, H %% 32, V %% 32 must be 0");
  hipStream_t st = (hipStream_t)stream;
  Temps tmp(st);
  _Float16* E = tmp.get<_Float16>((size_t)V * H);
  _Float16* ET = tmp.get<_Float16>((size_t)V * H);
  float* logits = tmp.get<float>((size_t)T * V);
  _Float16* g16 = tmp.get<_Float16>((size_t)T * V);
  float2* stats = tmp.get<float2>((size_t)T * ce_stats_per_row(V));
  float* rows = tmp.get<float>(T);
  float* lse = tmp.get<float>(T);
  const size_t pe = (size_t)gemm_pick_split(T, H, V, 64) * T * H;
  float* part = tmp.get<float>(pe);
  TRY_ARG(E && ET && logits && g16 && stats && rows && lse && part,
          "llmt_lm_head_ce: out of memory");
  TRY_HIP(pack_f16((const _Float16*)W, H, 0, V, H, E, H, 0, 0, st));
  TRY_HIP(pack_f16((const _Float16*)W, H, 1, H, V, ET, V, 0, 0, st));
  return head_ce_packed(st, (const _Float16*)hidden, E, ET, targets, T, seq_len, H, V, logits, g16,
                        stats, lse, rows, loss_mean, dlogits, dhidden, part, pe);
}

// ------------------------------------------------------------------ C3

static int attn_shape_ok(int B, int S, int nq, int nkv) {
  return B > 0 && S > 0 && nq > 0 && nkv > 0 && nq % nkv == 0;
}

int llmt_attention_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int B,
                       int S, int nq, int nkv, void* stream) {
  set_error("");
  TRY_ARG(q && k && v && o && lse && attn_shape_ok(B, S, nq, nkv),
          "llmt_attention_fwd: bad arguments");
  AttnArgs a{};
  a.q = (const _Float16*)q;
  a.ldq = (long long)nq * kHeadDim;
  a.k = (const _Float16*)k;
  a.ldk = (long long)nkv * kHeadDim;
  a.v = (const _Float16*)v;
  a.ldv = (long long)nkv * kHeadDim;
  a.nq = nq;
  a.nkv = nkv;
  a.S = S;
  a.sm_scale = 1.0f / sqrtf((float)kHeadDim);
  a.o = (_Float16*)o;
  a.ldo = (long long)nq * kHeadDim;
  a.lse = lse;
  TRY_HIP(attn_fwd(a, B, (hipStream_t)stream));
  return LLMT_OK;
}

int llmt_attention_bwd(const void* q, const void* k, const void* v, const void* o,
                       const float* lse, const float* dout, float* dq, float* dk, float* dv,
                       int B, int S, int nq, int nkv, void* stream) {
  set_error("");
  TRY_ARG(q && k && v && o && lse && dout && dq && dk && dv && attn_shape_ok(B, S, nq, nkv),
          "llmt_attention_bwd: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  const int T = B * S;
  Temps tmp(st);
  float* delta = tmp.get<float>((size_t)B * nq * S);
  float* dsc = tmp.get<float>((size_t)T * nq);
  _Float16* dO16 = tmp.get<_Float16>((size_t)T * nq * kHeadDim);
  TRY_ARG(delta && dsc && dO16, "llmt_attention_bwd: out of memory");
  const long long ldq = (long long)nq * kHeadDim, ldkv = (long long)nkv * kHeadDim;
  TRY_HIP(attn_delta(dout, 0, ldq, (const _Float16*)o, ldq, nq, S, T, delta, dO16, ldq, dsc, st));
  AttnArgs a{};
  a.q = (const _Float16*)q;
  a.ldq = ldq;
  a.k = (const _Float16*)k;
  a.ldk = ldkv;
  a.v = (const _Float16*)v;
  a.ldv = ldkv;
  a.nq = nq;
  a.nkv = nkv;
  a.S = S;
  a.sm_scale = 1.0f / sqrtf((float)kHeadDim);
  a.lse = const_cast<float*>(lse);  // read-only in the backward
  a.dO16 = dO16;
  a.ld16 = ldq;
  a.dsc = dsc;
  a.delta = delta;
  a.dq = dq;
  a.ldgq = ldq;
  a.dk = dk;
  a.dv = dv;
  a.ldgkv = ldkv;
  TRY_HIP(attn_bwd(a, B, st));
  return LLMT_OK;
}

// Config C3 on the caller's layouts, no copies, three launches after the
// RoPE tables: per-head QK-norm + RoPE of k_raw; the flash forward, which
// also normalises and rotates its q rows (keeping them for the backward) and
// prepares the dO operand from the fp16 dout (v read in place); the flash
// backward, whose dQ / dK epilogues run the QK-norm + RoPE backward into
// dq_raw / dk_raw (dv written in place).
int llmt_attention_block_bwd(const void* q_raw, const void* k_raw, const void* v,
                             const float* q_norm, const float* k_norm, const void* dout,
                             float* dq_raw, float* dk_raw, float* dv, int B, int S, int nq,
                             int nkv, float theta, float eps, void* stream) {
  set_error("");
  TRY_ARG(q_raw && k_raw && v && q_norm && k_norm && dout && dq_raw && dk_raw && dv &&
              attn_shape_ok(B, S, nq, nkv),
          "llmt_attention_block_bwd: bad arguments");
  TRY_ARG(((uintptr_t)q_raw | (uintptr_t)dout | (uintptr_t)q_norm | (uintptr_t)k_norm |
           (uintptr_t)dq_raw | (uintptr_t)dk_raw | (uintptr_t)dv) % 16 == 0 &&
              (uintptr_t)k_raw % 8 == 0 && (uintptr_t)v % 16 == 0,
          "llmt_attention_block_bwd: q_raw, v, dout, the norm weights and the fp32 outputs need "
          "16-byte alignment, k_raw 8");
  hipStream_t st = (hipStream_t)stream;
  const int T = B * S, Q = nq * kHeadDim, KV = nkv * kHeadDim;
  const size_t f16 = sizeof(_Float16), f32 = sizeof(float);
  const size_t need = 9 * 256 + (size_t)S * 64 * f32 * 2 + (size_t)T * Q * f16 * 3 +
                      (size_t)T * KV * f16 + (size_t)B * nq * S * f32 * 2 + (size_t)T * nq * f32;
  BlockWs* ws = nullptr;
  TRY_HIP(block_ws(st, need, &ws));
  float* cosT = ws->get<float>((size_t)S * 64);
  float* sinT = ws->get<float>((size_t)S * 64);
  _Float16* q16 = ws->get<_Float16>((size_t)T * Q);
  _Float16* k16 = ws->get<_Float16>((size_t)T * KV);
  _Float16* o16 = ws->get<_Float16>((size_t)T * Q);
  float* lse = ws->get<float>((size_t)B * nq * S);
  float* delta = ws->get<float>((size_t)B * nq * S);
  float* dsc = ws->get<float>((size_t)T * nq);
  _Float16* dO16 = ws->get<_Float16>((size_t)T * Q);
  TRY_ARG(q16 && k16 && o16 && lse && delta && dsc && dO16 && cosT && sinT,
          "llmt_attention_block_bwd: workspace layout");
  if (ws->rope_S != S || ws->rope_theta != (double)theta) {
    TRY_HIP(rope_tables(S, (double)theta, cosT, sinT, st));
    ws->rope_S = S;
    ws->rope_theta = (double)theta;
  }
  // k's QK-norm + RoPE on its own (every dK/dV and forward workgroup reads
  // all of it); q's runs inside the forward, which writes q16 for the
  // backward, and dO's operand preparation in the forward's epilogue
  const HeadRows fk[1] = {{(const _Float16*)k_raw, k_norm, k16, nkv}};
  TRY_HIP(head_norm_rope(fk, 1, cosT, sinT, S, T, eps, st));
  AttnArgs a{};
  a.q = q16;
  a.ldq = Q;
  a.k = k16;
  a.ldk = KV;
  a.v = (const _Float16*)v;
  a.ldv = KV;
  a.nq = nq;
  a.nkv = nkv;
  a.S = S;
  a.sm_scale = 1.0f / sqrtf((float)kHeadDim);
  a.o = o16;
  a.ldo = Q;
  a.lse = lse;
  a.qraw = (const _Float16*)q_raw;
  a.ldqr = Q;
  a.kraw = (const _Float16*)k_raw;
  a.ldkr = KV;
  a.qn = q_norm;
  a.cosT = cosT;
  a.sinT = sinT;
  a.eps = eps;
  a.q16w = q16;
  a.dout = (const _Float16*)dout;
  a.lddo = Q;
  a.dO16w = dO16;
  a.deltaw = delta;
  a.dscw = dsc;
  a.ld16 = Q;
  TRY_HIP(attn_fwd(a, B, st));
  a.dout = nullptr;
  a.dO16 = dO16;
  a.dsc = dsc;
  a.delta = delta;
  // dQ / dK go through the QK-norm + RoPE backward in the kernels' epilogues
  a.kn = k_norm;
  a.dq = dq_raw;
  a.ldgq = Q;
  a.dk = dk_raw;
  a.dv = dv;
  a.ldgkv = KV;
  TRY_HIP(attn_bwd(a, B, st));
  return LLMT_OK;
}

}  // extern "C"
