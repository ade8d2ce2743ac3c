// ctx.h — the training-step context behind the llmt_ctx handle.
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "../../include/llmt.h"
#include "ops.h"

namespace llmt {

constexpr int kHeadDim = 128;
constexpr int kRank = 16;

// Categories of the per-kernel profile (llmt_profile_kernels).
enum {
  CAT_GEMM_FWD = 0,
  CAT_GEMM_BWD = 1,
  CAT_GEMM_HEAD = 2,
  CAT_ATTN = 3,
  CAT_ROWS = 4,
  CAT_CE = 5,
  CAT_LORA = 6,
  CAT_ADAM = 7
};

// One recorded kernel launch: its kind (kernel name, plus the shape for
// GEMMs), category, a closure that launches it again on a given stream, and
// its algorithmic work: GEMMs 2 M N K flops and the streamed weight bytes;
// attention the flops of its causal products; the other kernels the bytes
// they read and write (split-K partials included).
struct Launch {
  int cat;
  std::string kind;
  std::function<hipError_t(hipStream_t)> fn;
  double flops, bytes;
};

// One frozen weight matrix as a GEMM B operand: fragment-packed fp16 or int8
// rows of length ld (the reduction dimension), with the int8 scale either per
// row (colscale, forward layout [out, in]) or per reduction index (kscale,
// transposed layout [in, out]).
struct WMat {
  const void* p = nullptr;
  const _Float16* colscale = nullptr;
  const _Float16* kscale = nullptr;
  int rows = 0, ld = 0, i8 = 0;
};

struct Layer {
  WMat wqkv, wqkvT;  // [Q + 2 KV, H] and [H, Q + 2 KV]
  WMat wo, woT;      // [H, Q] and [Q, H]
  WMat wgu, wguT;    // [2 I, H] (gate rows, then up rows) and [H, 2 I]
  WMat wd, wdT;      // [H, I] and [I, H]
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  float* q_norm = nullptr;
  float* k_norm = nullptr;
  bool ready = false;
};

// What the backward of one layer needs from its forward (sized for maxB*S).
struct Stash {
  float* x_in;       // [T, H] residual stream at the layer input
  _Float16* xn;      // [T, H] attention-norm output (GEMM / LoRA-A input)
  _Float16* qkraw;   // [T, Q + KV] q, k before the QK-norm (fp16)
  _Float16* qkv16;   // [T, Q + 2 KV] normed + rotated q, k and v
  float* h;          // [T, 64] LoRA h = x A^T for q, k, v, o
  _Float16* o16;     // [T, Q] attention output
  float* lse;        // [B, nq, S]
  float* x_mid;      // [T, H] residual after attention
  _Float16* xn2;     // [T, H] FFN-norm output
  _Float16* gu;      // [T, 2 I] gate, up pre-activations (fp16)
};

struct GemmOut {
  float* part;
  int split;
  long long ss;
  int ldp;
  int split_col;  // GemmArgs::split_col
};

struct Ctx {
  llmt_dims dims{};
  int maxB = 1, S = 0, wfmt = 0;
  // Token rows of a batch of B sequences as the kernels see them: B * S
  // rounded up to the GEMMs' 16-row granule.  Rows B * S .. rows(B) - 1 are
  // pad rows: their forward values and gradients are exactly zero (the
  // token gather leaves them zero, they have no target, and the attention
  // never reads or writes them), so they add nothing to the loss or to the
  // adapter gradients.
  int rows(int B) const { return (B * S + 15) & ~15; }
  // The batch whose pad rows are known to be zero in the buffers the step
  // writes only at real rows (0: none).  Entry points that write those
  // buffers at other rows reset it.
  int pad_batch = 0;
  hipError_t clear_pad_rows(int B);
  hipStream_t st = nullptr;
  bool own_stream = false;
  int H = 0, Q = 0, KV = 0, NT = 0, I = 0, V = 0, L = 0, nq = 0, nkv = 0, Tmax = 0;
  float lscale = 2.0f;

  std::vector<void*> blocks;
  size_t device_bytes = 0;

  std::vector<Layer> layers;
  _Float16* E = nullptr;   // [V, H] tied embedding / lm_head (packed, K = H)
  _Float16* ET = nullptr;  // [H, V] (packed, K = V)
  // The lm_head GEMM operands: E / ET while the head is tied to the
  // embedding; their own buffers after llmt_set_lm_head_f16.
  _Float16* Eh = nullptr;
  _Float16* EhT = nullptr;
  // An untied head's packed copies, kept for reuse after the head is tied
  // again (llmt_set_embed_f16).
  _Float16* head_own = nullptr;
  _Float16* headT_own = nullptr;
  float* final_norm = nullptr;
  bool embed_ready = false;

  // adapters: fp32 arenas + fp16 operand shadows
  size_t lora_per_layer = 0, lora_numel = 0;
  long long seg_off[8] = {};
  float *lora_p = nullptr, *lora_g = nullptr, *lora_m = nullptr, *lora_v = nullptr;
  _Float16* shadow = nullptr;
  long long shadow_per_layer = 0, sh_a_qkv = 0, sh_a_o = 0, sh_bt_qkv = 0, sh_bt_o = 0;
  _Float16* shadow_rm = nullptr;  // row-major twin of `shadow` (row epilogues)
  // A_q | A_k | A_v transposed, [L][H][3 R] (the LoRA dx term's MFMA operand
  // in the attention norm's backward)
  _Float16* shadow_at = nullptr;
  AdamHp* hp_dev = nullptr;
  AdamHp* host_hp = nullptr;

  float *cosT = nullptr, *sinT = nullptr;
  std::vector<Stash> stash;
  float* x_final = nullptr;
  _Float16* xf16 = nullptr;
  float* logits = nullptr;
  _Float16* grad16 = nullptr;
  float2* ce_stats = nullptr;  // [Tmax, ce_stats_per_row(V)]: CE chunk or logits-tile pairs
  float* lse_rows = nullptr;   // [Tmax]
  int head_tiles = 0;          // > 0: the last forward's logits GEMM wrote its tile pairs
  float* loss_rows = nullptr;
  float* loss_dev = nullptr;
  float* host_loss = nullptr;
  int* tok_buf = nullptr;
  int* tgt_buf = nullptr;

  float* part = nullptr;   // split-K partials
  size_t part_elems = 0;
  _Float16* a16 = nullptr;
  float* d_res = nullptr;
  _Float16* g16 = nullptr;
  float *rinv = nullptr, *rinv2 = nullptr;
  _Float16* dgu16 = nullptr;
  float *delta = nullptr, *dsc = nullptr;
  float* dqkv32 = nullptr;
  // Per layer (kept until the adapter gradients of all layers run in one
  // launch after the backward): dy of the q/k/v projections [T, NT], dy of
  // the o projection [T, H], the LoRA dh columns [T, 64].
  // Per layer, kept for the adapter gradients: the fp16 gradient operands of
  // the Q/K/V dX GEMM ([T, NT], the q/k/v projections' upstream gradient) and
  // of the O dX GEMM ([T, H], the o projection's), with their row factors.
  _Float16 *gq16_all = nullptr, *go16_all = nullptr;
  float *rq_all = nullptr, *ro_all = nullptr, *dh_all = nullptr;
  _Float16* gq16(int l) const { return gq16_all + (size_t)l * Tmax * NT; }
  _Float16* go16(int l) const { return go16_all + (size_t)l * Tmax * H; }
  float* rq(int l) const { return rq_all + (size_t)l * Tmax; }
  float* ro(int l) const { return ro_all + (size_t)l * Tmax; }
  float* dh(int l) const { return dh_all + (size_t)l * Tmax * 64; }
  LoraGradJob* lora_jobs = nullptr;  // device [L][kLoraJobs]
  LoraGradPlan lora_plan{};
  hipError_t lora_grads(int l0, int nl, int B, int accumulate);
  _Float16* dO16 = nullptr;  // [T, Q]: row-scaled fp16 dO of the attention backward

  // graph + profiling
  bool use_graph = false;
  hipGraphExec_t graph_exec = nullptr;
  int graph_batch = 0, graph_adam = -1;
  const int* graph_tok = nullptr;  // input pointers the graph copies from (NULL: none)
  const int* graph_tgt = nullptr;
  bool inputs_move = false;  // input pointers changed between steps: copies stay outside the graph
  // Profiling: with `recording` set, every kernel launch of the step is also
  // kept as a closure (kind, category, work) so that it can be replayed on
  // its own (llmt_profile_kernels).
  bool recording = false;
  std::vector<Launch> launches;
  std::vector<std::string> prof_names;  // kind names handed out by the last profile call

  ~Ctx();
  int init();
  void* alloc(size_t bytes);
  template <class T>
  T* alloc_n(size_t n) {
    return static_cast<T*>(alloc(n * sizeof(T)));
  }
  bool weights_ready() const {
    if (!embed_ready) return false;
    for (const Layer& l : layers)
      if (!l.ready) return false;
    return true;
  }

  // Launch one kernel (f(stream)), recording it when profiling with its
  // algorithmic work: flops (attention) and the bytes its interface moves
  // (the row kernels, CE, adapter gradients, AdamW).
  template <class F>
  hipError_t run(int cat, const char* kind, F&& f, double flops = 0, double bytes = 0) {
    if (recording)
      launches.push_back({cat, kind, std::function<hipError_t(hipStream_t)>(f), flops, bytes});
    return f(st);
  }
  // C = A B^T over the segments.  direct: split 1 into `direct` (ld ldc).
  // Otherwise the fp32 split-K partials land in `part` and *out describes
  // them; the consuming row epilogue sums them in split order.  glu16: the
  // fused SwiGLU epilogue (split 1, gemm_glu_ok shapes only) writes [gate |
  // up] fp16 [M, N] to gu16 and fp16(silu(gate) * up) [M, N / 2] to glu16
  // (direct and ldc unused).
  // rowstats (direct only): also the per-(row, column tile) softmax pairs
  // (GemmArgs::rowstats); *tiles gets their row width.  last_wave_split:
  // the consumer reads the partials through load_row, so an unsplit
  // large-tile GEMM may split only its last wave (gemm_split_col).
  hipError_t gemm(int cat, const _Float16* A, int lda, const BSeg* segs, int nseg, int M, int K,
                  float* direct, int ldc, GemmOut* out, _Float16* glu16 = nullptr,
                  _Float16* gu16 = nullptr, float2* rowstats = nullptr, int* tiles = nullptr,
                  bool last_wave_split = false);
  // A GEMM's partials as a row-epilogue input with raw h columns
  // [hcol, hcol + nh) and LoRA up-projection terms.
  RowIn row_in(const GemmOut& go, int hcol = 0, int nh = 0, int nterm = 0,
               const LoraTerm* terms = nullptr) const;
  BSeg wseg(const WMat& w) const;
  BSeg hseg(const _Float16* p, int rows, int ld) const;
  float* lora_ptr(float* arena, int l, int proj, int is_b) const;
  _Float16* shadow_ptr(int l, long long off) const;
  AdamShadow shadow_desc() const;
  AttnArgs attn_args(const Stash& s) const;

  hipError_t layer_fwd(int l, int B, const float* next_w, float* x_out, _Float16* xn_out);
  // Embedding + layers + lm_head logits (into logits_out, or the context's).
  hipError_t forward(const int* tok, int B, float* logits_out);
  // Fused CE over lg (NULL: the context's logits): loss, grad16, optional fp32 dlogits.
  hipError_t ce(const float* lg, const int* tgt, int B, float* dlogits_out);
  hipError_t head_bwd(int B);
  hipError_t layer_bwd(int l, int B);
  hipError_t backward(int B, int accumulate);
  hipError_t optimizer();
  hipError_t refresh_shadows();
  // tok / tgt: device token and target ids read in place (default: tok_buf, tgt_buf)
  hipError_t device_step(int B, int with_adam, const int* tok = nullptr, const int* tgt = nullptr);
};

}  // namespace llmt
