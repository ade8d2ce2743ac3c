/* llmt.h — C ABI of the MI355X-native LoRA training step (libllmt.so).
 *
 * Two layers share one set of gfx950 kernels:
 *
 *  1. The compat layer: the reference's own step API with the same names,
 *     argument order and struct layouts, now `extern "C"`.  A train.cu-style
 *     driver links against it unchanged.  As in the reference, the compat
 *     functions report failures on stderr and exit(EXIT_FAILURE)
 *     (reference include/utils.h:10-28), run on the legacy default stream and
 *     synchronise only where the reference does (the loss read-back).
 *  2. The native layer (llmt_*): an explicit context, an explicit stream,
 *     batch > 1, int error codes (0 = success, <0 = error, message via
 *     llmt_last_error()) and one host synchronisation per step.
 *
 * All pointers are device pointers unless the parameter name ends in _host.
 * Matrices are row-major; frozen weights are [out, in] like the reference;
 * token ids are int32.  References are file:line in visheshnarayan/llm.cu.
 */
#ifndef LLMT_H
#define LLMT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- model constants (reference include/config.h:5-21, include/lora.h:6-8) ---- */
#define LLMT_HIDDEN_SIZE       2048
#define LLMT_NUM_LAYERS        28
#define LLMT_NUM_HEADS         16
#define LLMT_NUM_KV_HEADS      8
#define LLMT_HEAD_DIM          128
#define LLMT_INTERMEDIATE_SIZE 6144
#define LLMT_VOCAB_SIZE        151936
#define LLMT_LORA_RANK         16
#define LLMT_LORA_ALPHA        32
#define LLMT_LORA_SCALE        2.0f
#define LLMT_RMS_NORM_EPS      1e-6f
#define LLMT_ROPE_THETA        1000000.0f

/* ======================================================================
 * 1. Compat layer — reference structs (include/lora.h:13-62, src/train.cu:10-24)
 * ====================================================================== */

/* include/lora.h:13-20 — one adapter: A [r, d_in], B [d_out, r], AdamW moments. */
typedef struct {
    float* A;
    float* B;
    float* mA; float* vA;
    float* mB; float* vB;
    int d_in, d_out;
} LoraAdapter;

/* include/lora.h:23-28 */
typedef struct {
    LoraAdapter wq[LLMT_NUM_LAYERS];
    LoraAdapter wk[LLMT_NUM_LAYERS];
    LoraAdapter wv[LLMT_NUM_LAYERS];
    LoraAdapter wo[LLMT_NUM_LAYERS];
} LoraWeights;

/* include/lora.h:31-34 */
typedef struct {
    float* dA;
    float* dB;
} LoraGrad;

/* include/lora.h:36-41 */
typedef struct {
    LoraGrad wq[LLMT_NUM_LAYERS];
    LoraGrad wk[LLMT_NUM_LAYERS];
    LoraGrad wv[LLMT_NUM_LAYERS];
    LoraGrad wo[LLMT_NUM_LAYERS];
} LoraGrads;

/* include/lora.h:44-62.  The layout is the reference's; the stashes
 * themselves are library-private (they live in the context, with the
 * softmax log-sum-exp in place of P), so lora_acts_alloc sets every slot to
 * NULL and the compat forward/backward never read or write them (the
 * reference's train.cu never reads acts either). */
typedef struct {
    float* layer_in[LLMT_NUM_LAYERS];
    float* attn_norm_out[LLMT_NUM_LAYERS];
    float* q_raw[LLMT_NUM_LAYERS];
    float* k_raw[LLMT_NUM_LAYERS];
    float* q_rope[LLMT_NUM_LAYERS];
    float* k_rope[LLMT_NUM_LAYERS];
    float* v_raw[LLMT_NUM_LAYERS];
    float* attn_w[LLMT_NUM_LAYERS];
    float* pre_o[LLMT_NUM_LAYERS];
    float* post_attn[LLMT_NUM_LAYERS];
    float* ffn_norm_out[LLMT_NUM_LAYERS];
    float* gate_raw[LLMT_NUM_LAYERS];
    float* up_raw[LLMT_NUM_LAYERS];
    float* hq[LLMT_NUM_LAYERS];
    float* hk[LLMT_NUM_LAYERS];
    float* hv[LLMT_NUM_LAYERS];
    float* ho[LLMT_NUM_LAYERS];
} LoraActs;

/* src/train.cu:10-17 (= src/kernels/lora_forward.cu:18-32).  The 21 pad slots
 * mirror src/main.cu:40-55: _pad[0..6] = fp16 (uint16 bits) copies of
 * wq, wk, wv, wo, w_gate, w_up, w_down; _pad[7..20] = (int8_t* q, float*
 * scale) pairs in the same order (q [out, in], scale fp32 [out], the
 * src/kernels/quantize.cu recipe).  Weight source, decided by layer 0: its
 * fp16 pads when set (fp16 weights; layers whose pads are NULL convert their
 * fp32 fields once); else its int8 pads when set (int8 weights, the scales
 * rounded to fp16 as the int8 GEMMs take them; layers whose int8 pads are
 * NULL quantise their fp32 fields); else the fp32 fields converted to fp16.
 * The fp32 weight fields may be NULL when the pads are supplied. */
typedef struct {
    float* attn_norm;
    float* ffn_norm;
    float* wq; float* wk; float* wv; float* wo;
    float* q_norm; float* k_norm;
    float* w_gate; float* w_up; float* w_down;
    void* _pad[21];
} LW;

/* src/train.cu:18-24.  _pad[0] = fp16 lm_head, _pad[1..2] = int8_t* lm_head
 * and its float* row scales (src/main.cu:63-64).  The head is read from the
 * fp16 pad, else the fp32 lm_head, else the int8 pair (as fp16 q * scale).
 * embed_table may be NULL when the lm_head is tied (the reference scripts
 * copy embed -> lm_head, scripts/run.sh:19); the gather then reads the
 * lm_head rows. */
typedef struct {
    float* embed_table;
    LW layers[LLMT_NUM_LAYERS];
    float* final_norm;
    float* lm_head;
    void* _pad[3];
} MW;

/* include/lora.h:66-90 */
void lora_weights_init(LoraWeights* lora);
void lora_weights_free(LoraWeights* lora);
void lora_grads_alloc(LoraGrads* grads, const LoraWeights* lora);
void lora_grads_free(LoraGrads* grads);
void lora_grads_zero(LoraGrads* grads);
void lora_acts_alloc(LoraActs* acts, int seq_len);
void lora_acts_free(LoraActs* acts, int seq_len);
/* src/kernels/lora.cu:181-202: y[seq, d_out] += 2 * (x A^T) B^T; h_buf = x A^T if non-NULL. */
void lora_forward_add(const float* x, const LoraAdapter* a, float* y, float* h_buf, int seq);
/* src/kernels/lora.cu:235-246 */
void adamw_step_lora(LoraWeights* lora, const LoraGrads* grads, float lr, float beta1,
                     float beta2, float eps, float wd, int step);
/* src/kernels/lora.cu:10-28 */
void scale_add_inplace(float* dst, const float* src, float scale, int n);
void gpu_zero(float* buf, int n);

/* src/kernels/lora_forward.cu:169-186.  The workspaces and acts are accepted
 * for ABI compatibility and not touched (the stashes live in the library's
 * context); logits receives the fp32 logits [seq, V].  Frozen weights are
 * uploaded (by the MW pad map above) on the first call for a given MW,
 * adapters on every call.  Any seq_len >= 2. */
void transformer_forward_lora(const int* token_ids, const MW* model, const LoraWeights* lora,
                              float* hidden, float* residual, float* norm_out,
                              float* q, float* k, float* v, float* k_exp, float* v_exp,
                              float* attn_out, float* gate_buf, float* up_buf,
                              float* logits, LoraActs* acts, int seq_len);
/* src/kernels/loss.cu:74-91: mean CE over the seq_len-1 rows with a target;
 * writes fp32 dlogits (row seq_len-1 zeroed); returns the loss (syncs). */
float cross_entropy_forward(const float* logits, const int* targets, float* dlogits, int seq_len);
/* src/kernels/lora_backward.cu:212-233.  Gradients are accumulated into
 * grads (callers zero them first, as src/train.cu:261 does). */
void transformer_backward_lora(const float* d_logits, const MW* model, const LoraWeights* lora,
                               const LoraActs* acts, LoraGrads* grads,
                               float* d_hidden, float* d_hidden2, float* d_norm,
                               float* d_q, float* d_k, float* d_v,
                               float* d_q_exp, float* d_k_exp, float* d_v_exp,
                               float* d_pre_o, float* d_gate, float* d_up,
                               float* dh_tmp, float* dx_lora, int seq_len);

/* ======================================================================
 * 2. Native layer
 * ====================================================================== */

typedef struct llmt_ctx llmt_ctx;

typedef struct {
    int hidden, n_layers, n_heads, n_kv_heads, head_dim, intermediate, vocab, rank;
    float alpha, eps, theta;
} llmt_dims;

typedef struct {
    float lr, beta1, beta2, eps, wd;
} llmt_hparams;

enum {
    LLMT_OK = 0,
    LLMT_ERR_ARG = -1,       /* bad argument / unsupported shape */
    LLMT_ERR_HIP = -2,       /* HIP runtime error */
    LLMT_ERR_IO = -3,        /* missing or short file */
    LLMT_ERR_STATE = -4      /* call order (e.g. backward before forward) */
};
enum { LLMT_WEIGHTS_F16 = 0, LLMT_WEIGHTS_I8 = 1 };
enum { LLMT_PROJ_Q = 0, LLMT_PROJ_K = 1, LLMT_PROJ_V = 2, LLMT_PROJ_O = 3 };
enum { LLMT_LORA_PARAM = 0, LLMT_LORA_GRAD = 1, LLMT_LORA_M = 2, LLMT_LORA_V = 3 };

const char* llmt_last_error(void);
void llmt_dims_qwen3_1_7b(llmt_dims* out);

/* Context for up to max_batch sequences of seq_len tokens (stashes and
 * workspaces are sized at creation).  stream may be NULL: the context then
 * creates its own stream, blocking with respect to the legacy default stream
 * (a captured HIP graph needs a non-default stream). */
int llmt_ctx_create(const llmt_dims* dims, int max_batch, int seq_len, int weight_format,
                    void* stream, llmt_ctx** out);
int llmt_ctx_destroy(llmt_ctx* ctx);
/* Bytes of device memory the context owns. */
size_t llmt_ctx_device_bytes(const llmt_ctx* ctx);

/* Frozen weights.  fp16 arguments are [out, in] fp16 device buffers; the
 * library copies them into its own packed, pre-transposed arena, so callers
 * may free theirs afterwards.  Norm weights are fp32 [n]. */
int llmt_set_layer_f16(llmt_ctx* ctx, int layer, const void* wq, const void* wk, const void* wv,
                       const void* wo, const void* w_gate, const void* w_up, const void* w_down,
                       const float* attn_norm, const float* ffn_norm, const float* q_norm,
                       const float* k_norm);
/* int8 [out, in] weights with fp16 per-output-row scales (the quantize.cu
 * recipe, produced e.g. by llmt_quantize_rows_i8).  A row whose fp16 scale is
 * 0 is taken as all zeros. */
int llmt_set_layer_i8(llmt_ctx* ctx, int layer, const int8_t* const q[7], const void* const scale[7],
                      const float* attn_norm, const float* ffn_norm, const float* q_norm,
                      const float* k_norm);
/* Tied embedding / lm_head [V, H] fp16 and the final norm [H] fp32.  Ties
 * the head to this embedding (again, after an llmt_set_lm_head_f16). */
int llmt_set_embed_f16(llmt_ctx* ctx, const void* embed_lm_head, const float* final_norm);
/* An untied lm_head [V, H] fp16 (the reference loads lm_head.weight.bin on its
 * own, src/train.cu:87-88): the logits and the head's dX use it, the token
 * gather keeps the embedding.  Allocates the head's packed copies on the
 * first call. */
int llmt_set_lm_head_f16(llmt_ctx* ctx, const void* lm_head);
/* Reference on-disk layout (src/train.cu:56-89, python/export_weights.py:19-26):
 * <dir>/<hf_param_name>.bin raw fp32 little-endian [out, in], no header.
 * lm_head.weight.bin is optional: absent or equal to the embedding means a
 * tied head, otherwise it is loaded as an untied head. */
int llmt_load_weights_dir(llmt_ctx* ctx, const char* dir);

/* Adapters live in one fp32 arena per kind (param, grad, m, v), ordered layer
 * by layer, q, k, v, o, A then B (A [r, d_in], B [d_out, r]). */
size_t llmt_lora_numel(const llmt_ctx* ctx);
size_t llmt_lora_offset(const llmt_ctx* ctx, int layer, int proj, int is_b);
/* Copy a whole arena to/from a caller device buffer (to_ctx: 1 = into ctx). */
int llmt_lora_copy(llmt_ctx* ctx, int kind, float* buf, int to_ctx);
/* Reference adapter files weights/lora_step{N}_layer{L}_{wq|wk|wv|wo}_{A|B}.bin
 * (src/train.cu:146-170) — raw fp32, A [16, d_in], B [d_out, 16]. */
int llmt_lora_save(llmt_ctx* ctx, const char* dir, int step);
int llmt_lora_load(llmt_ctx* ctx, const char* dir, int step);
/* AdamW moments for resuming a run (no counterpart in the reference, whose
 * driver cannot resume): <dir>/lora_step{N}_adamw.bin holds "LLMTADAM",
 * int32 version 1, int32 step, int64 numel, fp32 m, fp32 v. */
int llmt_lora_save_state(llmt_ctx* ctx, const char* dir, int step);
int llmt_lora_load_state(llmt_ctx* ctx, const char* dir, int step);
/* Seeded init on the device (the reference draws A with cuRAND, B = 0:
 * src/kernels/lora.cu:40-62; configs use A std a_std, B std b_std). */
int llmt_lora_init(llmt_ctx* ctx, uint64_t seed, float a_std, float b_std);

/* One training step (src/train.cu:251-288): forward, fused CE, backward,
 * AdamW with bias-correction step `step` (1-based).  tokens/targets: int32
 * device [batch, seq_len], any seq_len >= 2 and batch <= max_batch (the
 * kernels run on batch*seq_len rows rounded up to a multiple of 16; the pad
 * rows are zero and add nothing).  The loss is the mean over
 * batch*(seq_len-1) rows (src/kernels/loss.cu:86-90).  *loss_host is written
 * after the one host sync.  llmt_forward_backward runs everything but AdamW
 * (grads are left in the GRAD arena, overwritten, not accumulated). */
int llmt_step(llmt_ctx* ctx, const int* tokens, const int* targets, int batch,
              const llmt_hparams* hp, int step, float* loss_host);
int llmt_forward_backward(llmt_ctx* ctx, const int* tokens, const int* targets, int batch,
                          float* loss_host);
/* Capture llmt_step's device work into a HIP graph and replay it
 * (enable = 1); the graph is rebuilt when batch changes. */
int llmt_set_graph(llmt_ctx* ctx, int enable);
/* fp32 logits of the last forward: rows 0 .. batch*seq_len-1 in token order
 * (then the zero pad rows up to a multiple of 16), V wide. */
const float* llmt_logits(const llmt_ctx* ctx);
/* fp32 residual stream [batch*seq_len, H] at the input of `layer` (0..L-1)
 * from the last forward, the reference's LoraActs.layer_in[layer]
 * (include/lora.h:45, src/kernels/lora_forward.cu:205): layer 0's rows are
 * the gathered embedding rows E[token] (src/kernels/embed.cu:6-20).  NULL for
 * a layer outside the model. */
const float* llmt_layer_in(const llmt_ctx* ctx, int layer);

/* Single-layer forward/backward through layer `layer` (config C0): x, y, dy,
 * dx are fp32 [batch*seq_len, H], batch*seq_len a multiple of 16. The
 * backward writes the layer's adapter gradients into the GRAD arena and dx. */
int llmt_layer_forward(llmt_ctx* ctx, int layer, const float* x, float* y, int batch);
int llmt_layer_backward(llmt_ctx* ctx, int layer, const float* dy, float* dx, int batch);
/* AdamW over the whole arena (one multi-tensor launch). */
int llmt_adamw(llmt_ctx* ctx, const llmt_hparams* hp, int step);
/* Per-kernel timing of one llmt_step (no counterpart in the reference).  The
 * step (forward, CE, backward, AdamW: the adapters advance by this one step)
 * runs once eagerly with every kernel launch recorded; then the launches of
 * each kind (one kernel at one shape; a backward dX GEMM's name ends in
 * " dX") are replayed back to back, `reps`
 * times, as a HIP graph of their own and timed with HIP events on the
 * context's stream, so no events sit between kernels and no dependent-launch
 * gaps are counted (the kinds' totals sum to less than a step).  The
 * parameter and moment arenas are saved before the replays and restored
 * after; the GRAD arena and the stashes are left unspecified.  Per kind
 * k < *nkinds (<= max_kinds), in first-launch order: names[k] (owned by the
 * context, valid until its next llmt_profile_kernels or destroy), cats[k]
 * (0 forward GEMMs, 1 backward GEMMs, 2 lm_head GEMMs, 3 attention, 4 row
 * epilogues, 5 cross-entropy, 6 LoRA gradients, 7 AdamW), launches[k] per
 * step, us[k] = average launch duration in microseconds, flops[k] and
 * bytes[k] = algorithmic work of one launch: GEMMs 2 M N K and the streamed
 * weight bytes; attention the flops of its causal S x S x 128 products (two
 * forward, five backward) and no bytes; every other kernel no flops and the
 * bytes its interface reads and writes (split-K partials included). */
int llmt_profile_kernels(llmt_ctx* ctx, const int* tokens, const int* targets, int batch,
                         const llmt_hparams* hp, int step, int reps, int max_kinds, int* nkinds,
                         const char** names, int* cats, int* launches, float* us, double* flops,
                         double* bytes);

/* ---- standalone operators (stream may be NULL) ---- */

/* C = A B^T: A [M, K] fp16 (lda), B [N, K] fp16 (ldb), C [M, N] fp32 (ldc).
 * M % 16 == 0, K % 64 == 0. */
int llmt_gemm_f16(const void* A, int lda, const void* B, int ldb, float* C, int ldc,
                  int M, int N, int K, void* stream);
/* C = (A q^T) * scale[n]: q [N, K] int8, scale [N] fp16. */
int llmt_gemm_i8(const void* A, int lda, const int8_t* q, int ldq, const void* scale,
                 float* C, int ldc, int M, int N, int K, void* stream);
/* src/kernels/quantize.cu:8-44 bit-exact: q [rows, cols] int8, scale fp32 [rows]. */
int llmt_quantize_rows_i8(const float* w, int rows, int cols, int8_t* q, float* scale, void* stream);
/* Fused softmax + NLL + dlogits over rows of width V (src/kernels/loss.cu:13-71).
 * Row i is valid when (i % seq_len) < seq_len-1.  loss_rows [rows] (0 for
 * invalid rows), *loss_mean (device) = mean over valid rows, dlogits fp32
 * (may be NULL). */
int llmt_cross_entropy(const float* logits, const int* targets, int rows, int V, int seq_len,
                       float* dlogits, float* loss_rows, float* loss_mean, void* stream);
/* llmt_cross_entropy without any allocation: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  Same arguments, results and errors, plus
 * LLMT_ERR_ARG when rows * ceil(V / 8192) exceeds 262144 (the library's
 * built-in 2 MiB statistics scratch: 13,797 rows at V = 151936).  Calls that
 * overlap on one GPU share that scratch and race. */
int llmt_cross_entropy_noalloc(const float* logits, const int* targets, int rows, int V,
                               int seq_len, float* dlogits, float* loss_rows, float* loss_mean,
                               void* stream);
/* Config C1: logits = hidden W^T, fused CE, dlogits, dhidden = dlogits W.
 * hidden [T, H] fp16, W [V, H] fp16 row-major (packed into temporaries on
 * every call); outputs fp32; *loss_mean is a device float; dlogits may be
 * NULL.  T % 16 == 0, T % seq_len == 0. */
int llmt_lm_head_ce(const void* hidden, const void* W, const int* targets, int T, int seq_len,
                    int H, int V, float* loss_mean, float* dlogits, float* dhidden, void* stream);
/* Config C1 on a context's lm_head (already packed by llmt_set_embed_f16 /
 * llmt_set_lm_head_f16): hidden fp16 [batch*seq_len, H] (batch*seq_len a
 * multiple of 16), dlogits (may be NULL) and dhidden fp32 device buffers;
 * *loss_host after one host sync. */
int llmt_head_ce(llmt_ctx* ctx, const void* hidden16, const int* targets, int batch,
                 float* loss_host, float* dlogits, float* dhidden);
/* Causal GQA flash attention (config C3).  q [B,S,nq,128], k/v [B,S,nkv,128]
 * fp16, o fp16 [B,S,nq,128], lse fp32 [B,nq,S]. */
int llmt_attention_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                       int B, int S, int nq, int nkv, void* stream);
/* dq/dk/dv fp32 w.r.t. the attention inputs (post-norm, post-RoPE). do fp32. */
int llmt_attention_bwd(const void* q, const void* k, const void* v, const void* o,
                       const float* lse, const float* dout, float* dq, float* dk, float* dv,
                       int B, int S, int nq, int nkv, void* stream);
/* Config C3 end to end: raw (pre-QK-norm) q/k, v fp16; QK-RMSNorm (weights
 * q_norm/k_norm fp32 [128]) and RoPE(theta) forward, flash forward, then the
 * backward to dq_raw, dk_raw, dv (fp32). */
int llmt_attention_block_bwd(const void* q_raw, const void* k_raw, const void* v,
                             const float* q_norm, const float* k_norm, const void* dout,
                             float* dq_raw, float* dk_raw, float* dv,
                             int B, int S, int nq, int nkv, float theta, float eps, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LLMT_H */
