// llm_train — LoRA fine-tuning driver on top of libllmt's native layer.
//
// Same flags, files and output as the reference driver (src/train.cu:172-311):
//   --lr 3e-4 --steps 1000 --seq-len 512 --save-every 100 --log-every 10
// reads data/train_tokens.bin ([int32 n][int32 ids], python/tokenize_input.py
// :22-26), frozen weights from weights/<hf_param_name>.bin (raw fp32,
// src/train.cu:56-89), trains on non-overlapping (seq_len + 1)-token windows
// taken in order (window (step - 1) % num_seqs, src/train.cu:253-258) and
// writes weights/lora_step{N}_layer{L}_{wq|wk|wv|wo}_{A|B}.bin every
// --save-every steps and at the end (src/train.cu:146-170).
//
// Additions of this build (defaults reproduce the reference):
//   --batch B      B consecutive windows per step (loss = mean over B (S - 1) rows)
//   --int8         int8 frozen weights (the quantize.cu recipe, on the device)
//   --data PATH    token file (default data/train_tokens.bin)
//   --weights DIR  weights and adapter directory (default weights)
//   --seed N       adapter init seed (A ~ 0.02 N(0, 1), B = 0 as in the reference)
//   --resume N     continue after step N from lora_step{N}_* and lora_step{N}_adamw.bin
//   --no-graph     launch the step eagerly instead of replaying a HIP graph
//   --dims H,L,NQ,NKV,I,V  another Qwen3-shaped model (head_dim 128, rank 16,
//                  alpha 32); default Qwen3-1.7B (include/config.h:5-21)
// Errors print the library message and exit with status 1, as the reference
// exits on any failure (include/utils.h:10-28).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include <string>
#include <vector>

#include "llmt.h"

static void die_llmt(const char* what, int rc) {
  fprintf(stderr, "ERROR: %s failed (%d): %s\n", what, rc, llmt_last_error());
  exit(1);
}

#define CHECK_LLMT(call)              \
  do {                                \
    int rc_ = (call);                 \
    if (rc_ != LLMT_OK) die_llmt(#call, rc_); \
  } while (0)

#define CHECK_HIP(call)                                                              \
  do {                                                                               \
    hipError_t e_ = (call);                                                          \
    if (e_ != hipSuccess) {                                                          \
      fprintf(stderr, "ERROR: %s: %s\n", #call, hipGetErrorString(e_));              \
      exit(1);                                                                       \
    }                                                                                \
  } while (0)

struct Args {
  float lr = 3e-4f;
  int steps = 1000;
  int seq_len = 512;
  int save_every = 100;
  int log_every = 10;
  int batch = 1;
  int int8 = 0;
  int resume = 0;
  int graph = 1;
  unsigned long long seed = 1234;
  int dims[6] = {0, 0, 0, 0, 0, 0};  // H, L, NQ, NKV, I, V (0: Qwen3-1.7B)
  std::string data = "data/train_tokens.bin";
  std::string weights = "weights";
};

static Args parse(int argc, char** argv) {
  Args a;
  for (int i = 1; i < argc; ++i) {
    const char* f = argv[i];
    const bool has = i + 1 < argc;
    if (!strcmp(f, "--lr") && has) a.lr = (float)atof(argv[++i]);
    else if (!strcmp(f, "--steps") && has) a.steps = atoi(argv[++i]);
    else if (!strcmp(f, "--seq-len") && has) a.seq_len = atoi(argv[++i]);
    else if (!strcmp(f, "--save-every") && has) a.save_every = atoi(argv[++i]);
    else if (!strcmp(f, "--log-every") && has) a.log_every = atoi(argv[++i]);
    else if (!strcmp(f, "--batch") && has) a.batch = atoi(argv[++i]);
    else if (!strcmp(f, "--data") && has) a.data = argv[++i];
    else if (!strcmp(f, "--weights") && has) a.weights = argv[++i];
    else if (!strcmp(f, "--seed") && has) a.seed = strtoull(argv[++i], nullptr, 10);
    else if (!strcmp(f, "--resume") && has) a.resume = atoi(argv[++i]);
    else if (!strcmp(f, "--dims") && has) {
      if (sscanf(argv[++i], "%d,%d,%d,%d,%d,%d", &a.dims[0], &a.dims[1], &a.dims[2], &a.dims[3],
                 &a.dims[4], &a.dims[5]) != 6) {
        fprintf(stderr, "ERROR: --dims wants H,L,NQ,NKV,I,V\n");
        exit(1);
      }
    } else if (!strcmp(f, "--int8")) a.int8 = 1;
    else if (!strcmp(f, "--no-graph")) a.graph = 0;
    else {
      fprintf(stderr, "ERROR: unknown or incomplete argument %s\n", f);
      exit(1);
    }
  }
  if (a.steps < 0 || a.seq_len < 2 || a.batch < 1 || a.save_every < 1 || a.log_every < 1 ||
      a.resume < 0) {
    fprintf(stderr, "ERROR: invalid arguments\n");
    exit(1);
  }
  return a;
}

static std::vector<int32_t> read_tokens(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) {
    fprintf(stderr,
            "ERROR: %s not found. Tokenize training data first:\n"
            "  python python/tokenize_input.py --train <text_file>\n",
            path.c_str());
    exit(1);
  }
  int32_t n = 0;
  if (fread(&n, 4, 1, f) != 1 || n < 0) {
    fprintf(stderr, "ERROR: %s: bad header\n", path.c_str());
    exit(1);
  }
  std::vector<int32_t> ids((size_t)n);
  if (fread(ids.data(), 4, (size_t)n, f) != (size_t)n) {
    fprintf(stderr, "ERROR: %s: short read\n", path.c_str());
    exit(1);
  }
  fclose(f);
  return ids;
}

int main(int argc, char** argv) {
  const Args a = parse(argc, argv);
  printf("Training config: lr=%.2e steps=%d seq_len=%d\n", a.lr, a.steps, a.seq_len);

  const std::vector<int32_t> ids = read_tokens(a.data);
  printf("Loaded %d training tokens\n", (int)ids.size());
  const int win = a.seq_len + 1;
  const int num_seqs = (int)(ids.size() / (size_t)win);
  if (num_seqs == 0) {
    fprintf(stderr, "ERROR: need at least %d tokens, got %d\n", win, (int)ids.size());
    return 1;
  }
  printf("Training sequences available: %d\n", num_seqs);

  llmt_dims dims;
  llmt_dims_qwen3_1_7b(&dims);
  if (a.dims[0]) {
    dims.hidden = a.dims[0];
    dims.n_layers = a.dims[1];
    dims.n_heads = a.dims[2];
    dims.n_kv_heads = a.dims[3];
    dims.intermediate = a.dims[4];
    dims.vocab = a.dims[5];
  }
  for (int t : ids)
    if (t < 0 || t >= dims.vocab) {
      fprintf(stderr, "ERROR: token id %d outside [0, %d)\n", t, dims.vocab);
      return 1;
    }
  llmt_ctx* ctx = nullptr;
  CHECK_LLMT(llmt_ctx_create(&dims, a.batch, a.seq_len,
                             a.int8 ? LLMT_WEIGHTS_I8 : LLMT_WEIGHTS_F16, nullptr, &ctx));
  CHECK_LLMT(llmt_load_weights_dir(ctx, a.weights.c_str()));
  printf("Frozen model loaded from %s/ (%s)\n", a.weights.c_str(), a.int8 ? "int8" : "fp16");

  if (a.resume) {
    CHECK_LLMT(llmt_lora_load(ctx, a.weights.c_str(), a.resume));
    CHECK_LLMT(llmt_lora_load_state(ctx, a.weights.c_str(), a.resume));
    printf("Resumed LoRA adapters and AdamW state at step %d\n", a.resume);
  } else {
    CHECK_LLMT(llmt_lora_init(ctx, a.seed, 0.02f, 0.0f));
    printf("LoRA adapters initialized (rank=%d, alpha=%d, scale=%.1f)\n", dims.rank,
           (int)dims.alpha, dims.alpha / dims.rank);
  }
  CHECK_LLMT(llmt_set_graph(ctx, a.graph));

  const size_t per = (size_t)a.batch * a.seq_len;
  int32_t *d_tok = nullptr, *d_tgt = nullptr;
  CHECK_HIP(hipMalloc(&d_tok, per * 4));
  CHECK_HIP(hipMalloc(&d_tgt, per * 4));
  std::vector<int32_t> h_tok(per), h_tgt(per);
  mkdir(a.weights.c_str(), 0755);

  const llmt_hparams hp = {a.lr, 0.9f, 0.999f, 1e-8f, 0.01f};
  printf("\n=== Training ===\n");
  float running = 0.f;
  int count = 0;
  const int last = a.resume + a.steps;
  for (int step = a.resume + 1; step <= last; ++step) {
    // windows (step - 1) * B + b, in order: tokens [0, S), targets [1, S]
    for (int b = 0; b < a.batch; ++b) {
      const long long w = ((long long)(step - 1) * a.batch + b) % num_seqs;
      const int32_t* s = ids.data() + w * win;
      memcpy(h_tok.data() + (size_t)b * a.seq_len, s, (size_t)a.seq_len * 4);
      memcpy(h_tgt.data() + (size_t)b * a.seq_len, s + 1, (size_t)a.seq_len * 4);
    }
    CHECK_HIP(hipMemcpy(d_tok, h_tok.data(), per * 4, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(d_tgt, h_tgt.data(), per * 4, hipMemcpyHostToDevice));
    float loss = 0.f;
    CHECK_LLMT(llmt_step(ctx, d_tok, d_tgt, a.batch, &hp, step, &loss));
    running += loss;
    ++count;
    if (step % a.log_every == 0) {
      printf("step %4d  loss %.4f  (avg %.4f)\n", step, loss, running / count);
      fflush(stdout);
      running = 0.f;
      count = 0;
    }
    if (step % a.save_every == 0) {
      CHECK_LLMT(llmt_lora_save(ctx, a.weights.c_str(), step));
      CHECK_LLMT(llmt_lora_save_state(ctx, a.weights.c_str(), step));
      printf("Saved LoRA weights at step %d\n", step);
    }
  }
  CHECK_LLMT(llmt_lora_save(ctx, a.weights.c_str(), last));
  CHECK_LLMT(llmt_lora_save_state(ctx, a.weights.c_str(), last));
  printf("Saved LoRA weights at step %d\n", last);
  printf("\nTraining complete.\n");

  CHECK_HIP(hipFree(d_tok));
  CHECK_HIP(hipFree(d_tgt));
  CHECK_LLMT(llmt_ctx_destroy(ctx));
  return 0;
}
