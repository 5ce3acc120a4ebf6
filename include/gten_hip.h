/*
 * gten_hip.h -- C-ABI of the MI355X (gfx950) decode path of nanochatllms.cpp.
 *
 * The reference has no FFI layer: its operator API is the C++ free functions
 * of gten::ops (src/gten/ops.h:10-40) over gten::Tensor (src/gten/tensor.h),
 * driven by the model classes' logits() (src/gten/abc.h:12-28).  Each entry
 * point below names the reference interface it replaces.  All compute calls
 * are asynchronous on `stream` (a hipStream_t; NULL = the library's stream)
 * and return NC_OK or a negative status; nc_last_error() describes the last
 * failure.  Device pointers are plain HBM addresses; no torch types.
 *
 * Layouts (also in nanochatllms.cpp_amd/csrc/nc_layout.h):
 *   activation row, dtype Q8 : [nb*32 int8 codes][nb fp16 deltas][pad to 16 B]
 *   activation row, dtype F16: [cols fp16][pad], F32: [cols fp32][pad]
 *   weights Q4/Q8: codes + separate fp16 delta array, lane-permuted per block;
 *   weights F16: 64-column groups interleaved over 8-row groups.
 * nc_act_from_reference / nc_weight_from_reference convert from the
 * reference's byte layouts (34-byte Q8 blocks, 18-byte Q4 blocks).
 */
#ifndef GTEN_HIP_H
#define GTEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NC_OK 0
#define NC_ERR_ARG (-1)
#define NC_ERR_HIP (-2)
#define NC_ERR_NOMEM (-3)
#define NC_ERR_STATE (-4)

/* Dtypes, numbered as gten::Dtype (src/gten/gten_types.h:20-26). */
#define NC_I32 0
#define NC_F16 1
#define NC_F32 2
#define NC_Q8 3
#define NC_Q4 4

/* A device tensor: `rows` x `cols` values.  Activations: `data` holds rows of
 * `pitch` bytes (deltas inside each Q8 row, `deltas` unused).  Weights: `data`
 * holds the codes (or fp16 values), `deltas` the fp16 block deltas. */
typedef struct nc_tensor {
    void* data;
    void* deltas;
    int dtype;
    int rows;
    int cols;
    int pitch;
} nc_tensor;

/* ---- runtime ---------------------------------------------------------------- */
int nc_init(int device);
const char* nc_last_error(void);
int nc_malloc(void** ptr, size_t bytes);
int nc_free(void* ptr);
int nc_memcpy_h2d(void* dst, const void* src, size_t bytes);
int nc_memcpy_d2h(void* dst, const void* src, size_t bytes);
/* Device-to-device copy by a plain streaming kernel (bytes a multiple of
 * 16, 16-byte aligned pointers); also the reference point that scales HBM
 * byte counters of the profiler. */
int nc_copy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int nc_memset_d(void* dst, int value, size_t bytes);
int nc_synchronize(void);

/* ---- layouts (host-side, no GPU needed) -------------------------------------- */
/* Bytes of one activation row (Tensor::bstride(0) of the reference,
 * src/gten/tensor.h:96-116, in the device layout). */
int nc_act_pitch(int dtype, int cols);
/* Reference activation rows (Q8: 34-byte blocks; F16/F32 plain) <-> device
 * rows, both on the host. */
int nc_act_from_reference(const void* ref, void* dev_layout, int dtype, int rows, int cols);
int nc_act_to_reference(const void* dev_layout, void* ref, int dtype, int rows, int cols);
/* Sizes of a weight in the device layout. */
int nc_weight_bytes(int dtype, int rows, int cols, size_t* code_bytes, size_t* delta_bytes);
/* Reference weight payload (as read_into_weight stores it, src/gten/utils.cpp:
 * 29-48: Q8/Q4 blocks or fp16 rows) -> device layout, on the host. */
int nc_weight_from_reference(const void* ref, int dtype, int rows, int cols, void* codes, void* deltas);

/* ---- weights on the device ---------------------------------------------------- */
/* Deterministic N(0, stddev) fp32 values: Irwin-Hall sum of 12 24-bit
 * uniforms from a counter-based splitmix64 hash of (seed, tensor_id, index). */
int nc_gen_normal(uint64_t seed, uint32_t tensor_id, float stddev, int64_t n, float* out, void* stream);
/* q8_quantize / q4_quantize of the converters (src/tinyllama/
 * tinyllama_to_gten.py:24-91) from device fp32 [rows, cols] into `out`
 * (data/deltas preallocated with nc_weight_bytes).  F16 converts with RNE. */
int nc_weight_quantize(const float* w, nc_tensor* out, void* stream);

/* ---- ops: gten::ops (src/gten/ops.h:10-40) on device tensors ----------------- */
/* Each processes rows [start, n_ctx) like the reference's start_pos. */
/* token_embed (ops.h:37): out[r] = table[tokens[r]], Q4 rows requantized to Q8. */
int nc_token_embed(const nc_tensor* table, const int32_t* tokens, nc_tensor* out, int start, int n_ctx,
                   void* stream);
/* matmul_2d (ops.h:18): out[r, c] = dot(x[r], w[c]) with the reference's
 * lane/block summation order; out dtype F32 gives the raw dot products,
 * an activation dtype stores them requantized. */
int nc_matmul_2d(const nc_tensor* x, const nc_tensor* w, nc_tensor* out, int start, int n_ctx, void* stream);
/* nc_matmul_2d without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  An
 * activation-dtype output is staged in a fixed per-GPU array of
 * NC_NOALLOC_STAGE_BYTES instead of library-allocated memory, so
 * (n_ctx - start) * w->rows * 4 must not exceed it (else NC_ERR_ARG); an F32
 * output needs no staging.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race. */
#define NC_NOALLOC_STAGE_BYTES (8u << 20)
int nc_matmul_2d_noalloc(const nc_tensor* x, const nc_tensor* w, nc_tensor* out, int start, int n_ctx,
                         void* stream);
/* rms_norm (ops.h:26): d_norm = cols for the 2-D op, the head size for the
 * per-head (3-D) op; w is fp16 [d_norm]. */
int nc_rms_norm(const nc_tensor* x, const uint16_t* w, nc_tensor* out, int d_norm, int start, int n_ctx,
                void* stream);
/* layer_norm (ops.h:16). */
int nc_layer_norm(const nc_tensor* x, const uint16_t* w, const uint16_t* b, nc_tensor* out, int start, int n_ctx,
                  void* stream);
/* rotary_emb (ops.h:28).  `table` is nc_rope_table's (cos, sin) pairs. */
int nc_rotary_emb(const nc_tensor* x, nc_tensor* out, int d_head, float rope_pct, const float* table, int start,
                  int n_ctx, void* stream);
/* Host: (cos, sin) of m * powf(10000, -(2j/d_r)) for m < max_ctx, j < d_r/2,
 * evaluated with the host libm exactly as src/gten/ops.cpp:801-812. */
int nc_rope_table(int max_ctx, int d_head, float rope_pct, float* out);
int nc_silu(const nc_tensor* x, nc_tensor* out, int start, int n_ctx, void* stream);          /* ops.h:32 */
int nc_multiply(const nc_tensor* a, const nc_tensor* b, nc_tensor* out, int start, int n_ctx,
                void* stream);                                                                /* ops.h:20 */
int nc_add(const nc_tensor* a, const nc_tensor* b, nc_tensor* out, int start, int n_ctx, void* stream); /* ops.h:12 */
int nc_scale(nc_tensor* x, float s, int start, int n_ctx, void* stream);                        /* ops.h:30 */
int nc_bias_add(nc_tensor* x, const uint16_t* b, int start, int n_ctx, void* stream);           /* ops.h:14 */
/* qkv_attn (ops.h:24): causal GQA attention of rows [start, n_ctx), n_ctx up
 * to NC_MAX_CTX positions. */
int nc_qkv_attn(const nc_tensor* q, const nc_tensor* k, const nc_tensor* v, nc_tensor* out, int n_heads,
                int n_kv_heads, int d_head, int start, int n_ctx, void* stream);
/* The device's std::exp(float) as softmax and SiLU use it (src/gten/
 * ops.cpp:752,1072): y[i] = expf(x[i]). */
int nc_expf(const float* x, float* y, int64_t n, void* stream);
/* The same function evaluated on the host CPU (no GPU needed). */
float nc_expf_host(float x);
/* The left-to-right fp32 sum of non-negative terms of rms_norm (src/gten/
 * ops.cpp:833-835) as the fused decode kernels compute it on the device (a
 * workgroup-parallel restatement with the sequential loop's result):
 * out[b] = sum of t[b*n .. b*n+n), n a multiple of 256 up to 4096; fast[b]
 * = 1 when the parallel path (not its sequential fallback) produced it. */
int nc_block_seq_sum(const float* t, int n, int count, float* out, int* fast, void* stream);
/* Host run of the same decomposition (no GPU): binades predicted from a
 * double prefix scaled by (1 + skew); *fast = 1 when its checks passed. */
float nc_seq_sum_nonneg_host(const float* t, int n, double skew, int* fast);
/* The left-to-right fp32 sum of signed values of layer_norm's mean (src/gten/
 * ops.cpp:673-676) as the fused layer-norm prologues compute it on the
 * device, for values on the fp16 grid (multiples of 2^-24 below 2^17: fp16
 * activations, Q8 codes times fp16 deltas): out[b] = sum of x[b*n ..
 * b*n+n) for n = 1024, 2048 or 2304; passes[b] = the parallel passes made
 * (0 when its sequential fallback ran). */
int nc_block_seq_sum_grid(const float* x, int n, int count, float* out, int* passes, void* stream);
/* Host run of the same decomposition (no GPU); plant = 1 drops the rounding
 * error after each rounding step (a planted mistake for tests). */
float nc_seq_sum_grid_host(const float* x, int n, int plant, int* passes);
/* Test hook (no counterpart in the reference): the speculative fused decode
 * matvecs (q|k|v and gate|up with a norm prologue) compute their weight
 * terms from a row normalized with a predicted statistic (rms_norm: the sum
 * of squares; layer_norm: the variance), beside the exact sums, and
 * recompute every block whose exact row differs.  Launches made after this
 * call scale the prediction by skew (1: none), so that tests can force the
 * recomputation; when fixups (device int) is not null, each workgroup that
 * recomputed adds one to it.  Results are the same for every skew > 0. */
int nc_debug_spec(float skew, void* fixups);
/* Greedy pick of greedy_sample (src/gten/sampler.cpp:33-41): first index of
 * the maximum. */
int nc_argmax(const float* x, int n, int32_t* out, void* stream);
/* ---- tokenizers (host) ----------------------------------------------------
 * The reference's LLamaTokenizer (src/gten/tokenizer.cpp:25-248: BPE with
 * scores, byte fallback) and Gpt2Tokenizer (tokenizer.cpp:251-334: regex
 * words, longest entries), with their results.  A tokenizer handle is a
 * host object; none of these calls touch the GPU. */
/* LLamaTokenizer(path, vocab_size, eos, prompt_prefix, prompt_suffix,
 * tokens_prefix, tokens_suffix) (tokenizer.cpp:25-65). */
int nc_tokenizer_load_bpe(const char* path, int vocab_size, int eos, const char* prompt_prefix,
                          const char* prompt_suffix, const int32_t* tokens_prefix, int n_prefix,
                          const int32_t* tokens_suffix, int n_suffix, void** tokenizer);
/* Gpt2Tokenizer(vocab_path, n_vocab, eos) (tokenizer.cpp:251-269) with its
 * encode prefix and suffix tokens as arguments (tokenizer.h:59-60). */
int nc_tokenizer_load_words(const char* path, int vocab_size, int eos, const int32_t* tokens_prefix, int n_prefix,
                            const int32_t* tokens_suffix, int n_suffix, void** tokenizer);
/* The tokenizer nanochat.cpp builds for "tinyllama", "zephyr", "minicpm",
 * "openelm_sm|md|lg" (src/nanochat.cpp:189-229) from its vocabulary file. */
int nc_tokenizer_load_for_model(const char* model, const char* path, void** tokenizer);
/* Tokenizer::encode (tokenizer.cpp:99-130, 283-334): *n_out = the token
 * count; an error when it exceeds cap. */
int nc_tokenizer_encode(void* tokenizer, const char* text, int32_t* out, int cap, int* n_out);
/* Tokenizer::decode(prev_token, token) (tokenizer.cpp:77-90, 276-279): the
 * text of one token, valid until the tokenizer is freed. */
const char* nc_tokenizer_decode(void* tokenizer, int prev_token, int token);
int nc_tokenizer_eos(void* tokenizer);
int nc_tokenizer_free(void* tokenizer);

/* std::mt19937(seed) as a 625-word state (624 words, then the index of the
 * next word), written to host memory `state`; the reference seeds its
 * generator from std::random_device (src/gten/sampler.cpp:70-71). */
int nc_rng_seed(uint32_t seed, uint32_t* state);
/* One sampling step of topk_sample (src/gten/sampler.cpp:90-127) on the
 * device: logits[n_vocab] (device), top_k and temp clamped to 1000 and 2.0
 * as sampler.cpp:66-67 does, the mt19937 state rng_state (device, 625
 * words) advanced by the draw, the token to *token (device).  probs (device,
 * n_vocab doubles, may be NULL) receives the normalized weights the
 * discrete distribution holds.  Errors: top_k < 1 or above n_vocab,
 * temp <= 0 or NaN, n_vocab < 2. */
int nc_sample_topk(const float* logits, int n_vocab, float temp, int top_k, uint32_t* rng_state, int32_t* token,
                   double* probs, void* stream);
/* std::exp on double as the sampler uses it (src/gten/sampler.cpp:112-113,
 * the host glibc's exp): y[i] = exp(x[i]) on the device. */
int nc_exp(const double* x, double* y, int64_t n, void* stream);
/* The same function evaluated on the host CPU (no GPU needed). */
double nc_exp_host(double x);

/* ---- models: gten::Model::logits (src/gten/abc.h:25) and greedy_sample ------ */
#define NC_ARCH_LLAMA 0   /* src/tinyllama */
#define NC_ARCH_ZEPHYR 1  /* src/zephyr */
#define NC_ARCH_MINICPM 2 /* src/minicpm */
#define NC_ARCH_OPENELM 3 /* src/openelm */
#define NC_MAX_LAYERS 64

typedef struct nc_model_config {
    int arch;
    int wdtype; /* NC_F16, NC_Q8 or NC_Q4 (ModuleDtype mFloat16 / mQint8 / mQint4) */
    int n_vocab;
    int n_embd;
    int n_layers;
    int d_head;
    int max_ctx; /* inference context: prompt + generated tokens, <= NC_MAX_CTX */
    int eos;
    float rope_pct;
    int n_heads[NC_MAX_LAYERS];
    int n_kv_heads[NC_MAX_LAYERS];
    int n_ffn[NC_MAX_LAYERS];
} nc_model_config;

/* Weight slots (layer >= 0) and global tensors (layer = -1). */
#define NC_W_Q 0
#define NC_W_K 1
#define NC_W_V 2
#define NC_W_O 3
#define NC_W_GATE 4
#define NC_W_UP 5
#define NC_W_DOWN 6
#define NC_W_ATTN_NORM 7
#define NC_W_ATTN_NORM_B 8
#define NC_W_MLP_NORM 9
#define NC_W_MLP_NORM_B 10
#define NC_W_Q_BIAS 11
#define NC_W_K_BIAS 12
#define NC_W_V_BIAS 13
#define NC_W_Q_NORM 14
#define NC_W_K_NORM 15
#define NC_TID_EMB 0xFFFF0
#define NC_TID_NORM 0xFFFF1
#define NC_TID_NORM_B 0xFFFF2
#define NC_TID_LM 0xFFFF3

/* Model constructor (TinyLLama(n_ctx, dtype) and siblings): allocates every
 * weight and every [max_ctx, d] activation buffer in HBM.  max_ctx may be up
 * to NC_MAX_CTX, the longest max_ctx of the reference's models (Zephyr's,
 * src/zephyr/zephyr.h:12); its default inference context is 1024
 * (src/nanochat.cpp:40). */
#define NC_MAX_CTX 4096
int nc_model_create(const nc_model_config* cfg, void** model);
int nc_model_free(void* model);
/* Synthetic weights generated and quantized on the device (same values as
 * the CPU generator for the same seed). */
int nc_model_init_synthetic(void* model, uint64_t seed);
/* One weight from its reference payload bytes (read_into_weight,
 * src/gten/utils.cpp:29-48). */
int nc_model_set_weight(void* model, int layer, int slot, const void* ref_bytes, size_t n_bytes);
/* Model::load_from_ckpt (src/tinyllama/tinyllama.cpp:131-187 and its
 * siblings; records read as gten::read_layer_header / read_into_weight,
 * src/gten/utils.cpp:29-61): every weight from a .gten checkpoint file, in
 * the model's file order.  A wrong magic number, a payload size that does
 * not match the tensor, or a truncated file is an error (the reference
 * asserts). */
int nc_model_load_gten(void* model, const char* path);
/* The stored weight back in the reference's payload bytes. */
int nc_model_get_weight(void* model, int layer, int slot, void* ref_bytes, size_t n_bytes);
/* Model::logits(tokens, start_pos): processes rows [start_pos, n_tokens) and
 * copies the last row's fp32 logits to `logits` (host, n_vocab floats). */
int nc_model_logits(void* model, const int32_t* tokens, int n_tokens, int start_pos, float* logits);
/* Residual stream after `layer` at `row`, in the reference's byte layout. */
int nc_model_layer_out(void* model, int layer, int row, void* ref_bytes);
/* greedy_sample (src/gten/sampler.cpp:11-60) without the tokenizer: prefill
 * the prompt, then up to n_gen greedy steps with device-side argmax; stops
 * at eos.  *n_out = tokens produced. */
int nc_model_generate(void* model, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out, int* n_out);
/* topk_sample (src/gten/sampler.cpp:63-143) without the tokenizer and with
 * std::mt19937(seed) in place of the random_device-seeded generator: prefill
 * the prompt, then n_gen sampled tokens (logits, sampling and the next
 * step's inputs on the device, no host round trip); stops at eos.
 * *n_out = tokens produced. */
int nc_model_generate_topk(void* model, const int32_t* prompt, int n_prompt, int n_gen, float temp, int top_k,
                           uint32_t seed, int32_t* out, int* n_out);
/* Split form for timing: nc_model_prefill runs the start_pos = 0 call and
 * leaves the greedy token on the device; nc_model_decode runs n_steps more
 * calls (no host round trip between steps) and appends the tokens. */
int nc_model_prefill(void* model, const int32_t* prompt, int n_prompt);
int nc_model_decode(void* model, int n_steps, int32_t* out);
/* The same split for topk_sample's loop (src/gten/sampler.cpp:78-135, with
 * std::mt19937(seed)): nc_model_sample_begin runs the prompt and samples the
 * first token; nc_model_sample_steps samples n_steps more and copies every
 * token sampled since the prompt to out (when set). */
int nc_model_sample_begin(void* model, const int32_t* prompt, int n_prompt, float temp, int top_k, uint32_t seed);
int nc_model_sample_steps(void* model, int n_steps, int32_t* out);
/* The configuration the model was created with. */
int nc_model_get_config(void* model, nc_model_config* cfg);

/* ---- the text path: greedy_sample / topk_sample (src/gten/sampler.cpp) ----
 * Prompt text in, generated text out: the tokenizer's encode of the prompt
 * (chat prefixes and suffixes included), the model's tokens up to
 * n_predict - (prompt tokens) of them or the tokenizer's eos, and each
 * token's decode(prev, token) passed to `sink` as it is produced (prev = 1
 * for the first, as the reference's `(i == 0) ? 1 : tokens.back()`), then
 * "\n" -- the text the reference writes to std::cerr.  n_predict <= 0 takes
 * the model's max_ctx (the reference's min(inference ctx, train ctx) is the
 * max_ctx its callers give the model).  *n_tokens = tokens produced (eos not
 * counted).  Each call starts from position 0 like the reference's.
 * topk_sample clamps top_k to 1000 and temp to 2 as the reference does and
 * draws from std::mt19937(seed) in place of a random_device seed. */
typedef void (*nc_text_sink)(const char* text, void* user);
int nc_greedy_sample(void* model, void* tokenizer, const char* prompt, int n_predict, nc_text_sink sink, void* user,
                     int* n_tokens);
int nc_topk_sample(void* model, void* tokenizer, const char* prompt, int n_predict, float temp, int top_k,
                   uint32_t seed, nc_text_sink sink, void* user, int* n_tokens);
/* Timing of the model's matvec launches (the reference's Linear time,
 * print_perf in src/tinyllama/tinyllama.cpp:140-193, measured per launch):
 * between begin and end, HIP events on the model's stream bracket up to
 * max_launches matvec launches; end reports their count, summed duration,
 * summed algorithmic HBM bytes (weights once + activation rows + fp32
 * outputs) and the shortest / longest launch. */
int nc_model_profile_begin(void* model, int max_launches);
int nc_model_profile_end(void* model, int* launches, double* total_ms, double* total_bytes, double* min_ms,
                         double* max_ms);
/* The same launches one by one (after profile_end): duration, algorithmic
 * bytes and role (NC_PROF_*, plus NC_PROF_FUSED for the fused single-row
 * decode kernels, whose bytes also count their prologue inputs and
 * residual / SwiGLU rows); *n_out <= cap launches written. */
#define NC_PROF_QKV 0
#define NC_PROF_O 1
#define NC_PROF_GATE_UP 2
#define NC_PROF_DOWN 3
#define NC_PROF_LM_HEAD 4
#define NC_PROF_FUSED 8
int nc_model_profile_launches(void* model, int cap, float* ms, double* bytes, int* kind, int* n_out);

#ifdef __cplusplus
}
#endif
#endif
