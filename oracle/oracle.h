/*
 * oracle.h -- CPU restatement of the nanochatllms.cpp decode numerics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product (libgten_hip.so) never links or calls it.
 *
 * Every function states the reference file:line whose arithmetic it restates
 * (paths relative to the reference's src/ directory).  Byte layouts are the
 * reference's own: Q8 block = {f16 delta; i8 q[32]} (34 B), Q4 block =
 * {f16 delta; u8 p[16]} (18 B), element j of a Q4 block is the high nibble of
 * byte j (j < 16) or the low nibble of byte j-16, value = code - 7
 * (gten/quants.h:16-30, gten/quants.cpp:81-138).
 */
#ifndef NC_ORACLE_H
#define NC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same order as gten::Dtype (gten/gten_types.h:20-26). */
enum { OR_I32 = 0, OR_F16 = 1, OR_F32 = 2, OR_Q8 = 3, OR_Q4 = 4 };

#define OR_QBLOCK 32
#define OR_Q8_BLOCK_BYTES 34
#define OR_Q4_BLOCK_BYTES 18

/* ---- scalar conversions (gten/gten_types.h:69-139) ---------------------- */
float or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);
void or_fp16_to_fp32_array(const uint16_t* in, float* out, int64_t n);
void or_fp32_to_fp16_array(const float* in, uint16_t* out, int64_t n);

/* ---- row formats ---------------------------------------------------------- */
size_t or_row_bytes(int dtype, int cols);
/* read_row_to_float / write_row_from_float (gten/ops.cpp:41-123). */
void or_read_row(const void* row, int dtype, float* out, int n);
void or_write_row(const float* in, void* row, int dtype, int n);

/* Activation quantizer q8_quantize_row (gten/quants.cpp:16-30,140-158). */
void or_q8_quantize_row(const float* in, uint8_t* blocks, int n);
/* Weight quantizers q8_quantize / q4_quantize of the converters
 * (tinyllama/tinyllama_to_gten.py:24-91): torch.round (half to even),
 * fp32 delta and 1/delta, fp16 (RNE) stored delta.  n_blocks blocks of 32. */
void or_q8_quantize_weights(const float* w, int64_t n_blocks, uint8_t* out);
void or_q4_quantize_weights(const float* w, int64_t n_blocks, uint8_t* out);

/* ---- dot products (gten/ops.cpp:208-490, AVX paths) ----------------------- */
float or_dot_q8(const uint8_t* a, const uint8_t* b, int n);
float or_dot_q8_q4(const uint8_t* a, const uint8_t* b, int n);
float or_dot_f16(const uint16_t* a, const uint16_t* b, int n);
float or_dot_f32(const float* a, const float* b, int n);
float or_dot(const void* a, int adt, const void* b, int bdt, int n);

/* Sequential fp32 sum in index order (the scalar loops of gten/ops.cpp). */
float or_seq_sum(const float* y, int n);

/* ---- ops over a 2-D row-major buffer: rows [start, n_ctx) ---------------- */
/* y[r, c] = dot(x[r], w[c]) for every c, then written in out_dt
 * (matmul_2d_impl, gten/ops.cpp:579-614).  The fp32 dot results of the last
 * processed row are also returned in raw_out (length N) if non-NULL. */
void or_matmul(const void* x, int xdt, const void* w, int wdt, void* out, int odt,
               int K, int N, int start, int n_ctx, float* raw_out);
void or_rms_norm(const void* x, int dt, const uint16_t* w, void* out, int d, int start, int n_ctx);
void or_rms_norm_heads(const void* x, int dt, const uint16_t* w, void* out, int n_heads, int d_head,
                       int start, int n_ctx);
void or_layer_norm(const void* x, int dt, const uint16_t* w, const uint16_t* b, void* out, int d,
                   int start, int n_ctx);
void or_rotary_emb(const void* x, void* out, int dt, int d, int d_head, float rope_pct, int start,
                   int n_ctx);
void or_silu(const void* x, void* out, int dt, int d, int start, int n_ctx);
void or_multiply(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx);
void or_add(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx);
void or_scale(void* x, int dt, float s, int d, int start, int n_ctx);
void or_bias_add(void* x, int dt, const uint16_t* b, int d, int start, int n_ctx);
/* Causal GQA attention, rows [start, n_ctx) (gten/ops.cpp:1017-1220). */
void or_qkv_attn(const void* q, const void* k, const void* v, void* out, int dt, int n_heads,
                 int n_kv_heads, int d_head, int start, int n_ctx);
/* token_embed / copy_row (gten/ops.cpp:526-576). */
void or_token_embed(const void* table, int wdt, const int32_t* tokens, void* out, int adt, int d,
                    int start, int n_ctx);
/* First index of the maximum, strict '>' (gten/sampler.cpp:33-41). */
int or_argmax(const float* x, int n);

/* ---- expf as the reference calls it (std::exp on float) ------------------ */
float or_expf(float x);
int64_t or_expf_mismatches(const float* x, const float* y, int64_t n, int64_t* first);
int64_t or_check_expf_fn(float (*fn)(float), uint64_t start, uint64_t count, int64_t* first);

/* ---- deterministic synthetic data ---------------------------------------- */
uint64_t or_mix64(uint64_t z);
/* N(0, std) fp32 values: Irwin-Hall sum of 12 24-bit uniforms (exact integer
 * arithmetic), scaled in double and rounded once to fp32. */
void or_gen_normal(uint64_t seed, uint32_t tensor_id, float stddev, int64_t n, float* out);
/* Token ids uniform in [0, vocab). */
void or_gen_tokens(uint64_t seed, int n, int vocab, int32_t* out);

/* ---- decoder models ------------------------------------------------------- */
enum { OR_ARCH_LLAMA = 0, OR_ARCH_ZEPHYR = 1, OR_ARCH_MINICPM = 2, OR_ARCH_OPENELM = 3 };
#define OR_MAX_LAYERS 64

typedef struct {
    int arch;
    int wdtype; /* OR_F16, OR_Q8 or OR_Q4 */
    int n_vocab;
    int n_embd;
    int n_layers;
    int d_head;
    int max_ctx;
    int eos;
    float rope_pct;
    int n_heads[OR_MAX_LAYERS];
    int n_kv_heads[OR_MAX_LAYERS];
    int n_ffn[OR_MAX_LAYERS];
} or_config;

/* Weight tensor slots; tensor id = layer * 32 + slot for per-layer tensors,
 * OR_TID_* for the global ones.  Matches the generator's seeding. */
enum {
    OR_W_Q = 0, OR_W_K, OR_W_V, OR_W_O, OR_W_GATE, OR_W_UP, OR_W_DOWN,
    OR_W_ATTN_NORM, OR_W_ATTN_NORM_B, OR_W_MLP_NORM, OR_W_MLP_NORM_B,
    OR_W_Q_BIAS, OR_W_K_BIAS, OR_W_V_BIAS, OR_W_Q_NORM, OR_W_K_NORM,
    OR_W_NSLOTS
};
#define OR_TID_EMB 0xFFFF0u
#define OR_TID_NORM 0xFFFF1u
#define OR_TID_NORM_B 0xFFFF2u
#define OR_TID_LM 0xFFFF3u

typedef struct or_model or_model;

/* Shape of weight tensor (layer, slot); returns 0 if the arch has no such
 * tensor.  rows/cols describe the 2-D [rows, cols] weight (1-D: rows = 1). */
int or_weight_shape(const or_config* cfg, int layer, int slot, int* rows, int* cols, int* dtype);
/* Synthetic weight in its stored format: matrices N(0, 0.02) quantized to
 * wdtype (or fp16), norm gains 1.0, norm biases 0, qkv biases N(0, 0.02). */
void or_make_weight(const or_config* cfg, uint64_t seed, int layer, int slot, void* out);

or_model* or_model_create(const or_config* cfg);
void or_model_free(or_model* m);
/* Pointer to the stored weight (layer, slot), layer = -1 for global slots
 * addressed by OR_TID_* values. */
void* or_model_weight(or_model* m, int layer, int slot);
void or_model_init_synthetic(or_model* m, uint64_t seed);
/* Model::logits(tokens, start_pos): rows [start_pos, n_tokens), last row's
 * fp32 logits into `logits` (length n_vocab). */
void or_model_logits(or_model* m, const int32_t* tokens, int n_tokens, int start_pos, float* logits);
/* Bytes of the residual stream after layer `layer` (row `row`), Act dtype. */
const void* or_model_layer_out(or_model* m, int layer, int row);
size_t or_model_act_row_bytes(or_model* m);
/* greedy_sample (gten/sampler.cpp:11-60) without the tokenizer: returns the
 * number of generated tokens (stops at eos), tokens appended into out. */
int or_generate_greedy(or_model* m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out);
/* topk_sample (gten/sampler.cpp:63-143) with std::mt19937(seed) in place of
 * the random_device-seeded generator: n_gen steps, stopping before EOS. */
int or_generate_topk(or_model* m, const int32_t* prompt, int n_prompt, int n_gen, float temp, int top_k,
                     uint32_t seed, int32_t* out);

/* ---- top-k / temperature sampling (oracle_sample.c) ---------------------- */
/* std::mt19937 state: 624 words, then the index of the next word. */
void or_mt_seed(uint32_t seed, uint32_t* st);
uint32_t or_mt_next(uint32_t* st);
double or_mt_canonical(uint32_t* st);
/* One sampling step of topk_sample (gten/sampler.cpp:90-127) on a logits
 * row, drawing from the generator st; probs_out (n doubles, may be NULL)
 * receives the normalized weights std::discrete_distribution holds.
 * Requires 1 <= min(top_k, 1000) <= n and temp > 0. */
int or_topk_sample(const float* logits, int n, float temp, int top_k, uint32_t* st, double* probs_out);
/* glibc exp (std::exp on double) and checks of another exp against it. */
double or_exp(double x);
void or_exp_probe_inputs(uint64_t seed, int64_t start, int64_t n, double* x);
int64_t or_check_exp_fn(double (*fn)(double), uint64_t seed, int64_t count, double* first_x);
int64_t or_exp_mismatches(const double* x, const double* y, int64_t n, int64_t* first);

#ifdef __cplusplus
}
#endif
#endif
