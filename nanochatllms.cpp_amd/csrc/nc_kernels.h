// nc_kernels.h -- host-side launchers of the gfx950 kernels (internal API
// used by the C-ABI ops and the model runtime).
#pragma once

#include "nc_runtime.h"

namespace nc {

enum NormKindHost { kNormRms = 0, kNormLayer = 1 };
enum EwOpHost { kEwSilu = 0, kEwMul = 1, kEwAdd = 2, kEwScale = 3, kEwBias = 4 };

// fp32 rows -> activation rows (write_row_from_float).
int write_rows(const float* in, int in_pitch, uint8_t* out, int out_pitch, int dtype, int cols, int rows,
               hipStream_t st);

// x rows (pointer at the first row) times weight rows -> fp32 dots.  With
// events, the launch records them at the kernel's own start and end.
int matvec_raw(const uint8_t* x, int x_dtype, int x_pitch, int n_rows, const nc_tensor* w, float* out, int out_pitch,
               hipStream_t st, hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr,
               const nc_tensor* wc = nullptr);

// One fp16 row times the fused fp16 gate|up weight [2f, K] with the SwiGLU
// epilogue: the fp16 row m[f] out.  Built for f a multiple of 4 and the
// K the unrolled decode kernel covers (matvec_f16_glu_supported).
bool matvec_f16_glu_supported(const nc_tensor* w);
int matvec_f16_glu(const uint8_t* x, const nc_tensor* w, uint8_t* m_out, hipStream_t st,
                   hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);

// The norm of one fp16 row fused into the fp16 decode matvec that consumes
// it (d = 2048 or 2304): kind 0 layer_norm (nb the bias), 1 rms_norm;
// braw != nullptr adds the residual first (a + Act(Act(braw) [* bscale]),
// stored to h_out); the normalized row times w -> fp32 out, or with glu (w
// the fused gate|up weight) the SwiGLU row -> m_out.  dpos: the a / h_out
// rows sit at the device-held position.
bool dmv_f16_nrm_supported(const nc_tensor* w, int d, bool glu);
int dmv_f16_nrm_launch(int kind, const uint8_t* a, int a_pitch, const float* braw, float bscale, uint8_t* h_out,
                       int h_pitch, const uint16_t* nw, const uint16_t* nb, const nc_tensor* w, float* out,
                       uint8_t* m_out, bool glu, hipStream_t st, const int* dpos = nullptr,
                       hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr);

// x rows times Q4/Q8 weight rows -> fp32 dots on the matrix cores (the
// reference's block dot product, exact); used by matvec_raw for multi-row
// (prefill) products.
// wc (optional): the weight's chunk-major copy (chunk_layout_launch), read
// instead of w.
int gemm_q_raw(const uint8_t* x, int x_pitch, int n_rows, const nc_tensor* w, float* out, int out_pitch,
               hipStream_t st, hipEvent_t ev_start = nullptr, hipEvent_t ev_stop = nullptr,
               const nc_tensor* wc = nullptr);
// The chunk-major copy of a Q4 / Q8 weight with K % 128 == 0 (codes and
// deltas the same sizes as the weight's own) that gemm_q_raw reads.
bool chunk_layout_supported(const nc_tensor* w);
int chunk_layout_launch(const nc_tensor* w, void* codes, void* deltas, hipStream_t st);
constexpr int kGemmMinRows = 8;  // matvec_raw takes the matrix-core path from this many rows

// Norm over segments of d_norm values; with `add` the input is
// a + requant(braw) (scaled by bscale and requantized when bscale != 1),
// stored to h_out.  dpos != nullptr: a and h_out rows are taken at the
// device-held position (one row).
int norm_launch(int kind, int adt, bool add, const uint8_t* a, int a_pitch, const float* braw, int b_pitch,
                float bscale, uint8_t* h_out, int h_pitch, const uint16_t* w, const uint16_t* bias, uint8_t* out,
                int out_pitch, int d_norm, int row_cols, int rows, float post_scale, hipStream_t st,
                const int* dpos = nullptr);

// dpos != nullptr: the (single) row's position is read from the device.
int qkv_post_launch(int adt, const float* raw, int raw_pitch, int hq, int hkv, const uint16_t* bq, const uint16_t* bk,
                    const uint16_t* bv, const uint16_t* qn_w, const uint16_t* kn_w, const float* table, int d_half,
                    int start, int rows, uint8_t* q_out, int q_pitch, uint8_t* k_cache, int k_pitch,
                    uint8_t* v_cache, int v_pitch, hipStream_t st, const int* dpos = nullptr);

int silu_mul_launch(int adt, const float* raw, int raw_pitch, int f, uint8_t* out, int out_pitch, int rows,
                    hipStream_t st);

// dpos != nullptr: embeds the single token tokens[*dpos] (tokens = the
// sequence base).  out_cur (one row): the (single) row is also stored there.
int embed_launch(const nc_tensor* table, const int32_t* tokens, uint8_t* out, int out_pitch, int adt, int rows,
                 float post_scale, hipStream_t st, const int* dpos = nullptr, uint8_t* out_cur = nullptr);

int argmax_launch(const float* x, int n, int32_t* out, hipStream_t st);

// Greedy step epilogue under graph replay: argmax of x written to
// tokens[*dpos + 1], then *dpos advanced.  `scratch` is 16 zeroed bytes the
// kernel leaves zeroed.
int argmax_advance_launch(const float* x, int n, int32_t* tokens, int* dpos, unsigned long long* scratch,
                          hipStream_t st);

// One top-k / temperature sampling step (gten/sampler.cpp:90-127) of the
// logits row x[n] with the mt19937 state rng (625 words, updated): the token
// goes to tokens[pos + 1], pos being *dpos (then advanced by one) when dpos
// is given.  probs (optional): the n normalized weights.  dset (optional):
// device words {k, temp} (already clamped) read instead of top_k and temp.
int sample_topk_launch(const float* logits, int n, float temp, int top_k, uint32_t* rng, int32_t* tokens, int* dpos,
                       int pos, double* probs, hipStream_t st, const double* dset = nullptr);
void mt_seed_host(uint32_t seed, uint32_t* state);

int ew_launch(int op, int adt, const uint8_t* a, int a_pitch, const uint8_t* b, int b_pitch, const uint16_t* bias,
              float s, uint8_t* out, int out_pitch, int cols, int rows, hipStream_t st);

int rope_launch(int adt, const uint8_t* in, int in_pitch, uint8_t* out, int out_pitch, int cols, const float* table,
                int d_half, int start, int rows, hipStream_t st);

// dpos != nullptr: one query row at position *dpos over *dpos + 1 cached
// rows (decode under graph replay); max_ctx sizes the shared memory.
int attn_launch(int adt, const uint8_t* q, int q_pitch, const uint8_t* kc, int k_pitch, const uint8_t* vc, int v_pitch,
                uint8_t* out, int out_pitch, int hq, int hkv, int start, int n_ctx, hipStream_t st,
                const int* dpos = nullptr, int max_ctx = 0);

// Longest context (cached positions) the attention kernels take: Zephyr's
// max_ctx (zephyr/zephyr.h:12); TinyLlama and MiniCPM stop at 2048.
constexpr int kAttnMaxCtx = NC_MAX_CTX;

// Decode attention with the q/k/v post-processing fused in (Q8 activations;
// optional q / k / v biases, bias_add_inplace after the Linear outputs, or
// OpenELM's q / k norms): raw = the qkv matvec's fp32 row [q | k | v]; the new k / v
// rows are appended to the caches at the position (*dpos when set, else
// pos); out = the attention output Act row.  rope_cur, when set, is the
// position's RoPE (cos, sin) row at a fixed address (read instead of the
// table row, so that load does not wait for the position).
bool attn_decode_supported(int hq, int hkv, int max_ctx);
int attn_decode_launch(const float* raw, int hq, int hkv, const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                       const uint16_t* qn_w, const uint16_t* kn_w, const float* table, int d_half, int pos,
                       const int* dpos, uint8_t* kc, uint8_t* vc, int kv_pitch, uint8_t* out, int max_ctx,
                       hipStream_t st, const float* rope_cur = nullptr);
// The same for fp16 rows, with optional q / k / v biases (bias_add_inplace
// after the Linear outputs) and the RoPE pair read from the table at the
// (device-held) position.
int attn_decode_f16_launch(const float* raw, int hq, int hkv, const uint16_t* bq, const uint16_t* bk,
                           const uint16_t* bv, const uint16_t* qn_w, const uint16_t* kn_w, const float* table,
                           int d_half, int pos, const int* dpos, uint8_t* kc, uint8_t* vc, int kv_pitch, uint8_t* out,
                           int max_ctx, hipStream_t st);

}  // namespace nc
