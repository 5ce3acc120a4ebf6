// nc_decode.h -- the fused matvec kernels of the single-row decode step
// (Q8 activations, Q4/Q8 weights): prologue and epilogue kinds and the
// launch arguments.
#pragma once

#include "nc_runtime.h"

namespace nc {

// Prologue: how the activation row the matvec consumes is produced.
//   PRO_X       the stored Act row at x (attention output)
//   PRO_RMS     rms_norm(x[pos]) with gain norm_w (then post_scale)
//   PRO_RES_RMS h = Act(res_in[pos] + Act(raw_in [* bscale])) -- the
//               residual add of the previous Linear's output -- stored to
//               res_out[pos], then rms_norm(h) as PRO_RMS
//   PRO_LN, PRO_RES_LN  the same with layer_norm (gain norm_w, bias norm_b)
//               in place of rms_norm (Zephyr; rows of 2048 values)
// PRO_RMS / PRO_LN with x_pitch = 0 read the row at x itself, and
// PRO_RES_RMS / PRO_RES_LN with res_cur set read the residual row there:
// rows at a fixed address, so the first loads do not wait for the position.
enum DmvPrologue { PRO_X = 0, PRO_RMS = 1, PRO_RES_RMS = 2, PRO_LN = 3, PRO_RES_LN = 4 };

// Prologue kinds: with the residual add, with layer_norm, with a norm.
constexpr bool pro_res(int pro) { return pro == PRO_RES_RMS || pro == PRO_RES_LN; }
constexpr bool pro_ln(int pro) { return pro == PRO_LN || pro == PRO_RES_LN; }
constexpr bool pro_norm(int pro) { return pro != PRO_X; }
// Epilogue: EPI_RAW writes the fp32 dot products; EPI_ARGMAX also writes the
// greedy token to tokens[pos + 1] (and *pos_out = pos + 1 when dpos is set);
// EPI_SWIGLU takes fused gate|up weights [2f, K] and writes
// m_out = Act(Act(silu(Act(g))) * Act(u)) ([f] Act row; raw, when set, gets
// the fp32 gate|up values).
enum DmvEpilogue { EPI_RAW = 0, EPI_ARGMAX = 1, EPI_SWIGLU = 2 };

struct DmvArgs {
    const uint32_t* wq = nullptr;  // weight codes, lane-permuted blocks
    const uint16_t* wd = nullptr;  // weight deltas
    int N = 0, nb = 0;             // weight rows, 32-value blocks per row (K = 32 nb)
    int rows = 0, ngroups = 0;     // rows per group and groups: set by the launcher
    int pos = 0;                   // the row's position, or *dpos when dpos is set
    const int* dpos = nullptr;
    const uint8_t* x = nullptr;    // PRO_X: the row; PRO_RMS: [positions, K] Act rows
    int x_pitch = 0;
    const float* raw_in = nullptr;      // PRO_RES_RMS: [K] fp32
    const uint8_t* res_in = nullptr;    // PRO_RES_RMS: [positions, K] Act rows
    uint8_t* res_out = nullptr;         // PRO_RES_RMS: [positions, K] Act rows (row pos written)
    int res_pitch = 0;
    const uint8_t* res_cur = nullptr;   // PRO_RES_RMS: the residual input row (else res_in at pos)
    uint8_t* res_cur_out = nullptr;     // PRO_RES_RMS: the residual sum also stored here (a fixed row)
    float bscale = 1.0f;                // PRO_RES_RMS: scale of the branch output (1: none)
    const uint16_t* norm_w = nullptr;   // norm gain (fp16)
    const uint16_t* norm_b = nullptr;   // PRO_LN / PRO_RES_LN bias (fp16)
    float post_scale = 1.0f;            // scale of the normalized row (1: none)
    float* raw = nullptr;               // fp32 dot products [N]
    uint8_t* m_out = nullptr;           // EPI_SWIGLU
    int32_t* tokens = nullptr;          // EPI_ARGMAX
    int* pos_out = nullptr;
    unsigned long long* amax = nullptr;  // EPI_ARGMAX scratch (kDmvArgmaxWords zeroed words, left zeroed)
    // EPI_ARGMAX: the next step's inputs, prepared by the workgroup that
    // finds the greedy token (when emb_codes is set): the token's embedding
    // row (token_embed, then * emb_scale as MiniCPM) to emb_cur and, when
    // pos + 1 < max_ctx, to row pos + 1 of emb_rows; RoPE row pos + 1 of
    // rope_table to rope_cur.
    const uint32_t* emb_codes = nullptr;
    const uint16_t* emb_deltas = nullptr;
    float emb_scale = 1.0f;
    uint8_t* emb_cur = nullptr;
    uint8_t* emb_rows = nullptr;
    int emb_pitch = 0;
    int max_ctx = 0;
    const float* rope_table = nullptr;  // [max_ctx][rope_half] (cos, sin) pairs
    float* rope_cur = nullptr;
    int rope_half = 0;
    // Nonzero: wq / wd are an lm head in the head layout (head_layout_launch);
    // only with PRO_RES_RMS and EPI_RAW / EPI_ARGMAX.
    int head = 0;
    // Speculative norm launches (set by decode_matvec from nc_debug_spec):
    // the factor on the predicted sum of squares (1: none) and a device
    // counter of the workgroups that recomputed blocks (null: none).
    float spec_skew = 1.0f;
    int* spec_fixups = nullptr;
};

// The lm-head copy of a Q4 / Q8 weight [N, K] read by the head kernel: rows
// in groups of 16, per group and 16-byte chunk each (row, lane)'s codes in
// (row, lane) order (one contiguous 1 KB load per wavefront), deltas per
// group and 8 blocks in row order.  Supported for the model widths K = 2048
// and 2304 and N >= 64.
bool head_layout_supported(int wdtype, int N, int K);
int head_layout_bytes(int wdtype, int N, int K, size_t* code_bytes, size_t* delta_bytes);
int head_layout_launch(const nc_tensor* w, void* codes, void* deltas, hipStream_t st);

constexpr int kDmvArgmaxWords = 320 + 4096;

// Whether decode_matvec takes this weight dtype, shape, prologue and
// epilogue (norm prologues need K % 256 == 0 and K <= 4096; the argmax and
// SwiGLU epilogues come with a norm prologue).
bool decode_matvec_supported(int wdtype, int K, int N, int pro, int epi);

// One fused launch on `st`; with events, the dispatch records them at the
// kernel's own start and end.
int decode_matvec(const DmvArgs& a, int wdtype, int pro, int epi, hipStream_t st, hipEvent_t ev0 = nullptr,
                  hipEvent_t ev1 = nullptr);

// After a token was written to tokens[*pos_out] by another kernel: that
// token's embedding and RoPE rows, as the argmax epilogue prepares them (the
// emb_* and rope_* fields, nb of the embedding rows, tokens, pos_out).
int next_inputs_launch(const DmvArgs& a, int wdtype, hipStream_t st);

}  // namespace nc
