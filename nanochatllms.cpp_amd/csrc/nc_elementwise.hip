// nc_elementwise.hip -- norms, RoPE, SiLU/multiply/add/scale/bias, token
// embedding, requantization and argmax for gfx950.
//
// Each kernel restates one gten op (gten/ops.cpp) including the write of its
// output in the activation dtype (write_row_from_float, gten/ops.cpp:87-123):
// Q8 rows are requantized per 32-value block (absmax / 127, fp16 delta,
// roundf) on the 32 lanes that hold the block.  The fused variants used by
// the decode step take the fp32 output of a matvec and first apply the
// requantization the reference's Linear::forward performs on it
// (gten/modules.cpp:89-104), so their results equal the unfused op chain.
#include <algorithm>
#include <cmath>
#include <vector>

#include "nc_act.h"
#include "nc_seqsum.h"
#include "nc_kernels.h"

namespace nc {

constexpr int kNormMaxPerThread = 16;
constexpr int kNormMaxCols = 4096;

// ---------------------------------------------------------------- requant --

// write_row_from_float of fp32 rows (matmul output) into activation rows.
template <int ADT>
__global__ __launch_bounds__(256) void k_write_rows(const float* __restrict__ in, int in_pitch, uint8_t* __restrict__ out,
                                                   int out_pitch, int cols)
{
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int r = blockIdx.y;
    const bool valid = e < cols;
    const float v = valid ? in[(size_t)r * in_pitch + e] : 0.0f;
    act_store<ADT>(out + (size_t)r * out_pitch, e, act_delta_offset(cols), v, valid);
}

// ------------------------------------------------------------------ norms --

enum NormKind { kRms = 0, kLayerNorm = 1 };

// One workgroup per normalized segment (a row, or one head of a row).
// Input: the activation row a, or (ADD) the residual sum a + b where b is a
// matvec's fp32 output requantized as the Linear output (optionally scaled
// and requantized again, MiniCPM's ops::scale).  The sum is stored to h_out
// in the activation dtype and normalized from that stored value.
//   RMS: rms_norm_vec_f32 (gten/ops.cpp:830-846): sequential sum of squares,
//        rms = sqrtf(ss / n), y = x / (rms + 1e-6f) * w.
//   LN : vec_layer_norm_f32 (gten/ops.cpp:669-698): sequential mean and
//        variance, y = ((x - mean) / (sqrtf(var) + 1e-5f)) * w + b.
// post_scale != 1 applies ops::scale to the stored result (MiniCPM).
// Up to 1024 threads share the elementwise work; the sequential sums run on
// wavefront 0 alone while the others wait at the barrier.
template <int ADT, int KIND, bool ADD>
__global__ __launch_bounds__(1024) void k_norm(const uint8_t* __restrict__ a, int a_pitch,
                                               const float* __restrict__ braw, int b_pitch, float bscale,
                                               uint8_t* __restrict__ h_out, int h_pitch,
                                               const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias,
                                               uint8_t* __restrict__ out, int out_pitch, int n, int row_cols,
                                               float post_scale, const int* __restrict__ dpos)
{
    __shared__ __align__(16) float buf[kNormMaxCols];
    __shared__ float stat[2];
    __shared__ SsShared ssh;
    __shared__ SgShared sgh;
    const int tid = threadIdx.x;
    const int bs = blockDim.x;
    // a workgroup of 256 threads or more over a multiple of 256 values: the
    // non-negative sums (rms_norm's squares, layer_norm's squared
    // deviations) run as the workgroup-parallel restatement of the
    // sequential loop (same result) on the first 256 threads
    const bool block_sum = bs % kSsThreads == 0 && n % kSsThreads == 0;
    const int per = n / bs;
    const int r = blockIdx.y;
    const int seg0 = blockIdx.x * n;  // first column of this segment in the row
    const int dofs = act_delta_offset(row_cols);
    // under graph replay the input / stored-sum rows sit at the device-held position
    const size_t prow = dpos ? (size_t)dpos[0] : (size_t)r;
    const uint8_t* arow = a + prow * a_pitch;
    uint8_t* orow = out + (size_t)r * out_pitch;

    float xv[kNormMaxPerThread];
#pragma unroll
    for (int m = 0; m < kNormMaxPerThread; m++) {
        if (m >= per) continue;
        const int e = seg0 + tid + m * bs;
        float x = act_load<ADT>(arow, e, dofs);
        if (ADD) {
            float b = act_roundtrip<ADT>(braw[(size_t)r * b_pitch + e], true);
            if (bscale != 1.0f) b = act_roundtrip<ADT>(b * bscale, true);
            const float s = x + b;
            x = act_roundtrip<ADT>(s, true);
            act_store<ADT>(h_out + prow * h_pitch, e, dofs, s, true);
        }
        xv[m] = x;
        buf[tid + m * bs] = KIND == kRms ? x * x : x;
    }
    __syncthreads();
    if (KIND == kLayerNorm && bs == 1024 && n == 2 * 1024) {
        // the mean of a decode row (Zephyr's final norm): the exact
        // workgroup sum of the fp16-grid values
        const float s1 = block_seq_sum_grid<2, 1024>(buf, sgh);
        if (tid == 0) stat[0] = s1 / (float)n;
    } else if (KIND == kRms && block_sum) {
        const float s1 = block_seq_sum_nonneg(buf, n, ssh);
        if (tid == 0) {
            stat[0] = 0.0f;
            stat[1] = sqrtf(s1 / (float)n) + 1e-6f;  // rms + eps
        }
    } else if (tid < kWave) {
        const float s1 = seq_sum(buf, n);
        if (tid == 0) {
            stat[0] = KIND == kLayerNorm ? s1 / (float)n : 0.0f;
            stat[1] = sqrtf(s1 / (float)n) + 1e-6f;  // RMS: rms + eps
        }
    }
    __syncthreads();
    if (KIND == kLayerNorm) {
        const float mu = stat[0];
#pragma unroll
        for (int m = 0; m < kNormMaxPerThread; m++) {
            if (m >= per) continue;
            buf[tid + m * bs] = (xv[m] - mu) * (xv[m] - mu);
        }
        __syncthreads();
        if (block_sum) {
            const float ssq = block_seq_sum_nonneg(buf, n, ssh);
            if (tid == 0) stat[1] = sqrtf(ssq / (float)n) + 1e-05f;
        } else if (tid < kWave) {
            const float ssq = seq_sum(buf, n);
            if (tid == 0) stat[1] = sqrtf(ssq / (float)n) + 1e-05f;
        }
    }
    __syncthreads();
    const float mean = stat[0], denom = stat[1];
#pragma unroll
    for (int m = 0; m < kNormMaxPerThread; m++) {
        if (m >= per) continue;
        const int i = tid + m * bs;  // index within the segment (weight index)
        float y;
        if (KIND == kRms) y = xv[m] / denom * h2f(w[i]);
        else y = ((xv[m] - mean) / denom) * h2f(w[i]) + h2f(bias[i]);
        if (post_scale != 1.0f) y = act_roundtrip<ADT>(y, true) * post_scale;
        act_store<ADT>(orow, seg0 + i, dofs, y, true);
    }
}

// ------------------------------------------------------------------- rope --

// rotary_emb (gten/ops.cpp:775-821) on stored activation rows: one
// wavefront per 64-wide head; row r has position start + blockIdx.y.
template <int ADT>
__global__ __launch_bounds__(64) void k_rope(const uint8_t* __restrict__ in, int in_pitch, uint8_t* __restrict__ out,
                                             int out_pitch, int cols, const float2* __restrict__ table, int d_half,
                                             int start)
{
    const int lane = threadIdx.x;
    const int r = blockIdx.y;
    const int e = blockIdx.x * 64 + lane;
    const int dofs = act_delta_offset(cols);
    const float x = act_load<ADT>(in + (size_t)r * in_pitch, e, dofs);
    const float y = rope_lane(x, lane, d_half, table + (size_t)(start + r) * d_half);
    act_store<ADT>(out + (size_t)r * out_pitch, e, dofs, y, true);
}

// Decode-step epilogue of the fused q|k|v matvec: per 64-wide head segment
// of the fp32 output [q heads | k heads | v heads]:
//   Linear output requantized (+ fp16 bias, requantized: bias_add_inplace),
//   q/k: optional per-head RMSNorm (OpenELM's QK norm, requantized), RoPE at
//   the row's position (requantized); q -> q_out, k -> K cache row,
//   v -> V cache row.
template <int ADT, bool BIAS, bool QKNORM>
__global__ __launch_bounds__(64) void k_qkv_post(const float* __restrict__ raw, int raw_pitch, int hq, int hkv,
                                                 const uint16_t* __restrict__ bq, const uint16_t* __restrict__ bk,
                                                 const uint16_t* __restrict__ bv, const uint16_t* __restrict__ qn_w,
                                                 const uint16_t* __restrict__ kn_w, const float2* __restrict__ table,
                                                 int d_half, int start, uint8_t* __restrict__ q_out, int q_pitch,
                                                 uint8_t* __restrict__ k_cache, int k_pitch,
                                                 uint8_t* __restrict__ v_cache, int v_pitch, const int* __restrict__ dpos)
{
    __shared__ __align__(16) float buf[64];
    const int lane = threadIdx.x;
    const int seg = blockIdx.x;
    const int r = blockIdx.y;
    const int pos = (dpos ? dpos[0] : start) + r;
    const int kind = seg < hq ? 0 : (seg < hq + hkv ? 1 : 2);
    const int h = kind == 0 ? seg : (kind == 1 ? seg - hq : seg - hq - hkv);
    float x = act_roundtrip<ADT>(raw[(size_t)r * raw_pitch + seg * 64 + lane], true);
    if (BIAS) {
        const uint16_t* b = kind == 0 ? bq : (kind == 1 ? bk : bv);
        x = act_roundtrip<ADT>(x + h2f(b[h * 64 + lane]), true);
    }
    if (kind < 2) {
        if (QKNORM) {
            buf[lane] = x * x;
            __syncthreads();
            const float rms = sqrtf(seq_sum(buf, 64) / 64.0f);
            x = act_roundtrip<ADT>(x / (rms + 1e-6f) * h2f((kind == 0 ? qn_w : kn_w)[lane]), true);
        }
        x = rope_lane(x, lane, d_half, table + (size_t)pos * d_half);
    }
    uint8_t* dst;
    int cols;
    if (kind == 0) { dst = q_out + (size_t)r * q_pitch; cols = hq * 64; }
    else if (kind == 1) { dst = k_cache + (size_t)pos * k_pitch; cols = hkv * 64; }
    else { dst = v_cache + (size_t)pos * v_pitch; cols = hkv * 64; }
    act_store<ADT>(dst, h * 64 + lane, act_delta_offset(cols), x, true);
}

// ------------------------------------------------------------ elementwise --

enum EwOp { kSilu = 0, kMul = 1, kAdd = 2, kScale = 3, kBias = 4 };

// silu_impl / mul_impl / add_impl / scale / bias_add_inplace
// (gten/ops.cpp:733-757, 918-1014, 146-164, 639-666) on activation rows.
template <int ADT, int OP>
__global__ __launch_bounds__(256) void k_ew(const uint8_t* __restrict__ a, int a_pitch, const uint8_t* __restrict__ b,
                                            int b_pitch, const uint16_t* __restrict__ bias, float s,
                                            uint8_t* __restrict__ out, int out_pitch, int cols)
{
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int r = blockIdx.y;
    const bool valid = e < cols;
    const int dofs = act_delta_offset(cols);
    const int ec = valid ? e : 0;
    const float x = act_load<ADT>(a + (size_t)r * a_pitch, ec, dofs);
    float y;
    if (OP == kSilu) y = x / (1.0f + expf_ref(-x));
    else if (OP == kMul) y = x * act_load<ADT>(b + (size_t)r * b_pitch, ec, dofs);
    else if (OP == kAdd) y = x + act_load<ADT>(b + (size_t)r * b_pitch, ec, dofs);
    else if (OP == kScale) y = x * s;
    else y = x + h2f(bias[ec]);
    act_store<ADT>(out + (size_t)r * out_pitch, e, dofs, y, valid);
}

// Decode-step SwiGLU from the fused gate|up matvec output [gate | up]:
// gate and up requantized as Linear outputs, SiLU in place (requantized),
// multiply in place (requantized) -- ffn_forward, tinyllama/tinyllama.cpp:88-97.
template <int ADT>
__global__ __launch_bounds__(256) void k_silu_mul(const float* __restrict__ raw, int raw_pitch, int f,
                                                  uint8_t* __restrict__ out, int out_pitch)
{
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int r = blockIdx.y;
    const bool valid = e < f;
    const int ec = valid ? e : 0;
    const float* rr = raw + (size_t)r * raw_pitch;
    const float g = act_roundtrip<ADT>(rr[ec], valid);
    const float gs = act_roundtrip<ADT>(g / (1.0f + expf_ref(-g)), valid);
    const float u = act_roundtrip<ADT>(rr[f + ec], valid);
    act_store<ADT>(out + (size_t)r * out_pitch, e, act_delta_offset(f), gs * u, valid);
}

// -------------------------------------------------------------- embedding --

// token_embed / copy_row (gten/ops.cpp:526-576): Q8 and F16 rows copied,
// Q4 rows dequantized and requantized to Q8.  post_scale != 1 applies
// ops::scale afterwards (MiniCPM's embedding scale).
template <int WDT, int ADT>
__global__ __launch_bounds__(256) void k_embed(const uint32_t* __restrict__ codes, const uint16_t* __restrict__ deltas,
                                               int vocab, const int32_t* __restrict__ tokens, uint8_t* __restrict__ out,
                                               int out_pitch, int d, float post_scale, const int* __restrict__ dpos,
                                               uint8_t* __restrict__ out_cur)
{
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int r = dpos ? dpos[0] : (int)blockIdx.y;  // row of tokens / out
    const bool valid = e < d;
    const int ec = valid ? e : 0;
    int tok = tokens[r];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    uint8_t* orow = out + (size_t)r * out_pitch;
    const int dofs = act_delta_offset(d);
    const int nb = d / 32;
    float v;
    if (WDT == Q4 || WDT == Q8) {
        const size_t blk = (size_t)tok * nb + (ec >> 5);
        const float dw = h2f(deltas[blk]);
        if (WDT == Q8) {
            const int q = q8_weight_code(codes + blk * 8, ec & 31);
            if (post_scale == 1.0f) {
                if (valid) {
                    reinterpret_cast<int8_t*>(orow)[e] = (int8_t)q;
                    if ((e & 31) == 0) reinterpret_cast<uint16_t*>(orow + dofs)[e >> 5] = deltas[blk];
                    if (out_cur) {
                        reinterpret_cast<int8_t*>(out_cur)[e] = (int8_t)q;
                        if ((e & 31) == 0) reinterpret_cast<uint16_t*>(out_cur + dofs)[e >> 5] = deltas[blk];
                    }
                }
                return;
            }
            v = (float)q * dw;
        } else {
            v = (float)(q4_weight_code(codes + blk * 4, ec & 31) - 7) * dw;
        }
    } else {
        const int npad = (vocab + 7) & ~7;
        v = h2f(reinterpret_cast<const uint16_t*>(codes)[f16_weight_index(tok, ec, npad)]);
    }
    if (post_scale != 1.0f) v = act_roundtrip<ADT>(v, valid) * post_scale;
    act_store<ADT>(orow, e, dofs, v, valid);
    if (out_cur) act_store<ADT>(out_cur, e, dofs, v, valid);
}

// ----------------------------------------------------------------- argmax --

// First index of the maximum (strict '>' scan of gten/sampler.cpp:33-41).
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n, int32_t* __restrict__ out)
{
    __shared__ float sv[1024];
    __shared__ int si[1024];
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = tid; i < n; i += 1024) {
        const float v = x[i];
        if (v > best) { best = v; bi = i; }
    }
    sv[tid] = best;
    si[tid] = bi;
    __syncthreads();
    for (int s = 512; s > 0; s >>= 1) {
        if (tid < s) {
            const float v = sv[tid + s];
            const int i = si[tid + s];
            if (v > sv[tid] || (v == sv[tid] && i < si[tid])) { sv[tid] = v; si[tid] = i; }
        }
        __syncthreads();
    }
    if (tid == 0) out[0] = si[0] == 0x7fffffff ? 0 : si[0];
}

// Greedy step epilogue for graph replay: every workgroup reduces a slice of
// x to (value, first index), folded across workgroups with a 64-bit
// atomicMax on greedy_key (the index greedy_sample's scan takes).  The last
// workgroup to finish writes the token to tokens[pos + 1], advances pos and
// re-zeroes the scratch words for the next replay.
__global__ __launch_bounds__(256) void k_argmax_advance(const float* __restrict__ x, int n, int32_t* __restrict__ tokens,
                                                        int* __restrict__ dpos, unsigned long long* __restrict__ scratch)
{
    __shared__ unsigned long long sk[256];
    const int tid = threadIdx.x;
    unsigned long long best = 0;
    for (int i = blockIdx.x * 256 + tid; i < n; i += gridDim.x * 256) {
        const unsigned long long key = greedy_key(x[i], i);
        best = key > best ? key : best;
    }
    sk[tid] = best;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s && sk[tid + s] > sk[tid]) sk[tid] = sk[tid + s];
        __syncthreads();
    }
    if (tid == 0) {
        atomicMax(&scratch[0], sk[0]);
        __threadfence();
        const unsigned long long ticket = atomicAdd(&scratch[1], 1ull);
        if (ticket == gridDim.x - 1) {
            const unsigned long long key = atomicOr(&scratch[0], 0ull);
            const int pos = dpos[0];
            tokens[pos + 1] = (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
            dpos[0] = pos + 1;
            atomicExch(&scratch[0], 0ull);
            atomicExch(&scratch[1], 0ull);
        }
    }
}

// ============================================================ launchers ==

#define NC_ADT_DISPATCH(adt, KERNEL_CALL)                              \
    do {                                                               \
        if ((adt) == NC_Q8) { constexpr int ADT = Q8; KERNEL_CALL; }    \
        else if ((adt) == NC_F16) { constexpr int ADT = F16; KERNEL_CALL; } \
        else { constexpr int ADT = F32; KERNEL_CALL; }                 \
    } while (0)

int write_rows(const float* in, int in_pitch, uint8_t* out, int out_pitch, int dtype, int cols, int rows,
               hipStream_t st)
{
    if (rows <= 0) return NC_OK;
    const dim3 grid((cols + 255) / 256, rows);
    NC_ADT_DISPATCH(dtype, hipLaunchKernelGGL((k_write_rows<ADT>), grid, dim3(256), 0, st, in, in_pitch, out,
                                              out_pitch, cols));
    return launch_status("k_write_rows");
}

// Threads per norm workgroup: the largest multiple of 64 up to 1024 that
// divides the segment (each thread then owns n / bs values).
static int norm_block(int n)
{
    for (int bs = 1024; bs >= 64; bs -= 64)
        if (n % bs == 0) return bs;
    return n;
}

int norm_launch(int kind, int adt, bool add, const uint8_t* a, int a_pitch, const float* braw, int b_pitch,
                float bscale, uint8_t* h_out, int h_pitch, const uint16_t* w, const uint16_t* bias, uint8_t* out,
                int out_pitch, int d_norm, int row_cols, int rows, float post_scale, hipStream_t st, const int* dpos)
{
    if (rows <= 0) return NC_OK;
    const int bs = norm_block(d_norm);
    if (d_norm % 32 || row_cols % d_norm || d_norm % bs || d_norm / bs > kNormMaxPerThread || d_norm > kNormMaxCols)
        return fail(NC_ERR_ARG, "norm: unsupported size %d (row %d)", d_norm, row_cols);
    if (adt != NC_Q8 && adt != NC_F16) return fail(NC_ERR_ARG, "norm: activation dtype %d", adt);
    const dim3 grid(row_cols / d_norm, rows);
#define NORM_CALL(K, A)                                                                                           \
    hipLaunchKernelGGL((k_norm<ADT, K, A>), grid, dim3(bs), 0, st, a, a_pitch, braw, b_pitch, bscale, h_out, h_pitch, \
                       w, bias, out, out_pitch, d_norm, row_cols, post_scale, dpos)
    if (adt == NC_Q8) {
        constexpr int ADT = Q8;
        if (kind == kRms) { if (add) NORM_CALL(kRms, true); else NORM_CALL(kRms, false); }
        else { if (add) NORM_CALL(kLayerNorm, true); else NORM_CALL(kLayerNorm, false); }
    } else {
        constexpr int ADT = F16;
        if (kind == kRms) { if (add) NORM_CALL(kRms, true); else NORM_CALL(kRms, false); }
        else { if (add) NORM_CALL(kLayerNorm, true); else NORM_CALL(kLayerNorm, false); }
    }
#undef NORM_CALL
    return launch_status("k_norm");
}

int qkv_post_launch(int adt, const float* raw, int raw_pitch, int hq, int hkv, const uint16_t* bq, const uint16_t* bk,
                    const uint16_t* bv, const uint16_t* qn_w, const uint16_t* kn_w, const float* table, int d_half,
                    int start, int rows, uint8_t* q_out, int q_pitch, uint8_t* k_cache, int k_pitch,
                    uint8_t* v_cache, int v_pitch, hipStream_t st, const int* dpos)
{
    if (rows <= 0) return NC_OK;
    const dim3 grid(hq + 2 * hkv, rows);
    const bool bias = bq != nullptr, qkn = qn_w != nullptr;
#define QKV_CALL(B, N)                                                                                              \
    hipLaunchKernelGGL((k_qkv_post<ADT, B, N>), grid, dim3(64), 0, st, raw, raw_pitch, hq, hkv, bq, bk, bv, qn_w, kn_w, \
                       (const float2*)table, d_half, start, q_out, q_pitch, k_cache, k_pitch, v_cache, v_pitch, dpos)
    if (adt == NC_Q8) {
        constexpr int ADT = Q8;
        if (bias) { if (qkn) QKV_CALL(true, true); else QKV_CALL(true, false); }
        else { if (qkn) QKV_CALL(false, true); else QKV_CALL(false, false); }
    } else if (adt == NC_F16) {
        constexpr int ADT = F16;
        if (bias) { if (qkn) QKV_CALL(true, true); else QKV_CALL(true, false); }
        else { if (qkn) QKV_CALL(false, true); else QKV_CALL(false, false); }
    } else {
        return fail(NC_ERR_ARG, "qkv_post: activation dtype %d", adt);
    }
#undef QKV_CALL
    return launch_status("k_qkv_post");
}

int silu_mul_launch(int adt, const float* raw, int raw_pitch, int f, uint8_t* out, int out_pitch, int rows,
                    hipStream_t st)
{
    if (rows <= 0) return NC_OK;
    const dim3 grid((f + 255) / 256, rows);
    if (adt == NC_Q8) hipLaunchKernelGGL((k_silu_mul<Q8>), grid, dim3(256), 0, st, raw, raw_pitch, f, out, out_pitch);
    else if (adt == NC_F16) hipLaunchKernelGGL((k_silu_mul<F16>), grid, dim3(256), 0, st, raw, raw_pitch, f, out, out_pitch);
    else return fail(NC_ERR_ARG, "silu_mul: activation dtype %d", adt);
    return launch_status("k_silu_mul");
}

int embed_launch(const nc_tensor* table, const int32_t* tokens, uint8_t* out, int out_pitch, int adt, int rows,
                 float post_scale, hipStream_t st, const int* dpos, uint8_t* out_cur)
{
    if (rows <= 0) return NC_OK;
    const int d = table->cols;
    const dim3 grid((d + 255) / 256, rows);
    const uint32_t* c = (const uint32_t*)table->data;
    const uint16_t* dl = (const uint16_t*)table->deltas;
    if (table->dtype == NC_Q4 && adt == NC_Q8)
        hipLaunchKernelGGL((k_embed<Q4, Q8>), grid, dim3(256), 0, st, c, dl, table->rows, tokens, out, out_pitch, d, post_scale,
                           dpos, out_cur);
    else if (table->dtype == NC_Q8 && adt == NC_Q8)
        hipLaunchKernelGGL((k_embed<Q8, Q8>), grid, dim3(256), 0, st, c, dl, table->rows, tokens, out, out_pitch, d, post_scale,
                           dpos, out_cur);
    else if (table->dtype == NC_F16 && adt == NC_F16)
        hipLaunchKernelGGL((k_embed<F16, F16>), grid, dim3(256), 0, st, c, dl, table->rows, tokens, out, out_pitch, d, post_scale,
                           dpos, out_cur);
    else
        return fail(NC_ERR_ARG, "token_embed: table dtype %d with activation dtype %d", table->dtype, adt);
    return launch_status("k_embed");
}

int argmax_launch(const float* x, int n, int32_t* out, hipStream_t st)
{
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, st, x, n, out);
    return launch_status("k_argmax");
}

int argmax_advance_launch(const float* x, int n, int32_t* tokens, int* dpos, unsigned long long* scratch,
                          hipStream_t st)
{
    const int grid = std::min(64, (n + 255) / 256);
    hipLaunchKernelGGL(k_argmax_advance, dim3(grid), dim3(256), 0, st, x, n, tokens, dpos, scratch);
    return launch_status("k_argmax_advance");
}

int ew_launch(int op, int adt, const uint8_t* a, int a_pitch, const uint8_t* b, int b_pitch, const uint16_t* bias,
              float s, uint8_t* out, int out_pitch, int cols, int rows, hipStream_t st)
{
    if (rows <= 0) return NC_OK;
    const dim3 grid((cols + 255) / 256, rows);
#define EW_CALL(OPV) hipLaunchKernelGGL((k_ew<ADT, OPV>), grid, dim3(256), 0, st, a, a_pitch, b, b_pitch, bias, s, out, out_pitch, cols)
    NC_ADT_DISPATCH(adt, {
        switch (op) {
        case kSilu: EW_CALL(kSilu); break;
        case kMul: EW_CALL(kMul); break;
        case kAdd: EW_CALL(kAdd); break;
        case kScale: EW_CALL(kScale); break;
        default: EW_CALL(kBias); break;
        }
    });
#undef EW_CALL
    return launch_status("k_ew");
}

int rope_launch(int adt, const uint8_t* in, int in_pitch, uint8_t* out, int out_pitch, int cols, const float* table,
                int d_half, int start, int rows, hipStream_t st)
{
    if (rows <= 0) return NC_OK;
    if (cols % 64) return fail(NC_ERR_ARG, "rotary_emb: width %d is not a multiple of the 64-wide head", cols);
    const dim3 grid(cols / 64, rows);
    NC_ADT_DISPATCH(adt, hipLaunchKernelGGL((k_rope<ADT>), grid, dim3(64), 0, st, in, in_pitch, out, out_pitch, cols,
                                            (const float2*)table, d_half, start));
    return launch_status("k_rope");
}

}  // namespace nc

// ================================================================ C-ABI ==

using namespace nc;

static bool act_ok(const nc_tensor* t) { return t && t->data && is_act(t->dtype); }

static uint8_t* row_ptr(const nc_tensor* t, int r) { return (uint8_t*)t->data + (size_t)r * t->pitch; }

extern "C" {

int nc_rms_norm(const nc_tensor* x, const uint16_t* w, nc_tensor* out, int d_norm, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(act_ok(x) && act_ok(out) && w, "rms_norm: bad tensor");
    NC_CHECK_ARG(x->dtype == out->dtype && x->cols == out->cols, "rms_norm: shape/dtype mismatch");
    NC_CHECK_ARG(start >= 0 && n_ctx <= x->rows && n_ctx <= out->rows, "rms_norm: rows [%d, %d)", start, n_ctx);
    return norm_launch(kRms, x->dtype, false, row_ptr(x, start), x->pitch, nullptr, 0, 1.0f, nullptr, 0, w, nullptr,
                       row_ptr(out, start), out->pitch, d_norm, x->cols, n_ctx - start, 1.0f, stream_of(stream), nullptr);
}

int nc_layer_norm(const nc_tensor* x, const uint16_t* w, const uint16_t* b, nc_tensor* out, int start, int n_ctx,
                  void* stream)
{
    NC_CHECK_ARG(act_ok(x) && act_ok(out) && w && b, "layer_norm: bad tensor");
    NC_CHECK_ARG(x->dtype == out->dtype && x->cols == out->cols, "layer_norm: shape/dtype mismatch");
    NC_CHECK_ARG(start >= 0 && n_ctx <= x->rows && n_ctx <= out->rows, "layer_norm: rows [%d, %d)", start, n_ctx);
    return norm_launch(kLayerNorm, x->dtype, false, row_ptr(x, start), x->pitch, nullptr, 0, 1.0f, nullptr, 0, w, b,
                       row_ptr(out, start), out->pitch, x->cols, x->cols, n_ctx - start, 1.0f, stream_of(stream), nullptr);
}

int nc_rope_table(int max_ctx, int d_head, float rope_pct, float* out)
{
    NC_CHECK_ARG(out && max_ctx > 0 && d_head > 0, "rope_table: bad arguments");
    const int rope_d = static_cast<int>((float)d_head * rope_pct);
    const int d_half = rope_d / 2;
    const float d = static_cast<float>(rope_d);
    for (int i = 0; i < max_ctx; i++) {
        const float m = static_cast<float>(i);
        for (int j = 0; j < d_half; j++) {
            const float th = m * std::pow(10000.0f, -(2.0f * j / d));
            out[2 * ((size_t)i * d_half + j)] = std::cos(th);
            out[2 * ((size_t)i * d_half + j) + 1] = std::sin(th);
        }
    }
    return NC_OK;
}

int nc_rotary_emb(const nc_tensor* x, nc_tensor* out, int d_head, float rope_pct, const float* table, int start,
                  int n_ctx, void* stream)
{
    NC_CHECK_ARG(act_ok(x) && act_ok(out) && table, "rotary_emb: bad tensor");
    NC_CHECK_ARG(d_head == 64, "rotary_emb: head size %d (the kernels are built for 64)", d_head);
    NC_CHECK_ARG(x->dtype == out->dtype && x->cols == out->cols, "rotary_emb: shape/dtype mismatch");
    NC_CHECK_ARG(start >= 0 && n_ctx <= x->rows && n_ctx <= out->rows, "rotary_emb: rows [%d, %d)", start, n_ctx);
    const int d_half = static_cast<int>((float)d_head * rope_pct) / 2;
    return rope_launch(x->dtype, row_ptr(x, start), x->pitch, row_ptr(out, start), out->pitch, x->cols, table, d_half,
                       start, n_ctx - start, stream_of(stream));
}

static int ew_api(int op, const nc_tensor* a, const nc_tensor* b, const uint16_t* bias, float s, nc_tensor* out,
                  int start, int n_ctx, void* stream, const char* name)
{
    NC_CHECK_ARG(act_ok(a) && act_ok(out), "%s: bad tensor", name);
    NC_CHECK_ARG(a->dtype == out->dtype && a->cols == out->cols, "%s: shape/dtype mismatch", name);
    if (b) NC_CHECK_ARG(act_ok(b) && b->dtype == a->dtype && b->cols == a->cols, "%s: operand mismatch", name);
    NC_CHECK_ARG(start >= 0 && n_ctx <= a->rows && n_ctx <= out->rows, "%s: rows [%d, %d)", name, start, n_ctx);
    return ew_launch(op, a->dtype, row_ptr(a, start), a->pitch, b ? row_ptr(b, start) : nullptr, b ? b->pitch : 0,
                     bias, s, row_ptr(out, start), out->pitch, a->cols, n_ctx - start, stream_of(stream));
}

int nc_silu(const nc_tensor* x, nc_tensor* out, int start, int n_ctx, void* stream)
{
    return ew_api(kSilu, x, nullptr, nullptr, 0.0f, out, start, n_ctx, stream, "silu");
}

int nc_multiply(const nc_tensor* a, const nc_tensor* b, nc_tensor* out, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(b, "multiply: null operand");
    return ew_api(kMul, a, b, nullptr, 0.0f, out, start, n_ctx, stream, "multiply");
}

int nc_add(const nc_tensor* a, const nc_tensor* b, nc_tensor* out, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(b, "add: null operand");
    return ew_api(kAdd, a, b, nullptr, 0.0f, out, start, n_ctx, stream, "add");
}

int nc_scale(nc_tensor* x, float s, int start, int n_ctx, void* stream)
{
    return ew_api(kScale, x, nullptr, nullptr, s, x, start, n_ctx, stream, "scale");
}

int nc_bias_add(nc_tensor* x, const uint16_t* b, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(b, "bias_add: null bias");
    return ew_api(kBias, x, nullptr, b, 0.0f, x, start, n_ctx, stream, "bias_add");
}

int nc_token_embed(const nc_tensor* table, const int32_t* tokens, nc_tensor* out, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(table && table->data && tokens && act_ok(out), "token_embed: bad tensor");
    NC_CHECK_ARG(table->cols == out->cols, "token_embed: width mismatch");
    NC_CHECK_ARG(start >= 0 && n_ctx <= out->rows, "token_embed: rows [%d, %d)", start, n_ctx);
    return embed_launch(table, tokens + start, row_ptr(out, start), out->pitch, out->dtype, n_ctx - start, 1.0f,
                        stream_of(stream), nullptr);
}

int nc_argmax(const float* x, int n, int32_t* out, void* stream)
{
    NC_CHECK_ARG(x && out && n > 0, "argmax: bad arguments");
    return argmax_launch(x, n, out, stream_of(stream));
}

}  // extern "C"

namespace nc {
// One vector of n terms per workgroup through the block sum.
__global__ __launch_bounds__(kSsThreads) void k_block_seq_sum(const float* __restrict__ t, int n, float* __restrict__ out,
                                                             int* __restrict__ fast)
{
    extern __shared__ __align__(16) float buf[];
    __shared__ SsShared sh;
    const float* tv = t + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += kSsThreads) buf[i] = tv[i];
    __syncthreads();
    bool f = false;
    const float s = block_seq_sum_nonneg(buf, n, sh, &f);
    if (threadIdx.x == 0) {
        out[blockIdx.x] = s;
        fast[blockIdx.x] = f;
    }
}

// One row of n values per workgroup through the fp16-grid sum (4 values per
// thread).
template <int NT>
__global__ __launch_bounds__(NT) void k_block_seq_sum_grid(const float* __restrict__ x, float* __restrict__ out,
                                                           int* __restrict__ passes)
{
    constexpr int n = 4 * NT;
    __shared__ __align__(16) float buf[n];
    __shared__ SgShared sh;
    const float* xv = x + (size_t)blockIdx.x * n;
    for (int i = threadIdx.x; i < n; i += NT) buf[i] = xv[i];
    __syncthreads();
    int np = 0;
    const float s = block_seq_sum_grid<4, NT>(buf, sh, &np);
    if (threadIdx.x == 0) {
        out[blockIdx.x] = s;
        passes[blockIdx.x] = np;
    }
}

__global__ void k_expf(const float* __restrict__ x, float* __restrict__ y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = expf_ref(x[i]);
}
}  // namespace nc

// The kernels' expf evaluated on the host (the same source), so the
// algorithm can be checked against the host libm without a GPU.
extern "C" float nc_expf_host(float x) { return nc::expf_ref(x); }

// The sequential sum of non-negative terms (gten/ops.cpp:833-835) as the
// fused norm prologues compute it, over `count` vectors of n terms.
extern "C" int nc_block_seq_sum(const float* t, int n, int count, float* out, int* fast, void* stream)
{
    NC_CHECK_ARG(t && out && fast && count >= 0, "block_seq_sum: bad arguments");
    NC_CHECK_ARG(n > 0 && n % nc::kSsThreads == 0 && n <= nc::kSsThreads * nc::kSsMaxPer,
                 "block_seq_sum: n=%d (a multiple of %d up to %d)", n, nc::kSsThreads, nc::kSsThreads * nc::kSsMaxPer);
    if (!count) return NC_OK;
    hipLaunchKernelGGL(nc::k_block_seq_sum, dim3(count), dim3(nc::kSsThreads), (size_t)n * 4, stream_of(stream), t, n,
                       out, fast);
    return launch_status("k_block_seq_sum");
}

// The sequential sum of signed values on the fp16 grid (gten/ops.cpp:673-676)
// as the fused layer-norm prologues compute it, over `count` rows of n =
// 1024, 2048 or 2304 values; passes[b] = the parallel passes made (0: the
// plain loop ran).
extern "C" int nc_block_seq_sum_grid(const float* x, int n, int count, float* out, int* passes, void* stream)
{
    NC_CHECK_ARG(x && out && passes && count >= 0, "block_seq_sum_grid: bad arguments");
    NC_CHECK_ARG(n == 1024 || n == 2048 || n == 2304, "block_seq_sum_grid: n=%d (1024, 2048 or 2304)", n);
    if (!count) return NC_OK;
    hipStream_t st = stream_of(stream);
    if (n == 1024)
        hipLaunchKernelGGL(nc::k_block_seq_sum_grid<256>, dim3(count), dim3(256), 0, st, x, out, passes);
    else if (n == 2048)
        hipLaunchKernelGGL(nc::k_block_seq_sum_grid<512>, dim3(count), dim3(512), 0, st, x, out, passes);
    else
        hipLaunchKernelGGL(nc::k_block_seq_sum_grid<576>, dim3(count), dim3(576), 0, st, x, out, passes);
    return launch_status("k_block_seq_sum_grid");
}

// The fp16-grid decomposition on the host: exact double prefixes, then from
// each rounding step the next one found by a pass over the later steps.
// plant = 1 plants a mistake (the error after a rounding step is dropped),
// for tests that must catch it.
extern "C" float nc_seq_sum_grid_host(const float* x, int n, int plant, int* passes)
{
    std::vector<double> P(n + 1, 0.0);
    bool ok = true;
    for (int i = 0; i < n; i++) {
        ok = ok && nc::sg_on_grid(x[i]);
        P[i + 1] = P[i] + (double)x[i];
    }
    int np = 0;
    if (ok) {
        double e = 0.0;
        int r = 0;
        while (np < nc::kSgMaxPass) {
            np++;
            int f = n;
            for (int i = r; i < n; i++) {
                const double v = P[i + 1] + e;
                if ((double)(float)v != v) {
                    f = i;
                    break;
                }
            }
            if (f == n) {
                *passes = np;
                return (float)(P[n] + e);
            }
            const float si = (float)(P[f] + e);
            const float sn = si + x[f];
            e = plant ? 0.0 : (double)sn - P[f + 1];
            r = f + 1;
        }
    }
    float s = 0.0f;
    for (int i = 0; i < n; i++) s = s + x[i];
    *passes = 0;
    return s;
}

// The same segment / crossing decomposition run on the host with the
// kernels' representatives, composition and check functions, the binades
// predicted from a double-precision prefix scaled by (1 + skew), and each
// run's representatives started from that prediction: a skew makes
// predictions wrong on purpose, which the checks must catch (the result
// stays the sequential sum; *fast says whether the checks passed).
extern "C" float nc_seq_sum_nonneg_host(const float* t, int n, double skew, int* fast)
{
    using namespace nc;
    auto bits = [](float v) { return __builtin_bit_cast(int, v); };
    auto flt = [](int b) { return __builtin_bit_cast(float, b); };
    double P = 0.0;
    float pred = (float)(P * (1.0 + skew));
    int Eb = ss_binade(pred);
    int b0 = ss_rep_base(pred);
    float r0 = flt(b0), r1 = flt(b0 | 1);
    bool nz = false;
    float s = 0.0f;
    bool ok = true;
    auto close = [&]() {
        // the run's representatives must still be inside its binade
        return r1 < ss_top(Eb) && ss_apply(s, SsMap{bits(r0) - b0, bits(r1) - (b0 | 1), nz}, Eb);
    };
    for (int i = 0; i < n && ok; i++) {
        const double Pa = P + (double)t[i];
        pred = (float)(Pa * (1.0 + skew));
        const int Ea = ss_binade(pred);
        if (Ea == Eb) {
            r0 = r0 + t[i];
            r1 = r1 + t[i];
            nz = nz || t[i] != 0.0f;
        } else {
            ok = close();
            s = s + t[i];
            Eb = Ea;
            b0 = ss_rep_base(pred);
            r0 = flt(b0);
            r1 = flt(b0 | 1);
            nz = false;
        }
        P = Pa;
    }
    if (ok) ok = close();
    if (fast) *fast = ok;
    if (ok) return s;
    float r = 0.0f;
    for (int i = 0; i < n; i++) r = r + t[i];
    return r;
}

// The device's std::exp(float) (gten/ops.cpp:752,1072) over an array.
extern "C" int nc_expf(const float* x, float* y, int64_t n, void* stream)
{
    NC_CHECK_ARG(x && y && n >= 0, "expf: bad arguments");
    if (!n) return NC_OK;
    hipLaunchKernelGGL(k_expf, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream_of(stream), x, y, n);
    return launch_status("k_expf");
}
