// nc_dmv.h -- device code shared by the fused matvec kernels of the
// single-row decode step (nc_decode.hip: k_dmv, k_dmv_head; nc_decode_glu.hip:
// the gate|up kernels): Q8 activation chunks, the norm prologue and the
// speculative-norm driver, plus the launch entry of the gate|up kernels.
#pragma once

#include <hip/hip_ext.h>

#include <algorithm>
#include <type_traits>

#include "nc_act.h"
#include "nc_decode.h"
#include "nc_qdot.h"
#include "nc_seqsum.h"

namespace nc {

constexpr int kDmvThreads = 256;
constexpr int kDmvMaxItems = 12;    // weight blocks per thread and row group
constexpr int kDmvNormChunks = 2;   // norm prologues: 8-value chunks per thread (NCH <= 2: K <= 4096)
constexpr int kDmvMaxGrid = 4096;

// Q8 round trip of 8 values of one block held by a lane quad:
// q8_quantize_block (gten/quants.cpp:16-30) -- absmax, delta = absmax/127,
// fp16 delta stored, scale 1/delta from the fp32 delta, roundf -- and the
// read back (code * fp16 delta).  Codes and delta returned for storing.
struct Q8Chunk {
    int8_t q[8];
    uint16_t d16;
};

__device__ __forceinline__ Q8Chunk quad_quantize(const float (&v)[8])
{
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(v[i]));
    a = quad_max(a);
    const float delta = a / 127.0f;
    Q8Chunk r;
    r.d16 = f2h(delta);
    const float scale = delta != 0.0f ? 1.0f / delta : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) r.q[i] = (int8_t)roundf(v[i] * scale);
    return r;
}

// quad_quantize, which also returns the fp32 delta (dl) and whether a code
// of these 8 values could change when the block is recomputed from a
// denominator other than this one (unc).  Why that can be decided here:
// the block y = RN(RN(h / D) g) under another D' = D / rho is y' = y rho
// (1 + t) with |t| <= 4.0001u (u = 2^-24, one factor 1 +- u per rounding),
// and amax' lies within the same factors of amax rho, so the scaled value
// z = RN(y RN(1 / RN(amax / 127))) becomes z' = z (1 + t'), |t'| <= 14.0001u:
// rho cancels.  A code roundf(z) can then change only when a half-integer
// lies within 14.0001u |z| of z; unc flags every value with |z| within
// 16u |z| = 2^-20 |z| of one (both sides exact in fp32 for |z| < 2^23).
// The delta's fp16 rounding does depend on rho: the exact side checks it.
__device__ __forceinline__ Q8Chunk quad_quantize_cert(const float (&v)[8], float& dl, bool& unc)
{
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(v[i]));
    a = quad_max(a);
    const float delta = a / 127.0f;
    Q8Chunk r;
    r.d16 = f2h(delta);
    const float scale = delta != 0.0f ? 1.0f / delta : 0.0f;
    bool u = false;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float z = v[i] * scale;
        r.q[i] = (int8_t)roundf(z);
        const float az = fabsf(z);
        u = u || fabsf((az - floorf(az)) - 0.5f) <= az * 0x1p-20f;
    }
    dl = delta;
    unc = u;
    return r;
}

__device__ __forceinline__ void quad_roundtrip(float (&v)[8])
{
    const Q8Chunk c = quad_quantize(v);
    const float d = h2f(c.d16);
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)c.q[i] * d;
}

// Chunk ch (values 8ch .. 8ch+7) of a Q8 Act row of K values.
__device__ __forceinline__ void load_act_chunk(const uint8_t* row, int K, int ch, float (&v)[8])
{
    const uint2 q = *reinterpret_cast<const uint2*>(row + (size_t)ch * 8);
    const float d = h2f(reinterpret_cast<const uint16_t*>(row + K)[ch >> 2]);
    const uint32_t w[2] = {q.x, q.y};
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xFFu) * d;
}

__device__ __forceinline__ void store_act_chunk(uint8_t* row, int K, int ch, const Q8Chunk& c)
{
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; i++) w[i >> 2] |= (uint32_t)(uint8_t)c.q[i] << (8 * (i & 3));
    *reinterpret_cast<uint2*>(row + (size_t)ch * 8) = make_uint2(w[0], w[1]);
    if ((ch & 3) == 0) reinterpret_cast<uint16_t*>(row + K)[ch >> 2] = c.d16;
}

__device__ __forceinline__ void load_f32_chunk(const float* p, int ch, float (&v)[8])
{
    const float4 a = reinterpret_cast<const float4*>(p)[2 * ch];
    const float4 b = reinterpret_cast<const float4*>(p)[2 * ch + 1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// The prologue: builds the activation row the matvec consumes and stages
// it in LDS by AVX lane (xs).  The inputs are requested first, then
// load_w() requests the workgroup's first weights, and the row is built
// while the weights are in flight (LDS barriers do not wait for global
// loads).  sq: K floats of LDS for the squares and the Act row.  Ends with
// an LDS barrier.  ROWS_FIRST (norm prologues): the weights are requested
// only once the rows have arrived -- a launch that requests tens of MB
// would otherwise queue its rows behind its own weights.
template <int PRO, int NCH, bool ROWS_FIRST = false, int NT = kDmvThreads, class LoadW>
__device__ __forceinline__ int dmv_prologue(const DmvArgs& A, uint32_t* xs, float* sq, SsShared& ssh, SgShared& sgh,
                                            LoadW&& load_w)
{
    constexpr bool RES = pro_res(PRO), LN = pro_ln(PRO);
    const int tid = threadIdx.x;
    const int nb = A.nb, K = nb * 32;
    const int nch = K / 8;
    uint8_t* xq = reinterpret_cast<uint8_t*>(sq);
    if (PRO == PRO_X) {
        XRaw xr{};
        if (tid < nb) xr = load_x_block(A.x, nb, tid);
        // scheduling fences keep the row's loads first and every weight
        // load issued before anything waits on the row
        __builtin_amdgcn_sched_barrier(0);
        load_w();
        __builtin_amdgcn_sched_barrier(0);
        if (tid < nb) stage_x_block(xr, xs + tid * kStage);
        lds_barrier();
        return A.pos;  // not used after a PRO_X prologue
    } else {
        // h: the stored row (PRO_RMS, PRO_LN) or the residual sum (RES)
        float h[NCH][8], gain[NCH][8], bias[NCH][8];
        // rows of 2048 values: the block sum's first phase from the terms in
        // registers (thread j's chunk is the sum's chunk j)
        constexpr bool REG8 = NCH == 1;
        const bool reg8 = REG8 && K == 2048;
        float tsq[8];
        float av[NCH][8], ov[NCH][8];
        // A row at a fixed address (x_pitch = 0, res_cur) is requested
        // before the position: the position is then loaded after the row
        // and before the weights, so waiting for it does not wait for them.
        const bool fixed = !RES ? A.x_pitch == 0 : A.res_cur != nullptr;
        int pos = A.pos;
        const uint8_t* arow;
        if (fixed) {
            arow = !RES ? A.x : A.res_cur;
        } else {
            if (A.dpos) pos = load_pos(A.dpos);
            arow = !RES ? A.x + (size_t)pos * A.x_pitch : A.res_in + (size_t)pos * A.res_pitch;
        }
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int ch = tid + j * NT;
            const int cc = ch < nch ? ch : 0;
            load_act_chunk(arow, K, cc, av[j]);
            if (RES) load_f32_chunk(A.raw_in, cc, ov[j]);
            const uint4 gw = reinterpret_cast<const uint4*>(A.norm_w)[cc];
            const uint32_t gws[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
            for (int i = 0; i < 8; i++) gain[j][i] = h2f((uint16_t)(gws[i >> 1] >> (16 * (i & 1))));
            if (LN) {
                const uint4 bw = reinterpret_cast<const uint4*>(A.norm_b)[cc];
                const uint32_t bws[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
                for (int i = 0; i < 8; i++) bias[j][i] = h2f((uint16_t)(bws[i >> 1] >> (16 * (i & 1))));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        int posv = 0;
        if (fixed && A.dpos) posv = load_pos(A.dpos);
        if (ROWS_FIRST) wait_loads_done();
        __builtin_amdgcn_sched_barrier(0);
        load_w();
        __builtin_amdgcn_sched_barrier(0);
        if (fixed && A.dpos) pos = posv;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int ch = tid + j * NT;
            const bool valid = ch < nch;
            if (j * NT >= nch) break;  // uniform
            if (RES) {
                quad_roundtrip(ov[j]);
                if (A.bscale != 1.0f) {
#pragma unroll
                    for (int i = 0; i < 8; i++) ov[j][i] = ov[j][i] * A.bscale;
                    quad_roundtrip(ov[j]);
                }
                float s[8];
#pragma unroll
                for (int i = 0; i < 8; i++) s[i] = av[j][i] + ov[j][i];
                const Q8Chunk q = quad_quantize(s);
                if (valid && blockIdx.x == 0) {
                    store_act_chunk(A.res_out + (size_t)pos * A.res_pitch, K, ch, q);
                    if (A.res_cur_out) store_act_chunk(A.res_cur_out, K, ch, q);
                }
                const float d = h2f(q.d16);
#pragma unroll
                for (int i = 0; i < 8; i++) h[j][i] = (float)q.q[i] * d;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) h[j][i] = av[j][i];
            }
            if (valid) {
                // rms_norm: the squares; layer_norm: the values (the mean first)
                float t[8];
#pragma unroll
                for (int i = 0; i < 8; i++) t[i] = LN ? h[j][i] : h[j][i] * h[j][i];
                reinterpret_cast<float4*>(sq)[2 * ch] = make_float4(t[0], t[1], t[2], t[3]);
                reinterpret_cast<float4*>(sq)[2 * ch + 1] = make_float4(t[4], t[5], t[6], t[7]);
                if (REG8 && j == 0)
#pragma unroll
                    for (int i = 0; i < 8; i++) tsq[i] = t[i];
            }
        }
        if (LN || !reg8) lds_barrier();
        float mean = 0.0f;
        if (LN) {
            // layer_norm (gten/ops.cpp:669-698): the mean as the exact sum of
            // the Q8 row's values (on the fp16 grid), then the squared
            // deviations' exact sum
            static_assert(!LN || NCH == 1, "layer_norm prologue: rows of up to 8 values per thread");
            mean = block_seq_sum_grid<(LN ? 2048 / NT : 1), NT>(sq, sgh) / (float)K;
#pragma unroll
            for (int j = 0; j < NCH; j++) {
                const int ch = tid + j * NT;
                if (ch < nch) {
                    float t[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) t[i] = (h[j][i] - mean) * (h[j][i] - mean);
                    reinterpret_cast<float4*>(sq)[2 * ch] = make_float4(t[0], t[1], t[2], t[3]);
                    reinterpret_cast<float4*>(sq)[2 * ch + 1] = make_float4(t[4], t[5], t[6], t[7]);
                    if (j == 0)
#pragma unroll
                        for (int i = 0; i < 8; i++) tsq[i] = t[i];
                }
            }
        }
        // (reg8: the call's own barrier publishes the terms)
        if (!reg8 && LN) lds_barrier();
        const float ss = reg8 ? block_seq_sum_regs8(tsq, sq, ssh) : block_seq_sum_nonneg(sq, K, ssh);
        const float denom = LN ? sqrtf(ss / (float)K) + 1e-05f : sqrtf(ss / (float)K) + 1e-6f;
        // the normalized row as stored (codes, then deltas) over sq's bytes
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int ch = tid + j * NT;
            if (j * NT >= nch) break;  // uniform
            float y[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                y[i] = LN ? ((h[j][i] - mean) / denom) * gain[j][i] + bias[j][i] : h[j][i] / denom * gain[j][i];
            if (A.post_scale != 1.0f) {
                quad_roundtrip(y);
#pragma unroll
                for (int i = 0; i < 8; i++) y[i] = y[i] * A.post_scale;
            }
            const Q8Chunk q = quad_quantize(y);
            if (ch < nch) store_act_chunk(xq, K, ch, q);
        }
        lds_barrier();
        if (tid < nb) stage_x_block(load_x_block(xq, nb, tid), xs + tid * kStage);
        lds_barrier();
        return pos;
    }
}

constexpr int kGluThreads = 512;  // gate|up workgroup: 64 rows' block terms over 8 wavefronts
constexpr int kGluMaxItems = 18;  // 64 rows x NB blocks / threads, NB <= 72

// ================================================ speculative norm rows ==
// The gate|up norm-prologue launch with the weight-block terms computed
// beside the exact norm sums instead of after them.  Threads 0-255 build the
// row and run the exact norm as dmv_prologue does, synchronizing among
// themselves through an LDS counter; the other 512 threads hold the
// weights.  While the exact sums run they normalize the row with an
// approximate sum of squares (and mean, for layer_norm; any order),
// quantize it and compute every weight block's four terms against that row
// as the weights arrive.  Once the exact sum is known, threads 0-255
// quantize the exact row and compare it with the speculative one block by
// block (rms_norm: only the blocks the speculative side could not certify
// as unchanged, spec_rms_uncertain).  A block's terms are a function of its
// 32 codes and its fp16 delta alone, so where those match the speculative
// terms are the exact ones; the
// weight threads recompute the terms of every block that differs.  The fold
// then sees the terms of the exact row, and the result is the reference's
// bit for bit whatever the approximation was.  (With unit norm gains the
// normalized row is a rescaled Q8 row, and requantizing it meets exact ties
// that the last bit of the rms decides: a few blocks per row differ there.)
constexpr int kSpecExact = kSsThreads;  // threads of the exact path

// Dynamic LDS of the speculative prologue (after the kernel's fold terms).
struct SpecLds {
    float* sq;     // K terms of the exact sums: rms_norm's squares; layer_norm's values, then squared deviations
    float* h;      // K values of the row before the norm
    float* g;      // K norm gains
    float* b;      // K norm biases (layer_norm)
    uint8_t* row;  // the speculative Act row, then the exact one: K codes, nb fp16 deltas
    uint8_t* bad;  // nb flags: the block differs between the two rows
    float* dl;     // rms_norm: nb fp32 deltas of the speculative row (its first quantization's)
    uint8_t* uc;   // rms_norm: K / 8 flags: a code of the chunk may differ in the exact row
};

__host__ __device__ constexpr size_t spec_lds_bytes(int nb, bool ln)
{
    return (size_t)nb * 32 * 4 * (ln ? 4 : 3) + (((size_t)nb * 34 + 15) & ~(size_t)15) +
           (((size_t)nb + 15) & ~(size_t)15) + (size_t)nb * 4 + (((size_t)nb * 4 + 15) & ~(size_t)15);
}

__device__ __forceinline__ SpecLds spec_lds(float* base, int nb, bool ln)
{
    const int K = nb * 32;
    const int na = ln ? 4 : 3;
    SpecLds L;
    L.sq = base;
    L.h = base + K;
    L.g = base + 2 * K;
    L.b = ln ? base + 3 * K : nullptr;
    L.row = reinterpret_cast<uint8_t*>(base + na * K);
    L.bad = L.row + ((nb * 34 + 15) & ~15);
    L.dl = reinterpret_cast<float*>(L.bad + ((nb + 15) & ~15));
    L.uc = reinterpret_cast<uint8_t*>(L.dl + nb);
    return L;
}

// Sum of the K squares in some order (a prediction only), the same value on
// every lane of every wavefront that calls it: lane l adds K/64 terms, then
// a butterfly, then lane 0's value.
__device__ __forceinline__ float spec_approx_sum(const float* sq, int K)
{
    const int lane = threadIdx.x & (kWave - 1), c = K / kWave;
    float v = 0.0f;
    for (int k = 0; k < c; k += 4) {
        const float4 q = *reinterpret_cast<const float4*>(sq + lane * c + k);
        v = v + ((q.x + q.y) + (q.z + q.w));
    }
#pragma unroll
    for (int o = kWave / 2; o >= 1; o >>= 1) v = v + __shfl_xor(v, o);
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// The normalized chunk, quantized, as dmv_prologue computes it:
// rms_norm y = h / denom * g, layer_norm y = ((h - mean) / denom) * g + b,
// then the post scale's round trip.
template <bool LN>
__device__ __forceinline__ Q8Chunk spec_norm_chunk(const float (&h)[8], const float (&g)[8], const float (&b)[8],
                                                   float mean, float denom, float post)
{
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = LN ? ((h[i] - mean) / denom) * g[i] + b[i] : h[i] / denom * g[i];
    if (post != 1.0f) {
        quad_roundtrip(y);
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = y[i] * post;
    }
    return quad_quantize(y);
}

// spec_norm_chunk for rms_norm, which also returns the fp32 delta of the
// first quantization (the post scale's round trip, else the row's own) and
// its code flag (quad_quantize_cert): with those two the exact side can tell
// whether the chunk changes under its own denominator.  Once the first
// quantization's codes and fp16 delta are the same, everything after it is.
__device__ __forceinline__ Q8Chunk spec_rms_chunk_cert(const float (&h)[8], const float (&g)[8], float denom,
                                                       float post, float& dl, bool& unc)
{
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) y[i] = h[i] / denom * g[i];
    Q8Chunk q = quad_quantize_cert(y, dl, unc);
    if (post != 1.0f) {
        const float d = h2f(q.d16);
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = (float)q.q[i] * d;
#pragma unroll
        for (int i = 0; i < 8; i++) y[i] = y[i] * post;
        q = quad_quantize(y);
    }
    return q;
}

// Whether the exact row's chunk may differ from the speculative one
// (rms_norm; the caller ORs the flags of a block's lane quad).  dl, uc: the
// speculative chunk's first delta and code flag; r = RN(Ds / De), the ratio
// of the two denominators.  The exact delta dl' = RN(amax' / 127) lies in
// dl rho [1 - 6.0001u, 1 + 6.0001u] and rho = Ds / De in r [1 - u, 1 + 1.0001u],
// so dl' is inside [lo, hi] below (each product's rounding counted), and the
// fp16 rounding, monotone, gives dl's fp16 value everywhere in it when it
// gives it at both ends.  Deltas below 2^-66 (where values may be subnormal)
// are not certified.
__device__ __forceinline__ bool spec_rms_uncertain(float dl, bool uc, float r)
{
    if (uc || !(dl >= 0x1p-66f)) return true;
    const float p = dl * r;
    const float lo = p * 0x1.ffffecp-1f;  // 1 - 10u
    const float hi = p * 0x1.00000ap0f;   // 1 + 10u
    const uint16_t d16 = f2h(dl);
    return f2h(lo) != d16 || f2h(hi) != d16;
}

// LDS state of the two sides.
struct SpecSync {
    int exact;    // barrier counter of threads 0-255 (the exact sum)
    int spec;     // barrier counter of the weight threads
    int anybad;   // some block differs: the speculative results are void
    float wsum[kSpecExact / kWave];   // per exact wavefront: its part of the squares (the prediction)
    float wsum1[kSpecExact / kWave];  // ... and of the values (layer_norm's predicted mean)
    float dn;                         // the speculative row's denominator
};

// The two roles of a speculative norm launch.  The workgroup's first
// kSpecExact threads (the exact role) and the others (the weight role) run
// separate code: the kernel branches on a wave-uniform role, so the weight
// registers are not live on the exact role's path and each role's code is
// allocated registers of its own.  Both roles pass the same workgroup
// barriers in the same order:
//   B1  the row, its partial sums and the norm inputs are in LDS;
//   B2  the exact role has compared the rows, the weight role has held its
//       results (sy.anybad tells both what follows);
//   when a block differs: B3 exact row stored, B4 its terms recomputed,
//   then the kernel's exact tail (its own barriers).

// Exact role, up to B2 (B2 not passed).  Returns the exact row's chunks in
// qx for the blocks it requantized (stored over the speculative row by the
// caller where a block differs).
// When the weight role requests its weights (ISSUE): kIssueAfterRows after
// the exact role's rows have arrived; kIssueAfterSpecRow the same, the
// wavefronts that compute the speculative row after it; kIssueEarly as soon
// as the exact role has requested its rows (barrier B0).  Measured on-box:
// early issue TinyLlama-Q4 1,529 -> 1,558 tok/s but Zephyr-Q4 (layer_norm,
// whose longer exact path the weights then delay) 1,177 -> 1,166 and
// TinyLlama-Q8 1,384 -> 1,377; after the speculative row TinyLlama-Q4
// 1,513 -> 1,522, TinyLlama-Q8 1,374 -> 1,370.
enum { kIssueAfterRows = 0, kIssueAfterSpecRow = 1, kIssueEarly = 2 };
template <int WT, int PRO>
constexpr int spec_issue()
{
    return WT != Q4 ? kIssueAfterRows : (pro_ln(PRO) ? kIssueAfterSpecRow : kIssueEarly);
}

template <int PRO, int NCH, int NS, int ISSUE, int PRIO = 3>
__device__ __forceinline__ void spec_exact(const DmvArgs& A, const SpecLds& L, SsShared& ssh, SgShared& sgh,
                                           SpecSync& sy, Q8Chunk (&qx)[NCH])
{
    constexpr int NT = kSpecExact;
    constexpr bool RES = pro_res(PRO), LN = pro_ln(PRO);
    static_assert(!LN || NCH == 1, "layer_norm prologue: rows of 2048 values");
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int nb = A.nb, K = nb * 32;
    const int nch = K / 8;
    float h[NCH][8], gain[NCH][8], bias[NCH][8], av[NCH][8], ov[NCH][8];
    // rows of 2048 values: the block sum's first phase from the terms in
    // registers (thread j's chunk is the sum's chunk j)
    const bool reg8 = NCH == 1 && K == 2048;
    float v16[kSsMaxPer];
    float I = 0.0f;
    const bool fixed = !RES ? A.x_pitch == 0 : A.res_cur != nullptr;
    int pos = A.pos;
    if (tid == 0) {
        sy.exact = 0;
        sy.spec = 0;
        sy.anybad = 0;
    }
    // on the critical path (PRIO 3), these wavefronts issue first
    __builtin_amdgcn_s_setprio(PRIO);
    const uint8_t* arow;
    if (fixed) {
        arow = !RES ? A.x : A.res_cur;
    } else {
        if (A.dpos) pos = load_pos(A.dpos);
        arow = !RES ? A.x + (size_t)pos * A.x_pitch : A.res_in + (size_t)pos * A.res_pitch;
    }
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int ch = tid + j * NT;
        const int cc = ch < nch ? ch : 0;
        load_act_chunk(arow, K, cc, av[j]);
        if (RES) load_f32_chunk(A.raw_in, cc, ov[j]);
        const uint4 gw = reinterpret_cast<const uint4*>(A.norm_w)[cc];
        const uint32_t gws[4] = {gw.x, gw.y, gw.z, gw.w};
#pragma unroll
        for (int i = 0; i < 8; i++) gain[j][i] = h2f((uint16_t)(gws[i >> 1] >> (16 * (i & 1))));
        if (LN) {
            const uint4 bw = reinterpret_cast<const uint4*>(A.norm_b)[cc];
            const uint32_t bws[4] = {bw.x, bw.y, bw.z, bw.w};
#pragma unroll
            for (int i = 0; i < 8; i++) bias[j][i] = h2f((uint16_t)(bws[i >> 1] >> (16 * (i & 1))));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (fixed && A.dpos) pos = load_pos(A.dpos);
    if (ISSUE == kIssueEarly) {
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // B0: the rows requested, the weights may follow
        __builtin_amdgcn_sched_barrier(0);
    }
    float part = 0.0f, part1 = 0.0f;  // this thread's squares and values, for the prediction
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int ch = tid + j * NT;
        const bool valid = ch < nch;
        if (j * NT >= nch) break;  // uniform
        if (RES) {
            quad_roundtrip(ov[j]);
            if (A.bscale != 1.0f) {
#pragma unroll
                for (int i = 0; i < 8; i++) ov[j][i] = ov[j][i] * A.bscale;
                quad_roundtrip(ov[j]);
            }
            float sm[8];
#pragma unroll
            for (int i = 0; i < 8; i++) sm[i] = av[j][i] + ov[j][i];
            const Q8Chunk q = quad_quantize(sm);
            if (valid && blockIdx.x == 0) {
                store_act_chunk(A.res_out + (size_t)pos * A.res_pitch, K, ch, q);
                if (A.res_cur_out) store_act_chunk(A.res_cur_out, K, ch, q);
            }
            const float d = h2f(q.d16);
#pragma unroll
            for (int i = 0; i < 8; i++) h[j][i] = (float)q.q[i] * d;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) h[j][i] = av[j][i];
        }
        if (valid) {
            float sqv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) sqv[i] = h[j][i] * h[j][i];
            // the first exact sum's terms: the squares (rms_norm) or the values (layer_norm)
            const float(&t)[8] = LN ? h[j] : sqv;
            float4* sq4 = reinterpret_cast<float4*>(L.sq) + 2 * ch;
            sq4[0] = make_float4(t[0], t[1], t[2], t[3]);
            sq4[1] = make_float4(t[4], t[5], t[6], t[7]);
            part = part + (((sqv[0] + sqv[1]) + (sqv[2] + sqv[3])) + ((sqv[4] + sqv[5]) + (sqv[6] + sqv[7])));
            if (LN)
                part1 = part1 + (((h[j][0] + h[j][1]) + (h[j][2] + h[j][3])) +
                                 ((h[j][4] + h[j][5]) + (h[j][6] + h[j][7])));
            float4* h4 = reinterpret_cast<float4*>(L.h) + 2 * ch;
            h4[0] = make_float4(h[j][0], h[j][1], h[j][2], h[j][3]);
            h4[1] = make_float4(h[j][4], h[j][5], h[j][6], h[j][7]);
            float4* g4 = reinterpret_cast<float4*>(L.g) + 2 * ch;
            g4[0] = make_float4(gain[j][0], gain[j][1], gain[j][2], gain[j][3]);
            g4[1] = make_float4(gain[j][4], gain[j][5], gain[j][6], gain[j][7]);
            if (LN) {
                float4* b4 = reinterpret_cast<float4*>(L.b) + 2 * ch;
                b4[0] = make_float4(bias[j][0], bias[j][1], bias[j][2], bias[j][3]);
                b4[1] = make_float4(bias[j][4], bias[j][5], bias[j][6], bias[j][7]);
            }
            if (!LN && NCH == 1)
#pragma unroll
                for (int i = 0; i < kSsMaxPer; i++) v16[i] = i < 8 ? sqv[i] : 0.0f;
        }
    }
    if (!LN && reg8) I = ss_prefix<8>(v16, 8, ssh);
    part = wave_scan_add(part);
    if (lane == kWave - 1) sy.wsum[tid / kWave] = part;
    if (LN) {
        part1 = wave_scan_add(part1);
        if (lane == kWave - 1) sy.wsum1[tid / kWave] = part1;
    }
    lds_barrier();  // B1
    // the exact sums, then the exact row (held until the weight role is done)
    SsWaveBarrier<NT / kWave> bar{&sy.exact, 0};
    float mean = 0.0f;
    if constexpr (LN) {
        // layer_norm (gten/ops.cpp:669-698): the mean, the exact sum of the
        // Q8 row's values (on the fp16 grid), then the squared deviations
        // over the values in sq
        mean = block_seq_sum_grid<8, NT>(L.sq, sgh, nullptr, bar) / (float)K;
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; i++) t[i] = (h[0][i] - mean) * (h[0][i] - mean);
        float4* sq4 = reinterpret_cast<float4*>(L.sq) + 2 * tid;
        sq4[0] = make_float4(t[0], t[1], t[2], t[3]);
        sq4[1] = make_float4(t[4], t[5], t[6], t[7]);
#pragma unroll
        for (int i = 0; i < kSsMaxPer; i++) v16[i] = i < 8 ? t[i] : 0.0f;
        I = ss_prefix<8>(v16, 8, ssh);
        bar();
    }
    // (reg8: the first phase ran before the barrier that published the terms)
    const float ss = reg8 ? block_seq_sum_after<8, false, false>(v16, I, L.sq, K, ssh, nullptr, bar)
                          : block_seq_sum_nonneg_bar(L.sq, K, ssh, bar);
    const float denom = LN ? sqrtf(ss / (float)K) + 1e-05f : sqrtf(ss / (float)K) + 1e-6f;
    if constexpr (LN) {
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            if (j * NT >= nch) break;  // uniform
            qx[j] = spec_norm_chunk<LN>(h[j], gain[j], bias[j], mean, denom, A.post_scale);
        }
    }
    // once the speculative row is complete (every weight wavefront has
    // passed its first barrier), compare it block by block with the exact
    // one (a lane quad holds a block) while the weight role finishes
    while (__hip_atomic_load(&sy.spec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < NS / kWave) {
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    // rms_norm: only the blocks the speculative side could not certify are
    // requantized here (spec_rms_uncertain); the same denominator certifies
    // every block.  layer_norm requantizes every block.
    const float dns = LN ? 0.0f : sy.dn;
    const bool same = !LN && dns == denom;
    const float r = dns / denom;
    const bool okr = r > 0.0f && r < __builtin_inff();
    int any = 0;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int ch = tid + j * NT;
        if (j * NT >= nch) break;  // uniform
        const bool valid = ch < nch;
        const int cc = valid ? ch : 0;
        bool check = true;
        if constexpr (!LN) {
            bool unc = false;
            if (!same) unc = !okr || spec_rms_uncertain(L.dl[cc >> 2], L.uc[cc] != 0, r);
            int ui = unc ? 1 : 0;
            ui |= dpp_i<kDppQuadXor1>(ui);
            ui |= dpp_i<kDppQuadXor2>(ui);
            check = ui != 0;  // uniform over the block's lane quad
            if (check) qx[j] = spec_norm_chunk<false>(h[j], gain[j], bias[j], 0.0f, denom, A.post_scale);
        }
        int diff = 0;
        if (check) {
            const Q8Chunk& q = qx[j];
            const uint2 sc = *reinterpret_cast<const uint2*>(L.row + (size_t)cc * 8);
            const uint16_t sd = reinterpret_cast<const uint16_t*>(L.row + K)[cc >> 2];
            uint32_t w[2] = {0, 0};
#pragma unroll
            for (int i = 0; i < 8; i++) w[i >> 2] |= (uint32_t)(uint8_t)q.q[i] << (8 * (i & 3));
            diff = valid && (sc.x != w[0] || sc.y != w[1] || sd != q.d16) ? 1 : 0;
            diff |= dpp_i<kDppQuadXor1>(diff);
            diff |= dpp_i<kDppQuadXor2>(diff);
        }
        any |= diff;
        if (valid && (ch & 3) == 0) L.bad[ch >> 2] = (uint8_t)diff;
    }
    if (__builtin_amdgcn_ballot_w64(any != 0) && lane == 0) sy.anybad = 1;
    __builtin_amdgcn_s_setprio(0);
}

// The exact role's stores after B2 when a block differs: the exact row over
// the speculative one, then B3 and B4 (the weight role recomputes the
// differing blocks' terms between them).
template <int NCH>
__device__ __forceinline__ void spec_exact_fixup(const DmvArgs& A, const SpecLds& L, const Q8Chunk (&qx)[NCH])
{
    constexpr int NT = kSpecExact;
    const int K = A.nb * 32, nch = K / 8;
    if (A.spec_fixups && threadIdx.x == 0) atomicAdd(A.spec_fixups, 1);
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        const int ch = threadIdx.x + j * NT;
        if (j * NT >= nch) break;  // uniform
        // (only a differing block's chunks were requantized)
        if (ch < nch && L.bad[ch >> 2]) store_act_chunk(L.row, K, ch, qx[j]);
    }
    lds_barrier();  // B3
    lds_barrier();  // B4
}

// Weight role, up to B2 (B2 not passed): B1, the weight requests (issued
// after the exact role's rows have arrived, so that those are not queued
// behind them: q|k|v 7.46 -> 6.84 us), the speculative row (its first 256
// threads, a quad per block), a barrier among
// the weight wavefronts, every block's terms from that row (terms(1)), then
// spec_tail(bar): the fold and epilogue from those terms, held back.  NS:
// the weight role's threads; ISSUE: when the weights are requested (a
// wavefront waits at a large transfer's issue).
template <int PRO, int NCH, int NS, int ISSUE, class LoadW, class Terms, class SpecTail>
__device__ __forceinline__ void spec_weights(const DmvArgs& A, const SpecLds& L, SpecSync& sy, LoadW&& load_w,
                                             Terms&& terms, SpecTail&& spec_tail)
{
    constexpr int NT = kSpecExact;
    constexpr bool LN = pro_ln(PRO);
    const int nb = A.nb, K = nb * 32;
    const int nch = K / 8;
    constexpr bool ROW_FIRST = ISSUE == kIssueAfterSpecRow;
    if (ISSUE == kIssueEarly) {
        lds_barrier();  // B0
        load_w();
    }
    lds_barrier();  // B1
    const int sc = threadIdx.x - NT;
    if (ISSUE == kIssueAfterRows || (ROW_FIRST && sc >= NT)) load_w();
    if (sc < NT) {
        const float s2 = ((sy.wsum[0] + sy.wsum[1]) + sy.wsum[2]) + sy.wsum[3];
        float mn = 0.0f, dn;
        if (LN) {
            // mean and variance from the sums of the values and squares
            mn = (((sy.wsum1[0] + sy.wsum1[1]) + sy.wsum1[2]) + sy.wsum1[3]) / (float)K;
            const float var = fmaxf(s2 / (float)K - mn * mn, 0.0f) * A.spec_skew;
            dn = sqrtf(var) + 1e-05f;
        } else {
            dn = sqrtf(s2 * A.spec_skew / (float)K) + 1e-6f;
        }
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const int ch = sc + j * NT;
            if (j * NT >= nch) break;  // uniform
            const int cc = ch < nch ? ch : 0;
            float hv[8], gv[8], bv[8];
            load_f32_chunk(L.h, cc, hv);
            load_f32_chunk(L.g, cc, gv);
            if constexpr (LN) {
                load_f32_chunk(L.b, cc, bv);
                const Q8Chunk q = spec_norm_chunk<LN>(hv, gv, bv, mn, dn, A.post_scale);
                if (ch < nch) store_act_chunk(L.row, K, ch, q);
            } else {
                // with each chunk's first delta and code flag, for the exact side
                float dl;
                bool uc;
                const Q8Chunk q = spec_rms_chunk_cert(hv, gv, dn, A.post_scale, dl, uc);
                if (ch < nch) {
                    store_act_chunk(L.row, K, ch, q);
                    L.uc[ch] = uc ? 1 : 0;
                    if ((ch & 3) == 0) L.dl[ch >> 2] = dl;
                }
            }
        }
        if (sc == 0) sy.dn = dn;
        if (ROW_FIRST) load_w();
    }
    SsWaveBarrier<NS / kWave> sbar{&sy.spec, 0};
    sbar();
    terms(1);
    spec_tail(sbar);
}

// Compute units of the current device.
int device_cus();

// The gate|up launch with the SwiGLU epilogue (nc_decode_glu.hip): K = 32 nb
// of 1280, 1536, 2048 or 2304, a norm prologue (rms_norm; layer_norm at
// K = 2048).
int glu_dispatch(const DmvArgs& A, int wdtype, int pro, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1);

}  // namespace nc
