// nc_attention.hip -- causal GQA attention over the HBM-resident KV cache.
//
// Replaces qkv_attn -> qk_masked_softmax -> transpose_v -> qkv_matmul
// (gten/ops.cpp:1017-1220).  For query row r of head h (kv head g):
//   s_c  = dot(q_h, k_{c,g}) * (1/sqrtf(d_head)) for c <= r, -inf after,
//          with the reference's dot product of the activation dtype (Q8:
//          four integer lane sums per block, fp32 terms folded in block order;
//          F16: eight fp32 lanes summed left to right);
//   p    = softmax over the whole n_ctx row: max, expf(s - max), sequential
//          sum, divide; the probability row is requantized in the activation
//          dtype (Q8 blocks of 32 positions, last one partial) and read back;
//   o_j  = 8-lane fp32 dot of p with V column j over n_ctx positions (lane =
//          position mod 8, lanes summed left to right, then the n_ctx mod 8
//          tail in order); the 64 outputs are requantized as the attention
//          output row.
// The masked positions give p = 0 exactly (expf(-inf) = 0, requantized to
// 0): they add nothing to the sequential sum, to the absmax of their
// 32-position blocks or to the P.V lane chains (each starts at +0, and
// adding +/-0 leaves a running sum unchanged, its sign included).  So a row
// stops at its own position; only the lane/tail split keeps the call's
// n_ctx (its multiple of 8).
// The K and V caches are the K/V Linear outputs (rows = positions) in the
// activation dtype, as the reference keeps them (gten/modules.cpp:78-87).
// Any context up to kAttnMaxCtx positions: scores in shared memory, K rows
// read into registers one row ahead, the V slice streamed through shared
// memory in double-buffered chunks of kAvc positions under the P.V chains.
#include "nc_act.h"
#include "nc_kernels.h"
#include "nc_seqsum.h"

namespace nc {

__device__ __forceinline__ uint32_t pick_pair2(uint32_t lo, uint32_t hi, int odd)
{
    return odd ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
}

// Lane-permuted dwords of one 32-code block (see nc_matvec.hip).
__device__ __forceinline__ void lane_dwords(const uint4 a, const uint4 b, uint32_t xa[4], uint32_t xb[4])
{
    const uint32_t X[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xa[k] = pick_pair2(X[k >> 1], X[2 + (k >> 1)], k & 1);
        xb[k] = pick_pair2(X[4 + (k >> 1)], X[6 + (k >> 1)], k & 1);
    }
}

constexpr int kAttnThreads = 256;
constexpr int kAvc = 128;          // positions per staged V chunk
constexpr int kAttnSeqMax = 1024;  // single-row softmax sums up to this long run as one wavefront's loop

// One position's V head slice in shared memory: Q8 codes (64) + fp16
// deltas (2 x 2) rounded to 16, or 64 fp16 values; 16-byte parts of it.
template <int ADT>
__host__ __device__ constexpr int v_stage_bytes()
{
    return ADT == Q8 ? 80 : 128;
}
template <int ADT>
__host__ __device__ constexpr int v_parts()
{
    return ADT == Q8 ? 4 : 8;
}

// ---- K rows and scores ----------------------------------------------------

// A K row of head g: 64 Q8 codes and the two deltas (one dword), or 64 fp16
// values.
template <int ADT>
struct KRowT {
    uint4 q[ADT == Q8 ? 4 : 8];
    uint32_t d;
};

template <int ADT>
__device__ __forceinline__ KRowT<ADT> load_k(const uint8_t* kc, int k_pitch, int kvd, int g, int c)
{
    KRowT<ADT> r;
    const uint8_t* row = kc + (size_t)c * k_pitch;
    const uint4* p = reinterpret_cast<const uint4*>(row + g * (ADT == Q8 ? 64 : 128));
#pragma unroll
    for (int v = 0; v < (ADT == Q8 ? 4 : 8); v++) r.q[v] = p[v];
    r.d = ADT == Q8 ? reinterpret_cast<const uint32_t*>(row + kvd)[g] : 0u;
    return r;
}

// The query head: Q8 lane dwords and deltas, or 64 fp32 values.
template <int ADT>
struct QHead {
    uint32_t qa[2][4], qb[2][4];
    float dq[2];
    float qv[ADT == Q8 ? 1 : 64];
};

template <int ADT>
__device__ __forceinline__ void load_q(QHead<ADT>& Q, const uint8_t* qrow, int h, int qd)
{
    if (ADT == Q8) {
        const uint4* p = reinterpret_cast<const uint4*>(qrow + h * 64);
#pragma unroll
        for (int b = 0; b < 2; b++) {
            lane_dwords(p[2 * b], p[2 * b + 1], Q.qa[b], Q.qb[b]);
            Q.dq[b] = h2f(reinterpret_cast<const uint16_t*>(qrow + qd)[h * 2 + b]);
        }
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(qrow + h * 128);
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const uint4 t = p[v];
            const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                Q.qv[8 * v + 2 * e] = h2f((uint16_t)(w[e] & 0xFFFFu));
                Q.qv[8 * v + 2 * e + 1] = h2f((uint16_t)(w[e] >> 16));
            }
        }
    }
}

// dot(q_h, k) as vec_dot_product of the activation dtype (gten/ops.cpp:
// 208-242, 292-384), times scale.
template <int ADT>
__device__ __forceinline__ float score(const QHead<ADT>& Q, const KRowT<ADT>& K, float scale)
{
    if (ADT == Q8) {
        float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int b = 0; b < 2; b++) {
            uint32_t ka[4], kb[4];
            lane_dwords(K.q[2 * b], K.q[2 * b + 1], ka, kb);
            const float dd = Q.dq[b] * h2f((uint16_t)(K.d >> (16 * b)));
#pragma unroll
            for (int k = 0; k < 4; k++) {
                int L = __builtin_amdgcn_sdot4((int)Q.qa[b][k], (int)ka[k], 0, false);
                L = __builtin_amdgcn_sdot4((int)Q.qb[b][k], (int)kb[k], L, false);
                a4[k] = a4[k] + (float)L * dd;
            }
        }
        return ((a4[0] + a4[1]) + (a4[2] + a4[3])) * scale;
    } else {
        // products of two fp16 values are exact in fp32, so the fused
        // multiply-add equals the reference's multiply then add
        float a8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int v = 0; v < 8; v++) {
            const uint32_t w[4] = {K.q[v].x, K.q[v].y, K.q[v].z, K.q[v].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                a8[2 * e] = __builtin_fmaf(Q.qv[8 * v + 2 * e], h2f((uint16_t)(w[e] & 0xFFFFu)), a8[2 * e]);
                a8[2 * e + 1] = __builtin_fmaf(Q.qv[8 * v + 2 * e + 1], h2f((uint16_t)(w[e] >> 16)), a8[2 * e + 1]);
            }
        }
        const float s = a8[0] + a8[1] + a8[2] + a8[3] + a8[4] + a8[5] + a8[6] + a8[7];
        return s * scale;
    }
}

// ---- V chunks -------------------------------------------------------------

// The 16-byte parts of one V chunk a thread carries (parts tid + 256 i,
// position = part / v_parts within the chunk), and for Q8 the delta dword of
// position tid (threads below kAvc).
template <int ADT>
struct VChunkT {
    static constexpr int NP = kAvc * v_parts<ADT>() / kAttnThreads;
    uint32_t p[NP][4];  // plain words: an array of the uint4 union type stays in scratch memory
    uint32_t d;
};

// Loads chunk ch; positions are clamped to the rows that exist (those past
// the context are never read back).
template <int ADT>
__device__ __forceinline__ void load_vc(VChunkT<ADT>& v, const uint8_t* vc, int v_pitch, int kvd, int g, int ch,
                                        int rows)
{
    constexpr int VP = v_parts<ADT>();
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < VChunkT<ADT>::NP; i++) {
        const int idx = tid + i * kAttnThreads;
        const int c = min(ch * kAvc + idx / VP, rows - 1);
        const uint4 t4 = reinterpret_cast<const uint4*>(vc + (size_t)c * v_pitch + g * (ADT == Q8 ? 64 : 128))[idx % VP];
        v.p[i][0] = t4.x;
        v.p[i][1] = t4.y;
        v.p[i][2] = t4.z;
        v.p[i][3] = t4.w;
    }
    if (ADT == Q8) {
        const int c = min(ch * kAvc + (tid & (kAvc - 1)), rows - 1);
        v.d = reinterpret_cast<const uint32_t*>(vc + (size_t)c * v_pitch + kvd)[g];
    }
}

template <int ADT>
__device__ __forceinline__ void store_vc(const VChunkT<ADT>& v, uint8_t* buf)
{
    constexpr int VP = v_parts<ADT>(), VB = v_stage_bytes<ADT>();
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < VChunkT<ADT>::NP; i++) {
        const int idx = tid + i * kAttnThreads;
        reinterpret_cast<uint4*>(buf + (idx / VP) * VB)[idx % VP] = make_uint4(v.p[i][0], v.p[i][1], v.p[i][2], v.p[i][3]);
    }
    if (ADT == Q8 && tid < kAvc) reinterpret_cast<uint32_t*>(buf + tid * VB + 64)[0] = v.d;
}

// Values of columns 2m and 2m + 1 of a staged position.
template <int ADT>
__device__ __forceinline__ void v_pair(const uint8_t* vrow, int m, float& v0, float& v1)
{
    if (ADT == Q8) {
        const uint32_t codes = reinterpret_cast<const uint16_t*>(vrow)[m];
        const float d = h2f(reinterpret_cast<const uint16_t*>(vrow + 64)[m >> 4]);  // block of column 2m
        v0 = (float)(int8_t)(codes & 0xFFu) * d;
        v1 = (float)(int8_t)(codes >> 8) * d;
    } else {
        const uint32_t w = reinterpret_cast<const uint32_t*>(vrow)[m];
        v0 = h2f((uint16_t)(w & 0xFFFFu));
        v1 = h2f((uint16_t)(w >> 16));
    }
}

template <int ADT>
__device__ __forceinline__ float v_one(const uint8_t* vrow, int j)
{
    if (ADT == Q8)
        return (float)reinterpret_cast<const int8_t*>(vrow)[j] * h2f(reinterpret_cast<const uint16_t*>(vrow + 64)[j >> 5]);
    return h2f(reinterpret_cast<const uint16_t*>(vrow)[j]);
}

// ---- one query row per workgroup -------------------------------------------

// Workgroup (h, r): query row r of q / out (pointers at row `start`), the
// row's absolute position start + r (or *dpos: decode under graph replay,
// n_ctx = *dpos + 1).  Shared memory: scores [round_up(lds_ctx, 256)],
// P.V lane sums [8][64], two V chunk buffers.
template <int ADT>
__global__ __launch_bounds__(kAttnThreads) void k_attn(const uint8_t* __restrict__ q, int q_pitch,
                                                       const uint8_t* __restrict__ kc, int k_pitch,
                                                       const uint8_t* __restrict__ vc, int v_pitch,
                                                       uint8_t* __restrict__ out, int out_pitch, int hq, int hkv,
                                                       int start, int n_ctx, float scale,
                                                       const int* __restrict__ dpos, int lds_ctx)
{
    constexpr int VB = v_stage_bytes<ADT>();
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[8];
    __shared__ SsShared ssh;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = blockIdx.x;
    const int qr = blockIdx.y;
    const int g = h / (hq / hkv);
    const int qcols = hq * 64, kvcols = hkv * 64;
    const int qd = act_delta_offset(qcols), kvd = act_delta_offset(kvcols);
    // V chunk 0 does not depend on the position
    VChunkT<ADT> vch;
    load_vc<ADT>(vch, vc, v_pitch, kvd, g, 0, lds_ctx);
    if (dpos) {
        start = load_pos(dpos);
        n_ctx = start + 1;
    }
    const int row = start + qr;  // absolute position of the query
    const int n = row + 1;       // positions with p != 0
    const int n8 = n_ctx & ~7;   // the call's 8-lane part
    const int spad = (lds_ctx + kSsThreads - 1) & ~(kSsThreads - 1);
    float* S = sm;
    float* acc = S + spad;
    uint8_t* Vb = reinterpret_cast<uint8_t*>(acc + 512);
    const uint8_t* qrow = q + (size_t)qr * q_pitch;

    // ---- scores (thread = position), the next K row requested before the
    // current one is used
    {
        QHead<ADT> Q;
        load_q<ADT>(Q, qrow, h, qd);
        int c = tid;
        if (c < n) {
            KRowT<ADT> cur = load_k<ADT>(kc, k_pitch, kvd, g, c);
            for (;;) {
                const int cn = c + kAttnThreads;
                KRowT<ADT> nxt = cur;
                if (cn < n) nxt = load_k<ADT>(kc, k_pitch, kvd, g, cn);
                S[c] = score<ADT>(Q, cur, scale);
                if (cn >= n) break;
                cur = nxt;
                c = cn;
            }
        }
    }
    const int nch = (n + kAvc - 1) / kAvc;
    store_vc<ADT>(vch, Vb);
    if (nch > 1) load_vc<ADT>(vch, vc, v_pitch, kvd, g, 1, lds_ctx);
    lds_barrier();

    // ---- softmax: max (order-free), expf, sequential sum, divide, requantize
    float mx = -INFINITY;
    for (int c = tid; c < n; c += kAttnThreads) mx = fmaxf(mx, S[c]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red[w] = mx;
    lds_barrier();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const bool long_row = n > kAttnSeqMax;
    const int npad = (n + kSsThreads - 1) & ~(kSsThreads - 1);
    for (int c = tid; c < (long_row ? npad : n); c += kAttnThreads) S[c] = c < n ? expf_ref(S[c] - mx) : 0.0f;
    lds_barrier();
    float sum;
    if (long_row) {
        sum = block_seq_sum_nonneg(S, npad, ssh);  // exact; the zero padding changes nothing
    } else {
        if (w == 0) {
            const float ss = seq_sum(S, n);
            if (lane == 0) red[4] = ss;
        }
        lds_barrier();
        sum = red[4];
    }
    for (int c0 = 0; c0 < n; c0 += kAttnThreads) {
        const int c = c0 + tid;
        const bool valid = c < n;
        const float p = valid ? S[c] / sum : 0.0f;
        const float pr = act_roundtrip<ADT>(p, valid);
        if (valid) S[c] = pr;
    }
    lds_barrier();

    // ---- P.V: thread = (lane l = tid / 32, columns 2m, 2m + 1), chains over
    // positions l, l + 8, ... < min(n, n8) in order, chunk by chunk
    const int l = tid >> 5, m = tid & 31;
    const int lim = min(n, n8);
    float a0 = 0.0f, a1 = 0.0f;
    for (int ch = 0; ch < nch; ch++) {
        const uint8_t* B = Vb + (ch & 1) * (kAvc * VB);
        const int c0 = ch * kAvc;
        const int cend = min(c0 + kAvc, lim);
        int c = c0;
        for (; c + 64 <= cend; c += 64) {
            float p[8], v0[8], v1[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                p[u] = S[c + 8 * u + l];
                v_pair<ADT>(B + (c + 8 * u + l - c0) * VB, m, v0[u], v1[u]);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                a0 = p[u] * v0[u] + a0;
                a1 = p[u] * v1[u] + a1;
            }
        }
        for (; c < cend; c += 8) {
            if (c + l < cend) {  // lim is a multiple of 8 here (n = n_ctx); kept exact for any lim
                float v0, v1;
                v_pair<ADT>(B + (c + l - c0) * VB, m, v0, v1);
                const float p = S[c + l];
                a0 = p * v0 + a0;
                a1 = p * v1 + a1;
            }
        }
        if (ch + 1 < nch) {
            store_vc<ADT>(vch, Vb + ((ch + 1) & 1) * (kAvc * VB));
            if (ch + 2 < nch) load_vc<ADT>(vch, vc, v_pitch, kvd, g, ch + 2, lds_ctx);
        }
        lds_barrier();
    }
    *reinterpret_cast<float2*>(acc + l * 64 + 2 * m) = make_float2(a0, a1);
    lds_barrier();
    if (w == 0) {
        const int j = lane;
        float s = acc[j];
#pragma unroll
        for (int q8 = 1; q8 < 8; q8++) s = s + acc[q8 * 64 + j];
        // the tail [n8, n): within the last chunk, still in its buffer
        const uint8_t* B = Vb + ((nch - 1) & 1) * (kAvc * VB);
        const int c0 = (nch - 1) * kAvc;
        for (int c = n8; c < n; c++) s = s + S[c] * v_one<ADT>(B + (c - c0) * VB, j);
        act_store<ADT>(out + (size_t)qr * out_pitch, h * 64 + j, qd, s, true);
    }
}

// ---- R query rows per workgroup (prefill) ---------------------------------

// R consecutive query rows of one head per workgroup, with the arithmetic of
// k_attn: every K row and the V slice are read once for all of them.  Row i
// stops at its own position (see the file comment).  Shared memory: scores
// [R][mpad], two V chunk buffers.
template <int ADT, int R>
__global__ __launch_bounds__(kAttnThreads) void k_attn_rows(const uint8_t* __restrict__ q, int q_pitch,
                                                            const uint8_t* __restrict__ kc, int k_pitch,
                                                            const uint8_t* __restrict__ vc, int v_pitch,
                                                            uint8_t* __restrict__ out, int out_pitch, int hq, int hkv,
                                                            int start, int n_ctx, int rows, float scale)
{
    constexpr int VB = v_stage_bytes<ADT>();
    extern __shared__ __align__(16) float sm[];
    __shared__ float outs[R][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // the last row groups (the longest causal rows) are dispatched first, so
    // the short ones fill the tail of the launch
    const int h = blockIdx.x, qr0 = (gridDim.y - 1 - blockIdx.y) * R;
    const int nr = min(R, rows - qr0);
    const int m = start + qr0 + nr;  // positions attended by any of the rows
    const int mpad = (m + 3) & ~3;
    float* S = sm;                                                // [R][mpad]
    uint8_t* Vb = reinterpret_cast<uint8_t*>(S + R * mpad);       // 2 x [kAvc][VB]
    const int g = h / (hq / hkv);
    const int qcols = hq * 64, kvcols = hkv * 64;
    const int qd = act_delta_offset(qcols), kvd = act_delta_offset(kvcols);
    VChunkT<ADT> vch;
    load_vc<ADT>(vch, vc, v_pitch, kvd, g, 0, m);

    // ---- scores: thread = (row i, positions c0 + (256 / R) k); the R rows
    // sharing a position read its K row together
    {
        const int i = tid % R;
        const int ic = min(i, nr - 1);
        const int row = start + qr0 + i;  // absolute position of the query
        QHead<ADT> Q;
        load_q<ADT>(Q, q + (size_t)(qr0 + ic) * q_pitch, h, qd);
        const int lim = i < nr ? min(row + 1, m) : 0;
        int c = tid / R;
        if (c < lim) {
            KRowT<ADT> cur = load_k<ADT>(kc, k_pitch, kvd, g, c);
            for (;;) {
                const int cn = c + kAttnThreads / R;
                KRowT<ADT> nxt = cur;
                if (cn < lim) nxt = load_k<ADT>(kc, k_pitch, kvd, g, cn);
                S[i * mpad + c] = score<ADT>(Q, cur, scale);
                if (cn >= lim) break;
                cur = nxt;
                c = cn;
            }
        }
    }
    const int nch = (m + kAvc - 1) / kAvc;
    store_vc<ADT>(vch, Vb);
    if (nch > 1) load_vc<ADT>(vch, vc, v_pitch, kvd, g, 1, m);
    lds_barrier();

    // ---- softmax of row i: max, expf, sequential sum over [0, row],
    // divide, requantize in 32-position blocks.  Eight rows: rows w and w + 4
    // on the two halves of wavefront w (32 positions per half and step), so
    // their sequential sums run side by side; otherwise row i on wave i % 4.
    if constexpr (R == 8) {
        const int hl = lane & 31, i = w + 4 * (lane >> 5);
        const int n = i < nr ? start + qr0 + i + 1 : 0;  // this half's positions
        float* Si = S + min(i, R - 1) * mpad;
        float mx = -INFINITY;
        for (int c = hl; c < n; c += 32) mx = fmaxf(mx, Si[c]);
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        for (int c = hl; c < n; c += 32) Si[c] = expf_ref(Si[c] - mx);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        const float sum = seq_sum(Si, n);
        // the trip count is uniform within a half, so each 32-position
        // block's absmax sees all 32 lanes of its half
        for (int c0 = 0; c0 < n; c0 += 32) {
            const int c = c0 + hl;
            const bool valid = c < n;
            const float p = valid ? Si[c] / sum : 0.0f;
            const float pr = act_roundtrip<ADT>(p, valid);
            if (valid) Si[c] = pr;
        }
    } else
    for (int i = w; i < nr; i += kAttnThreads / kWave) {
        const int n = start + qr0 + i + 1;  // positions of this row
        float* Si = S + i * mpad;
        float mx = -INFINITY;
        for (int c = lane; c < n; c += kWave) mx = fmaxf(mx, Si[c]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        for (int c = lane; c < n; c += kWave) Si[c] = expf_ref(Si[c] - mx);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        const float sum = seq_sum(Si, n);
        for (int c0 = 0; c0 < n; c0 += kWave) {
            const int c = c0 + lane;
            const bool valid = c < n;
            const float p = valid ? Si[c] / sum : 0.0f;
            const float pr = act_roundtrip<ADT>(p, valid);
            if (valid) Si[c] = pr;
        }
    }
    lds_barrier();

    // ---- P.V: thread = (column j, lanes 2 lp and 2 lp + 1) for every row;
    // row i's lane chains cover positions < min(n_i, n8), n8 = the call's
    // n_ctx rounded down to 8 (the reference's 8-lane part), then the lane
    // sums left to right across the quad and the tail positions in order
    const int j = tid >> 2, lp = tid & 3;
    const int n8 = (n_ctx / 8) * 8;
    float a[R][2];
#pragma unroll
    for (int i = 0; i < R; i++) a[i][0] = a[i][1] = 0.0f;
    const int lim_max = min(m, n8);
    // below the first row's limit every row takes both positions: the
    // probabilities are read without per-row branches (which would wait for
    // each read in turn)
    const int lim_all = min(start + qr0 + 1, n8);
    for (int ch = 0; ch < nch; ch++) {
        const uint8_t* B = Vb + (ch & 1) * (kAvc * VB);
        const int c0 = ch * kAvc;
        const int cend = min(c0 + kAvc, lim_max);
        for (int c8 = c0; c8 < cend; c8 += 8) {
            const int c = c8 + 2 * lp;  // buffer rows past cend exist; the row limits mask them
            const float v0 = v_one<ADT>(B + (c - c0) * VB, j), v1 = v_one<ADT>(B + (c + 1 - c0) * VB, j);
            if (c + 1 < lim_all) {
                float2 sp[R];
#pragma unroll
                for (int i = 0; i < R; i++) sp[i] = *reinterpret_cast<const float2*>(S + i * mpad + c);
#pragma unroll
                for (int i = 0; i < R; i++) {
                    a[i][0] = sp[i].x * v0 + a[i][0];
                    a[i][1] = sp[i].y * v1 + a[i][1];
                }
                continue;
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int lim = min(start + qr0 + i + 1, n8);
                const float* Si = S + i * mpad;
                if (c < lim) a[i][0] = Si[c] * v0 + a[i][0];
                if (c + 1 < lim) a[i][1] = Si[c + 1] * v1 + a[i][1];
            }
        }
        if (ch + 1 < nch) {
            store_vc<ADT>(vch, Vb + ((ch + 1) & 1) * (kAvc * VB));
            if (ch + 2 < nch) load_vc<ADT>(vch, vc, v_pitch, kvd, g, ch + 2, m);
        }
        lds_barrier();
    }
    {
        const uint8_t* B = Vb + ((nch - 1) & 1) * (kAvc * VB);
        const int c0 = (nch - 1) * kAvc;
#pragma unroll
        for (int i = 0; i < R; i++) {
            // left-to-right lane sum through the quad: lp 0 holds lanes 0, 1,
            // lp 1 lanes 2, 3, ...
            float t = a[i][0] + a[i][1];
#pragma unroll
            for (int k = 1; k < 4; k++) {
                const float tin = dpp_f<0x90, 0xf, false>(t, t);  // quad_perm [0, 0, 1, 2]: lane lp reads lp - 1
                if (lp == k) t = (tin + a[i][0]) + a[i][1];
            }
            if (lp == 3 && i < nr) {
                // the tail [n8, n): within the last chunk, still in its buffer
                const int n = start + qr0 + i + 1;
                for (int c = n8; c < n; c++) t = t + S[i * mpad + c] * v_one<ADT>(B + (c - c0) * VB, j);
                outs[i][j] = t;
            }
        }
    }
    lds_barrier();
    for (int i = w; i < nr; i += kAttnThreads / kWave)
        act_store<ADT>(out + (size_t)(qr0 + i) * out_pitch, h * 64 + lane, qd, outs[i][lane], true);
}

// ---- launchers -------------------------------------------------------------

template <int ADT>
size_t attn_lds(int ctx)
{
    const size_t spad = ((size_t)ctx + kSsThreads - 1) & ~(size_t)(kSsThreads - 1);
    return (spad + 512) * 4 + 2 * (size_t)kAvc * v_stage_bytes<ADT>();
}

template <int ADT, int R>
size_t attn_rows_lds(int m)
{
    return (size_t)R * ((m + 3) & ~3) * 4 + 2 * (size_t)kAvc * v_stage_bytes<ADT>();
}

template <int ADT>
int attn_go(const uint8_t* q, int q_pitch, const uint8_t* kc, int k_pitch, const uint8_t* vc, int v_pitch,
            uint8_t* out, int out_pitch, int hq, int hkv, int start, int n_ctx, hipStream_t st, const int* dpos,
            int max_ctx)
{
    // with dpos the single query row and the context come from the device;
    // the shared memory is then sized for max_ctx positions
    const int rows = dpos ? 1 : n_ctx - start;
    const float scale = 1.0f / sqrtf(64.0f);
    if (!dpos && rows > 1) {
        // prefill: several query rows per workgroup, fewer for long rows
        // (their scores stay within 32 KB of shared memory)
        const int m = n_ctx;  // the last group attends at most n_ctx positions
        auto go_rows = [&](auto kern, size_t lds, int R) {
            const dim3 grid(hq, (rows + R - 1) / R);
            hipLaunchKernelGGL(kern, grid, dim3(kAttnThreads), lds, st, q, q_pitch, kc, k_pitch, vc, v_pitch, out,
                               out_pitch, hq, hkv, start, n_ctx, rows, scale);
            return launch_status("k_attn_rows");
        };
        // four rows per workgroup when eight would leave fewer than 1024
        // workgroups (64-row prompts: TinyLlama-Q4 prefill +4%, its fp16
        // rows +3%; Zephyr-Q4's 128 rows +4%, in on-box A/Bs; at MiniCPM's
        // 2,304 workgroups eight stay 1% ahead, and sixteen were 10% behind)
        const bool few = hq * ((rows + 7) / 8) < 1024;
        if (m <= 1024 && !few) return go_rows(k_attn_rows<ADT, 8>, attn_rows_lds<ADT, 8>(m), 8);
        if (m <= 2048) return go_rows(k_attn_rows<ADT, 4>, attn_rows_lds<ADT, 4>(m), 4);
        return go_rows(k_attn_rows<ADT, 2>, attn_rows_lds<ADT, 2>(m), 2);
    }
    const int lds_ctx = dpos ? max_ctx : n_ctx;
    hipLaunchKernelGGL(k_attn<ADT>, dim3(hq, rows), dim3(kAttnThreads), attn_lds<ADT>(lds_ctx), st, q, q_pitch, kc,
                       k_pitch, vc, v_pitch, out, out_pitch, hq, hkv, start, n_ctx, scale, dpos, lds_ctx);
    return launch_status("k_attn");
}

int attn_launch(int adt, const uint8_t* q, int q_pitch, const uint8_t* kc, int k_pitch, const uint8_t* vc, int v_pitch,
                uint8_t* out, int out_pitch, int hq, int hkv, int start, int n_ctx, hipStream_t st, const int* dpos,
                int max_ctx)
{
    const int rows = dpos ? 1 : n_ctx - start;
    if (rows <= 0) return NC_OK;
    if (hkv <= 0 || hq % hkv) return fail(NC_ERR_ARG, "qkv_attn: %d query heads over %d kv heads", hq, hkv);
    const int ctx = dpos ? max_ctx : n_ctx;
    if (ctx <= 0 || ctx > kAttnMaxCtx)
        return fail(NC_ERR_ARG, "qkv_attn: context %d (at most %d positions)", ctx, kAttnMaxCtx);
    if (adt == NC_Q8)
        return attn_go<Q8>(q, q_pitch, kc, k_pitch, vc, v_pitch, out, out_pitch, hq, hkv, start, n_ctx, st, dpos, max_ctx);
    if (adt == NC_F16)
        return attn_go<F16>(q, q_pitch, kc, k_pitch, vc, v_pitch, out, out_pitch, hq, hkv, start, n_ctx, st, dpos,
                            max_ctx);
    return fail(NC_ERR_ARG, "qkv_attn: activation dtype %d", adt);
}

}  // namespace nc

using namespace nc;

extern "C" int nc_qkv_attn(const nc_tensor* q, const nc_tensor* k, const nc_tensor* v, nc_tensor* out, int n_heads,
                           int n_kv_heads, int d_head, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(q && k && v && out && q->data && k->data && v->data && out->data, "qkv_attn: null tensor");
    NC_CHECK_ARG(d_head == 64, "qkv_attn: head size %d (the kernels are built for 64)", d_head);
    NC_CHECK_ARG(q->dtype == k->dtype && k->dtype == v->dtype && v->dtype == out->dtype,
                 "qkv_attn: dtypes differ");  // the reference's assert, gten/ops.cpp:1216
    NC_CHECK_ARG(q->cols == n_heads * 64 && k->cols == n_kv_heads * 64 && v->cols == k->cols && out->cols == q->cols,
                 "qkv_attn: widths do not match the head counts");
    NC_CHECK_ARG(start >= 0 && start <= n_ctx && n_ctx <= k->rows && n_ctx <= v->rows && n_ctx <= q->rows &&
                     n_ctx <= out->rows,
                 "qkv_attn: rows [%d, %d)", start, n_ctx);
    return attn_launch(q->dtype, (const uint8_t*)q->data + (size_t)start * q->pitch, q->pitch,
                       (const uint8_t*)k->data, k->pitch, (const uint8_t*)v->data, v->pitch,
                       (uint8_t*)out->data + (size_t)start * out->pitch, out->pitch, n_heads, n_kv_heads, start, n_ctx,
                       stream_of(stream), nullptr, n_ctx);
}
