// nc_attention.hip -- causal GQA attention over the HBM-resident KV cache.
//
// Replaces qkv_attn -> qk_masked_softmax -> transpose_v -> qkv_matmul
// (gten/ops.cpp:1017-1220).  One workgroup per (query head, query row):
//   s_c  = dot(q_h, k_{c,g}) * (1/sqrtf(d_head)) for c <= row, -inf after,
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
// The K and V caches are the K/V Linear outputs (rows = positions) in the
// activation dtype, as the reference keeps them (gten/modules.cpp:78-87).
#include "nc_act.h"
#include "nc_kernels.h"

namespace nc {

__device__ __forceinline__ uint32_t pick_pair2(uint32_t lo, uint32_t hi, int odd)
{
    return odd ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
}

// Lane-permuted dwords of one 32-code block (see nc_matvec.hip).
__device__ __forceinline__ void lane_dwords(const uint8_t* codes, uint32_t xa[4], uint32_t xb[4])
{
    const uint4* p = reinterpret_cast<const uint4*>(codes);
    const uint4 a = p[0], b = p[1];
    const uint32_t X[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        xa[k] = pick_pair2(X[k >> 1], X[2 + (k >> 1)], k & 1);
        xb[k] = pick_pair2(X[4 + (k >> 1)], X[6 + (k >> 1)], k & 1);
    }
}

constexpr int kAttnThreads = 256;
constexpr int kAttnMaxV = 8;  // uint4 V-staging loads per thread prefetched into registers

// Bytes of one position's V head slice in shared memory: Q8 codes (64) +
// fp16 deltas (2 x 2) rounded to 16, or 64 fp16 values.
template <int ADT>
__host__ __device__ constexpr int v_stage_bytes()
{
    return ADT == Q8 ? 80 : 128;
}

template <int ADT>
__global__ __launch_bounds__(kAttnThreads) void k_attn(const uint8_t* __restrict__ q, int q_pitch,
                                                       const uint8_t* __restrict__ kc, int k_pitch,
                                                       const uint8_t* __restrict__ vc, int v_pitch,
                                                       uint8_t* __restrict__ out, int out_pitch, int hq, int hkv,
                                                       int start, int n_ctx, float scale,
                                                       const int* __restrict__ dpos)
{
    // decode under graph replay: one query row at the position held on the device
    if (dpos) {
        start = dpos[0];
        n_ctx = start + 1;
    }
    extern __shared__ __align__(16) float sm[];
    const int npad = (n_ctx + 3) & ~3;
    float* S = sm;                                                   // scores / probabilities
    float* red = S + npad;                                           // 64
    float* acc = red + 64;                                           // [8][64]
    uint8_t* Vs = reinterpret_cast<uint8_t*>(acc + 512);             // [n_ctx][v_stage_bytes]
    constexpr int VB = v_stage_bytes<ADT>();
    const int tid = threadIdx.x;
    const int h = blockIdx.x;
    const int qr = blockIdx.y;       // row within q / out (pointers start at row `start`)
    const int row = start + qr;      // absolute position of the query
    const int g = h / (hq / hkv);
    const int qcols = hq * 64, kvcols = hkv * 64;
    const int qd = act_delta_offset(qcols), kvd = act_delta_offset(kvcols);
    const uint8_t* qrow = q + (size_t)qr * q_pitch;

    // ---- V head slice: the first kAttnMaxV loads per thread are issued before
    // the scores and parked in shared memory after them; any rest follows
    constexpr int VPARTS = ADT == Q8 ? 4 : 8;  // 16-byte code/value loads per position
    const int vtotal = n_ctx * VPARTS;
    uint4 vreg[kAttnMaxV];
    uint32_t dreg[kAttnMaxV];
#pragma unroll
    for (int i = 0; i < kAttnMaxV; i++) {
        const int idx = tid + i * kAttnThreads;
        const int c = idx < vtotal ? idx / VPARTS : 0, part = idx % VPARTS;
        const uint8_t* vrow = vc + (size_t)c * v_pitch;
        vreg[i] = reinterpret_cast<const uint4*>(vrow + g * (ADT == Q8 ? 64 : 128))[part];
        dreg[i] = ADT == Q8 ? reinterpret_cast<const uint32_t*>(vrow + kvd)[g] : 0u;
    }

    // ---- scores
    if (ADT == Q8) {
        uint32_t qa[2][4], qb[2][4];
        float dq[2];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            lane_dwords(qrow + h * 64 + b * 32, qa[b], qb[b]);
            dq[b] = h2f(reinterpret_cast<const uint16_t*>(qrow + qd)[h * 2 + b]);
        }
        for (int c = tid; c < n_ctx; c += kAttnThreads) {
            float s = -INFINITY;
            if (c <= row) {
                const uint8_t* krow = kc + (size_t)c * k_pitch;
                float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    uint32_t ka[4], kb[4];
                    lane_dwords(krow + g * 64 + b * 32, ka, kb);
                    const float dd = dq[b] * h2f(reinterpret_cast<const uint16_t*>(krow + kvd)[g * 2 + b]);
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        int L = __builtin_amdgcn_sdot4((int)qa[b][k], (int)ka[k], 0, false);
                        L = __builtin_amdgcn_sdot4((int)qb[b][k], (int)kb[k], L, false);
                        a4[k] = a4[k] + (float)L * dd;
                    }
                }
                s = ((a4[0] + a4[1]) + (a4[2] + a4[3])) * scale;
            }
            S[c] = s;
        }
    } else {
        float qv[64];
        const uint16_t* qh = reinterpret_cast<const uint16_t*>(qrow) + h * 64;
#pragma unroll
        for (int e = 0; e < 64; e++) qv[e] = h2f(qh[e]);
        for (int c = tid; c < n_ctx; c += kAttnThreads) {
            float s = -INFINITY;
            if (c <= row) {
                const uint16_t* kh = reinterpret_cast<const uint16_t*>(kc + (size_t)c * k_pitch) + g * 64;
                float a8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int m = 0; m < 8; m++)
#pragma unroll
                    for (int j = 0; j < 8; j++) a8[j] = __builtin_fmaf(qv[8 * m + j], h2f(kh[8 * m + j]), a8[j]);
                s = a8[0] + a8[1] + a8[2] + a8[3] + a8[4] + a8[5] + a8[6] + a8[7];
                s = s * scale;
            }
            S[c] = s;
        }
    }
#pragma unroll
    for (int i = 0; i < kAttnMaxV; i++) {
        const int idx = tid + i * kAttnThreads;
        if (idx < vtotal) {
            const int c = idx / VPARTS, part = idx % VPARTS;
            reinterpret_cast<uint4*>(Vs + (size_t)c * VB)[part] = vreg[i];
            if (ADT == Q8 && part == 0) reinterpret_cast<uint32_t*>(Vs + (size_t)c * VB + 64)[0] = dreg[i];
        }
    }
    for (int idx = tid + kAttnMaxV * kAttnThreads; idx < vtotal; idx += kAttnThreads) {
        const int c = idx / VPARTS, part = idx % VPARTS;
        const uint8_t* vrow = vc + (size_t)c * v_pitch;
        reinterpret_cast<uint4*>(Vs + (size_t)c * VB)[part] =
            reinterpret_cast<const uint4*>(vrow + g * (ADT == Q8 ? 64 : 128))[part];
        if (ADT == Q8 && part == 0)
            reinterpret_cast<uint32_t*>(Vs + (size_t)c * VB + 64)[0] = reinterpret_cast<const uint32_t*>(vrow + kvd)[g];
    }
    __syncthreads();

    // ---- softmax: max (order-free), expf, sequential sum, divide, requantize
    float mx = -INFINITY;
    for (int c = tid; c < n_ctx; c += kAttnThreads) mx = fmaxf(mx, S[c]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int c = tid; c < n_ctx; c += kAttnThreads) S[c] = expf_ref(S[c] - mx);
    __syncthreads();
    if (tid < kWave) {
        const float sum = seq_sum(S, n_ctx);
        if (tid == 0) red[8] = sum;
    }
    __syncthreads();
    const float sum = red[8];
    // every thread walks its positions in 32-lane blocks; lanes past n_ctx
    // still take part in the block reduction with valid = false
    for (int c0 = 0; c0 < n_ctx; c0 += kAttnThreads) {
        const int c = c0 + tid;
        const bool valid = c < n_ctx;
        const float p = valid ? S[c] / sum : 0.0f;
        const float pr = act_roundtrip<ADT>(p, valid);
        if (valid) S[c] = pr;
    }
    __syncthreads();

    // ---- P @ V from shared memory: thread = (column j, lanes l0, l0 + 1)
    const int j = tid & 63;
    auto vval = [&](int c) -> float {
        const uint8_t* vr = Vs + (size_t)c * VB;
        if (ADT == Q8)
            return (float)reinterpret_cast<const int8_t*>(vr)[j] * h2f(reinterpret_cast<const uint16_t*>(vr + 64)[j >> 5]);
        return h2f(reinterpret_cast<const uint16_t*>(vr)[j]);
    };
    {
        const int l0 = (tid >> 6) * 2;
        const int n8 = (n_ctx / 8) * 8;
#pragma unroll
        for (int li = 0; li < 2; li++) {
            const int l = l0 + li;
            float a = 0.0f;
            for (int c = l; c < n8; c += 8) a = S[c] * vval(c) + a;  // positions in order
            acc[l * 64 + j] = a;
        }
    }
    __syncthreads();
    if (tid < 64) {
        float s = acc[j];
#pragma unroll
        for (int l = 1; l < 8; l++) s = s + acc[l * 64 + j];
        for (int c = (n_ctx / 8) * 8; c < n_ctx; c++) s = s + S[c] * vval(c);
        act_store<ADT>(out + (size_t)qr * out_pitch, h * 64 + j, qd, s, true);
    }
}

// Prefill: kArRows consecutive query rows of one head per workgroup, with
// the same arithmetic as k_attn.  The V slice and every K row are read once
// for all of them, and each row stops at its own position: past it the
// reference's probabilities are exact zeros (expf(-inf) = 0, requantized to
// 0), so they add nothing to the sequential softmax sum, to the absmax of
// their 32-position blocks, or to the P.V lane chains (each starts at +0,
// and adding +/-0 leaves a running sum unchanged, its sign included).
constexpr int kArRows = 8;

template <int ADT>
__global__ __launch_bounds__(kAttnThreads) void k_attn_rows(const uint8_t* __restrict__ q, int q_pitch,
                                                            const uint8_t* __restrict__ kc, int k_pitch,
                                                            const uint8_t* __restrict__ vc, int v_pitch,
                                                            uint8_t* __restrict__ out, int out_pitch, int hq, int hkv,
                                                            int start, int n_ctx, int rows, float scale)
{
    extern __shared__ __align__(16) float sm[];
    __shared__ float outs[kArRows][64];
    constexpr int VB = v_stage_bytes<ADT>();
    constexpr int VPARTS = ADT == Q8 ? 4 : 8;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = blockIdx.x, qr0 = blockIdx.y * kArRows;
    const int nr = min(kArRows, rows - qr0);
    const int m = start + qr0 + nr;  // positions attended by any of the rows
    const int mpad = (m + 3) & ~3;
    float* S = sm;                                                  // [kArRows][mpad]
    uint8_t* Vs = reinterpret_cast<uint8_t*>(S + kArRows * mpad);   // [m][VB]
    const int g = h / (hq / hkv);
    const int qcols = hq * 64, kvcols = hkv * 64;
    const int qd = act_delta_offset(qcols), kvd = act_delta_offset(kvcols);

    // ---- V head slice of positions [0, m)
    for (int idx = tid; idx < m * VPARTS; idx += kAttnThreads) {
        const int c = idx / VPARTS, part = idx % VPARTS;
        const uint8_t* vrow = vc + (size_t)c * v_pitch;
        reinterpret_cast<uint4*>(Vs + (size_t)c * VB)[part] =
                reinterpret_cast<const uint4*>(vrow + g * (ADT == Q8 ? 64 : 128))[part];
        if (ADT == Q8 && part == 0)
            reinterpret_cast<uint32_t*>(Vs + (size_t)c * VB + 64)[0] = reinterpret_cast<const uint32_t*>(vrow + kvd)[g];
    }

    // ---- scores: thread = (row i, positions c0 + 32 k); the eight rows
    // sharing a position read its K row together
    {
        const int i = tid & (kArRows - 1);
        const int ic = min(i, nr - 1);
        const int row = start + qr0 + i;  // absolute position of the query
        const uint8_t* qrow = q + (size_t)(qr0 + ic) * q_pitch;
        if (ADT == Q8) {
            uint32_t qa[2][4], qb[2][4];
            float dq[2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                lane_dwords(qrow + h * 64 + b * 32, qa[b], qb[b]);
                dq[b] = h2f(reinterpret_cast<const uint16_t*>(qrow + qd)[h * 2 + b]);
            }
            for (int c = tid / kArRows; c < m; c += kAttnThreads / kArRows) {
                if (i < nr && c <= row) {
                    const uint8_t* krow = kc + (size_t)c * k_pitch;
                    float a4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int b = 0; b < 2; b++) {
                        uint32_t ka[4], kb[4];
                        lane_dwords(krow + g * 64 + b * 32, ka, kb);
                        const float dd = dq[b] * h2f(reinterpret_cast<const uint16_t*>(krow + kvd)[g * 2 + b]);
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            int L = __builtin_amdgcn_sdot4((int)qa[b][k], (int)ka[k], 0, false);
                            L = __builtin_amdgcn_sdot4((int)qb[b][k], (int)kb[k], L, false);
                            a4[k] = a4[k] + (float)L * dd;
                        }
                    }
                    S[i * mpad + c] = ((a4[0] + a4[1]) + (a4[2] + a4[3])) * scale;
                }
            }
        } else {
            float qv[64];
            const uint16_t* qh = reinterpret_cast<const uint16_t*>(qrow) + h * 64;
#pragma unroll
            for (int e = 0; e < 64; e++) qv[e] = h2f(qh[e]);
            for (int c = tid / kArRows; c < m; c += kAttnThreads / kArRows) {
                if (i < nr && c <= row) {
                    const uint16_t* kh = reinterpret_cast<const uint16_t*>(kc + (size_t)c * k_pitch) + g * 64;
                    float a8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                    for (int mm = 0; mm < 8; mm++)
#pragma unroll
                        for (int j = 0; j < 8; j++) a8[j] = __builtin_fmaf(qv[8 * mm + j], h2f(kh[8 * mm + j]), a8[j]);
                    const float sc = a8[0] + a8[1] + a8[2] + a8[3] + a8[4] + a8[5] + a8[6] + a8[7];
                    S[i * mpad + c] = sc * scale;
                }
            }
        }
    }
    __syncthreads();

    // ---- softmax of row i on wave i % 4: max, expf, sequential sum over
    // [0, row], divide, requantize in 32-position blocks
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
    __syncthreads();

    // ---- P.V: thread = (column j, lanes 2 lp and 2 lp + 1) for every row;
    // row i's lane chains cover positions < min(n_i, n8), n8 = the call's
    // n_ctx rounded down to 8 (the reference's 8-lane part), then the lane
    // sums left to right across the quad and the tail positions in order
    {
        const int j = tid >> 2, lp = tid & 3;
        const int n8 = (n_ctx / 8) * 8;
        auto vval = [&](int c) -> float {
            const uint8_t* vr = Vs + (size_t)c * VB;
            if (ADT == Q8)
                return (float)reinterpret_cast<const int8_t*>(vr)[j] * h2f(reinterpret_cast<const uint16_t*>(vr + 64)[j >> 5]);
            return h2f(reinterpret_cast<const uint16_t*>(vr)[j]);
        };
        float a[kArRows][2];
#pragma unroll
        for (int i = 0; i < kArRows; i++) a[i][0] = a[i][1] = 0.0f;
        const int lim_max = min(m, n8);
        for (int c8 = 0; c8 < lim_max; c8 += 8) {
            const int c = c8 + 2 * lp;
            const float v0 = vval(min(c, m - 1)), v1 = vval(min(c + 1, m - 1));
#pragma unroll
            for (int i = 0; i < kArRows; i++) {
                const int lim = min(start + qr0 + i + 1, n8);
                const float* Si = S + i * mpad;
                if (c < lim) a[i][0] = Si[c] * v0 + a[i][0];
                if (c + 1 < lim) a[i][1] = Si[c + 1] * v1 + a[i][1];
            }
        }
#pragma unroll
        for (int i = 0; i < kArRows; i++) {
            // left-to-right lane sum through the quad: lp 0 holds lanes 0, 1,
            // lp 1 lanes 2, 3, ...
            float t = a[i][0] + a[i][1];
#pragma unroll
            for (int k = 1; k < 4; k++) {
                const float tin = dpp_f<0x90, 0xf, false>(t, t);  // quad_perm [0, 0, 1, 2]: lane lp reads lp - 1
                if (lp == k) t = (tin + a[i][0]) + a[i][1];
            }
            if (lp == 3 && i < nr) {
                const int n = start + qr0 + i + 1;
                for (int c = n8; c < n; c++) t = t + S[i * mpad + c] * vval(c);
                outs[i][j] = t;
            }
        }
    }
    __syncthreads();
    for (int i = w; i < nr; i += kAttnThreads / kWave)
        act_store<ADT>(out + (size_t)(qr0 + i) * out_pitch, h * 64 + lane, qd, outs[i][lane], true);
}

int attn_launch(int adt, const uint8_t* q, int q_pitch, const uint8_t* kc, int k_pitch, const uint8_t* vc, int v_pitch,
                uint8_t* out, int out_pitch, int hq, int hkv, int start, int n_ctx, hipStream_t st, const int* dpos,
                int max_ctx)
{
    // with dpos the single query row and the context come from the device;
    // n_ctx then only bounds the shared-memory size (max_ctx)
    const int rows = dpos ? 1 : n_ctx - start;
    if (rows <= 0) return NC_OK;
    if (hkv <= 0 || hq % hkv) return fail(NC_ERR_ARG, "qkv_attn: %d query heads over %d kv heads", hq, hkv);
    const float scale = 1.0f / sqrtf(64.0f);
    const int lds_ctx = dpos ? max_ctx : n_ctx;
    const int vb = adt == NC_Q8 ? v_stage_bytes<Q8>() : v_stage_bytes<F16>();
    const size_t lds = ((size_t)((lds_ctx + 3) & ~3) + 64 + 512) * 4 + (size_t)lds_ctx * vb;
    if (lds > 64 * 1024) return fail(NC_ERR_ARG, "qkv_attn: context %d too long", lds_ctx);
    // prefill: several query rows per workgroup when their shared memory fits
    if (!dpos && rows > 1) {
        const int m = n_ctx;  // the last group attends at most n_ctx positions
        const size_t lds_r = (size_t)kArRows * ((m + 3) & ~3) * 4 + (size_t)m * vb;
        if (lds_r <= 64 * 1024) {
            const dim3 grid_r(hq, (rows + kArRows - 1) / kArRows);
            if (adt == NC_Q8)
                hipLaunchKernelGGL((k_attn_rows<Q8>), grid_r, dim3(kAttnThreads), lds_r, st, q, q_pitch, kc, k_pitch, vc,
                                   v_pitch, out, out_pitch, hq, hkv, start, n_ctx, rows, scale);
            else if (adt == NC_F16)
                hipLaunchKernelGGL((k_attn_rows<F16>), grid_r, dim3(kAttnThreads), lds_r, st, q, q_pitch, kc, k_pitch, vc,
                                   v_pitch, out, out_pitch, hq, hkv, start, n_ctx, rows, scale);
            else
                return fail(NC_ERR_ARG, "qkv_attn: activation dtype %d", adt);
            return launch_status("k_attn_rows");
        }
    }
    const dim3 grid(hq, rows);
    if (adt == NC_Q8)
        hipLaunchKernelGGL((k_attn<Q8>), grid, dim3(kAttnThreads), lds, st, q, q_pitch, kc, k_pitch, vc, v_pitch, out, out_pitch,
                           hq, hkv, start, n_ctx, scale, dpos);
    else if (adt == NC_F16)
        hipLaunchKernelGGL((k_attn<F16>), grid, dim3(kAttnThreads), lds, st, q, q_pitch, kc, k_pitch, vc, v_pitch, out, out_pitch,
                           hq, hkv, start, n_ctx, scale, dpos);
    else
        return fail(NC_ERR_ARG, "qkv_attn: activation dtype %d", adt);
    return launch_status("k_attn");
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
