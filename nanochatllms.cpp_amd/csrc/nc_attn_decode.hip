// nc_attn_decode.hip -- single-row decode attention with the q/k/v post-
// processing fused in (Q8 activations; the fp16 kernel below).
//
// One workgroup per query head h (group g = h / (hq / hkv)) does what
// k_qkv_post + k_attn do for the decode row, with the same arithmetic:
//   q_h, k_g, v_g from the fused qkv matvec output: requantized as Linear
//     outputs; Zephyr's biases added (requantized); OpenELM's per-head QK
//     RMSNorm (requantized); RoPE of q and k
//     (requantized when stored) -- gten/modules.cpp:242-267, openelm.cpp:33-60;
//   the group's first head appends k_g and v_g to the caches at the position
//     (the others take that position from shared memory, so no workgroup
//     waits for another);
//   scores, softmax (max, expf, sequential sum, divide, requantize per 32
//     positions) and P.V as qkv_attn (gten/ops.cpp:1017-1220): the Q8 dot's
//     four lane sums per block, P.V as eight fp32 lanes (position mod 8)
//     summed left to right, then the n mod 8 tail.
// Any context up to kAttnMaxCtx positions: the scores sit in shared memory
// and the K rows are read straight into registers (the next row requested
// before the current one is used).  For caches of up to kAdResMax positions
// the whole V slice is staged into shared memory while the scores run, in a
// layout where one dword read gives a lane chain four positions' codes and
// one 16-byte read four positions' deltas or probabilities, so the P.V lane
// chains then run without a barrier.  Longer caches stream the V slice
// through shared memory in double-buffered chunks of kAdVc positions.  The softmax denominator of a long row is the
// exact workgroup-parallel restatement of the sequential sum (nc_seqsum.h);
// short rows take the plain loop on one wavefront.
#include <type_traits>

#include "nc_act.h"
#include "nc_kernels.h"
#include "nc_seqsum.h"

namespace nc {

// f(0), f(1), ..., f(N - 1) with compile-time indices (register arrays stay
// in registers even where a plain loop would not be unrolled).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

constexpr int kAdThreads = 512;
constexpr int kAdMaxK = 2;      // K rows per thread requested at kernel start, at most
constexpr int kAdVB = 80;       // LDS bytes per staged V position: 64 codes, 2 fp16 deltas, pad
constexpr int kAdVc = 128;      // positions per staged V chunk (2 16-byte parts per thread)
constexpr int kAdSeqMax = 1024; // softmax rows up to this long are summed by one wavefront's loop
constexpr int kAdResMax = 1024; // caches up to this long hold the whole V slice in shared memory
// s_waitcnt immediate that waits for every vector memory load (vmcnt 0) and
// leaves the export and LDS/scalar counters alone (expcnt 7, lgkmcnt 15).
constexpr int kVmcnt0 = 0x0F70;

__device__ __forceinline__ uint32_t ad_pick(uint32_t lo, uint32_t hi, int odd)
{
    return odd ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
}

// The Q8 dot of two 64-value heads as vec_dot_product_q8 (gten/ops.cpp:
// 292-384) computes it: per 32-block four int32 lane sums, fp32 terms
// folded block by block, (a0 + a1) + (a2 + a3).  Codes as 4 uint4 per head.
__device__ __forceinline__ float head_dot_q8(const uint4 (&a)[4], const float (&da)[2], const uint4 (&b)[4],
                                             const float (&db)[2])
{
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
        const uint32_t A[8] = {a[2 * blk].x, a[2 * blk].y, a[2 * blk].z, a[2 * blk].w,
                               a[2 * blk + 1].x, a[2 * blk + 1].y, a[2 * blk + 1].z, a[2 * blk + 1].w};
        const uint32_t B[8] = {b[2 * blk].x, b[2 * blk].y, b[2 * blk].z, b[2 * blk].w,
                               b[2 * blk + 1].x, b[2 * blk + 1].y, b[2 * blk + 1].z, b[2 * blk + 1].w};
        const float dd = da[blk] * db[blk];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // elements {2k, 2k+1, 2k+8, 2k+9} and the same + 16: lane k of the AVX dot
            const uint32_t xa = ad_pick(A[k >> 1], A[2 + (k >> 1)], k & 1);
            const uint32_t xb = ad_pick(A[4 + (k >> 1)], A[6 + (k >> 1)], k & 1);
            const uint32_t ya = ad_pick(B[k >> 1], B[2 + (k >> 1)], k & 1);
            const uint32_t yb = ad_pick(B[4 + (k >> 1)], B[6 + (k >> 1)], k & 1);
            int L = __builtin_amdgcn_sdot4((int)xa, (int)ya, 0, false);
            L = __builtin_amdgcn_sdot4((int)xb, (int)yb, L, false);
            acc[k] = acc[k] + (float)L * dd;
        }
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// Wavefront maximum: DPP within 16-lane rows, then the four row results.
__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f<kDppQuadXor1, 0xf, false>(v, v));
    v = fmaxf(v, dpp_f<kDppQuadXor2, 0xf, false>(v, v));
    v = fmaxf(v, dpp_f<0x141, 0xf, false>(v, v));
    v = fmaxf(v, dpp_f<0x140, 0xf, false>(v, v));
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// A K row's 64 codes and its two fp16 deltas (as one dword).
struct KRow {
    uint4 q[4];
    uint32_t d;
};

__device__ __forceinline__ KRow load_krow(const uint8_t* kslice, const uint8_t* kdelta, int c, int kv_pitch, int g)
{
    KRow r;
    const uint4* p = reinterpret_cast<const uint4*>(kslice + (size_t)c * kv_pitch);
#pragma unroll
    for (int v = 0; v < 4; v++) r.q[v] = p[v];
    r.d = reinterpret_cast<const uint32_t*>(kdelta + (size_t)c * kv_pitch)[g];
    return r;
}

__device__ __forceinline__ float score_of(const uint4 (&qv)[4], const float (&dq)[2], const KRow& k)
{
    const float dk[2] = {h2f((uint16_t)(k.d & 0xFFFFu)), h2f((uint16_t)(k.d >> 16))};
    return head_dot_q8(qv, dq, k.q, dk);
}

// The V parts of one chunk a thread carries: 16-byte parts tid + i
// kAdThreads (position = part / 4 within the chunk), and the delta dword of
// position tid (threads below kAdVc).
constexpr int kAdVParts = kAdVc * 4 / kAdThreads;
static_assert(kAdVParts >= 1 && kAdVParts * kAdThreads == kAdVc * 4 && kAdVc <= kAdThreads, "V chunk parts");
struct VChunk {
    uint32_t p[kAdVParts][4];  // plain words: an array of the uint4 union type stays in scratch memory
    uint32_t d;
};

// Loads chunk `ch`; positions are clamped to the cache's rows (those past the
// context are never read back).
__device__ __forceinline__ void load_vchunk(VChunk& v, const uint8_t* vslice, const uint8_t* vdelta, int ch,
                                            int kv_pitch, int g, int kv_rows)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAdVParts; i++) {
        const int idx = tid + i * kAdThreads;
        const int c = min(ch * kAdVc + (idx >> 2), kv_rows - 1);
        const uint4 t4 = reinterpret_cast<const uint4*>(vslice + (size_t)c * kv_pitch)[idx & 3];
        v.p[i][0] = t4.x;
        v.p[i][1] = t4.y;
        v.p[i][2] = t4.z;
        v.p[i][3] = t4.w;
    }
    const int c = min(ch * kAdVc + (tid & (kAdVc - 1)), kv_rows - 1);
    v.d = reinterpret_cast<const uint32_t*>(vdelta + (size_t)c * kv_pitch)[g];
}

// Parks a loaded chunk in a shared-memory buffer [kAdVc][kAdVB]; the new
// position `pos` (not yet in the cache for every head) comes from s_v.
__device__ __forceinline__ void store_vchunk(const VChunk& v, uint8_t* buf, int ch, int pos, const uint8_t* s_v)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAdVParts; i++) {
        const int idx = tid + i * kAdThreads;
        const int cl = idx >> 2, part = idx & 3;
        uint4 t4 = make_uint4(v.p[i][0], v.p[i][1], v.p[i][2], v.p[i][3]);
        if (ch * kAdVc + cl == pos) t4 = reinterpret_cast<const uint4*>(s_v)[part];
        reinterpret_cast<uint4*>(buf + cl * kAdVB)[part] = t4;
    }
    if (tid < kAdVc) {
        uint32_t d = v.d;
        if (ch * kAdVc + tid == pos) d = reinterpret_cast<const uint32_t*>(s_v + 64)[0];
        reinterpret_cast<uint32_t*>(buf + tid * kAdVB + 64)[0] = d;
    }
}

// MK K rows per thread are requested into registers at the start (every
// slot, so the load counts are static and the waits exact); later rows are
// read in the score loop, one row ahead.  The launcher sizes MK to the cache:
// issuing the loads is itself a cost.  VP > 0: the V slice of the positions
// < n is resident in shared memory (the cache holds at most VP rows); VP == 0
// streams it in chunks.
//
// Resident layout (VP > 0): positions c = 32 k4 + 8 j + l (lane l = c mod 8
// of the P.V chains, k4 = c / 32, j = (c / 8) mod 4):
//   codes   [l][k4][column 64] dwords, byte j = the code at position c;
//   deltas  [block 2][l][VP / 8] fp32, entry c / 8;
//   P       [l][sT] fp32 (the probabilities, entry c / 8).
template <bool QKNORM, bool BIAS, int MK, int VP>
__global__ __launch_bounds__(kAdThreads) void k_attn_dec(const float* __restrict__ raw, int hq, int hkv,
                                                         const uint16_t* __restrict__ bq,
                                                         const uint16_t* __restrict__ bk,
                                                         const uint16_t* __restrict__ bv,
                                                         const uint16_t* __restrict__ qn_w,
                                                         const uint16_t* __restrict__ kn_w,
                                                         const float2* __restrict__ table, int d_half, int pos_host,
                                                         const int* __restrict__ dpos, uint8_t* __restrict__ kc,
                                                         uint8_t* __restrict__ vc, int kv_pitch,
                                                         uint8_t* __restrict__ out, float scale,
                                                         const float2* __restrict__ rope_cur, int kv_rows)
{
    extern __shared__ __align__(16) float sm[];
    __shared__ __align__(16) uint8_t s_q[kAdVB], s_k[kAdVB], s_v[kAdVB];
    __shared__ __align__(16) float s_nrm[2][64];
    __shared__ float red[kAdThreads / kWave];
    __shared__ float s_sum;
    __shared__ SsShared ssh;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // workgroup i runs on XCD i % 8: with hq % 8 == 0, XCD x takes heads
    // x * hq/8 .. (x + 1) * hq/8 - 1, so the query heads of one kv head share
    // an XCD and its L2 fetches their K/V slice once (a bijection on [0, hq))
    const int h = hq % 8 == 0 ? (int)(blockIdx.x % 8) * (hq / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int gs = hq / hkv, g = h / gs;
    // this wave's raw q / k / v value does not depend on the position: it is
    // requested before the position is known
    const int col = w == 0 ? h * 64 : (w == 1 ? hq * 64 + g * 64 : hq * 64 + hkv * 64 + g * 64);
    const float raw_x = w < 3 ? raw[col + lane] : 0.0f;
    // the Linear's bias of this value (Zephyr's q/k/v projections)
    uint16_t bias16 = 0;
    if (BIAS && w < 3) bias16 = (w == 0 ? bq + h * 64 : (w == 1 ? bk : bv) + g * 64)[lane];
    // the lane's RoPE pair (q and k waves) is requested before the K / V
    // rows: the vector memory counter completes in order, so a pair
    // requested after them would be waited for together with all of them
    const int pair = lane < d_half ? lane : lane - d_half;
    const bool rope_lane_in = w < 2 && lane < 2 * d_half;
    float2 rp = make_float2(0.0f, 0.0f);
    if (rope_cur && rope_lane_in) rp = rope_cur[pair];
    const int kvd = act_delta_offset(hkv * 64);
    const uint8_t* kslice = kc + g * 64;
    const uint8_t* vslice = vc + g * 64;
    // the first V chunk does not depend on the position either
    constexpr bool kRes = VP > 0;
    static_assert(VP % 32 == 0 && VP <= kAdResMax, "resident V: whole 32-position groups");
    VChunk vch;
    if constexpr (!kRes) load_vchunk(vch, vslice, vc + kvd, 0, kv_pitch, g, kv_rows);
    const int pos = dpos ? load_pos(dpos) : pos_host;
    if (!rope_cur && rope_lane_in) rp = table[(size_t)pos * d_half + pair];
    __builtin_amdgcn_sched_barrier(0);
    const int n = pos + 1;
    // shared memory: scores [spad] (whole 256-position chunks, zero-padded
    // for the block sum); resident V: P [8][sT], P.V lane sums [8][64], codes,
    // deltas; streamed V: P.V lane sums, two V chunk buffers
    const int spad = (kv_rows + kSsThreads - 1) & ~(kSsThreads - 1);
    const int sT = spad / 8 + 4;  // padded: the transposed P stores hit distinct banks
    float* S = sm;
    float* PT = S + spad;
    float* acc = kRes ? PT + 8 * sT : S + spad;
    uint8_t* Vb = reinterpret_cast<uint8_t*>(acc + 512);
    uint32_t* CT = reinterpret_cast<uint32_t*>(acc + 512);
    float* DT = reinterpret_cast<float*>(CT + VP * 16);
    constexpr int K4 = VP / 32, TPT = (VP + kAdThreads - 1) / kAdThreads;

    // ---- K rows (positions < pos) into registers
    KRow kr[MK];
    static_for<0, MK>([&](auto I) {
        const int c = tid + I * kAdThreads;
        kr[I] = load_krow(kslice, kc + kvd, c < pos ? c : 0, kv_pitch, g);
    });

    // ---- q_h (wave 0), k_g (wave 1), v_g (wave 2) of the new position
    if (w < 3) {
        float x = q8_roundtrip_lane(raw_x, true);  // the Linear output as stored
        // + bias, stored (bias_add_inplace, gten/ops.cpp:639-666)
        if (BIAS) x = q8_roundtrip_lane(x + h2f(bias16), true);
        if (w < 2) {
            if (QKNORM) {
                // RMSNorm3D over the head (rms_norm_vec_f32, gten/ops.cpp:830-903)
                float* buf = s_nrm[w];
                buf[lane] = x * x;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
                const float rms = sqrtf(seq_sum(buf, 64) / 64.0f);
                x = q8_roundtrip_lane(x / (rms + 1e-6f) * h2f((w == 0 ? qn_w : kn_w)[lane]), true);
            }
            x = rope_lane_pair(x, lane, d_half, rp);
        }
        uint16_t d16;
        const int8_t code = q8_quant_lane(x, true, &d16);
        uint8_t* st = w == 0 ? s_q : (w == 1 ? s_k : s_v);
        st[lane] = (uint8_t)code;
        if ((lane & 31) == 0) reinterpret_cast<uint16_t*>(st + 64)[lane >> 5] = d16;
        if (w > 0 && h % gs == 0) {
            // the group's first head appends the new K / V row to the cache
            uint8_t* row = (w == 1 ? kc : vc) + (size_t)pos * kv_pitch;
            row[g * 64 + lane] = (uint8_t)code;
            if ((lane & 31) == 0) reinterpret_cast<uint16_t*>(row + kvd)[g * 2 + (lane >> 5)] = d16;
        }
    }
    // resident V: the rows of positions < n requested (after this wave's
    // q/k/v work, so that work is not queued behind them).  Item t =
    // (k4, l, part q) covers rows 32 k4 + l + {0, 8, 16, 24}, bytes 16 q..
    uint32_t vw[kRes ? TPT : 1][4][4];
    uint32_t vd[kRes ? TPT : 1];
    if constexpr (kRes) {
        static_for<0, TPT>([&](auto T) {
            const int t = tid + T * kAdThreads;
            const int q = t & 3, l = (t >> 2) & 7, k4 = t >> 5;
            if (t < VP && 32 * k4 + l < n) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int c = min(32 * k4 + 8 * j + l, kv_rows - 1);
                    const uint4 x = reinterpret_cast<const uint4*>(vslice + (size_t)c * kv_pitch)[q];
                    vw[T][j][0] = x.x;
                    vw[T][j][1] = x.y;
                    vw[T][j][2] = x.z;
                    vw[T][j][3] = x.w;
                }
            }
            if (t < n) vd[T] = reinterpret_cast<const uint32_t*>(vc + kvd + (size_t)t * kv_pitch)[g];
        });
    }
    lds_barrier();

    // streamed V: the first chunk into buffer 0; the second one requested
    const int nch = (n + kAdVc - 1) / kAdVc;
    if constexpr (!kRes) {
        store_vchunk(vch, Vb, 0, pos, s_v);
        if (nch > 1) load_vchunk(vch, vslice, vc + kvd, 1, kv_pitch, g, kv_rows);
    }

    // ---- scores of positions c <= pos (thread = position)
    {
        uint4 qv[4];
        float dq[2];
#pragma unroll
        for (int v = 0; v < 4; v++) qv[v] = reinterpret_cast<const uint4*>(s_q)[v];
        dq[0] = h2f(reinterpret_cast<const uint16_t*>(s_q + 64)[0]);
        dq[1] = h2f(reinterpret_cast<const uint16_t*>(s_q + 64)[1]);
        static_for<0, MK>([&](auto I) {
            const int c = tid + I * kAdThreads;
            if (c < pos) S[c] = score_of(qv, dq, kr[I]) * scale;
        });
        int c = tid + MK * kAdThreads;
        if (c < pos) {
            KRow cur = load_krow(kslice, kc + kvd, c, kv_pitch, g);
            for (;;) {
                const int cn = c + kAdThreads;
                KRow nxt = cur;
                if (cn < pos) nxt = load_krow(kslice, kc + kvd, cn, kv_pitch, g);
                S[c] = score_of(qv, dq, cur) * scale;
                if (cn >= pos) break;
                cur = nxt;
                c = cn;
            }
        }
        if (tid == (pos & (kAdThreads - 1))) {
            KRow kk;
#pragma unroll
            for (int v = 0; v < 4; v++) kk.q[v] = reinterpret_cast<const uint4*>(s_k)[v];
            kk.d = reinterpret_cast<const uint32_t*>(s_k + 64)[0];
            S[pos] = score_of(qv, dq, kk) * scale;
        }
    }
    if constexpr (kRes) {
        // ---- resident V into shared memory: four rows' dwords transposed so
        // each output dword holds one column at four positions of a chain;
        // the new position's row comes from s_v.  Every vector load is waited
        // for here: the compiler cannot tell which are still in flight past
        // the divergent score branches, and would otherwise wait inside the
        // P.V loop.
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        static_for<0, TPT>([&](auto T) {
            const int t = tid + T * kAdThreads;
            const int q = t & 3, l = (t >> 2) & 7, k4 = t >> 5;
            if (t < VP && 32 * k4 + l < n) {
                uint32_t r[4][4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const bool cur = 32 * k4 + 8 * j + l == pos;
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        r[j][i] = cur ? reinterpret_cast<const uint32_t*>(s_v)[4 * q + i] : vw[T][j][i];
                }
                uint4* dst = reinterpret_cast<uint4*>(CT + (l * K4 + k4) * 64 + 16 * q);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t lo01 = __builtin_amdgcn_perm(r[1][i], r[0][i], 0x05010400u);
                    const uint32_t hi01 = __builtin_amdgcn_perm(r[1][i], r[0][i], 0x07030602u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(r[3][i], r[2][i], 0x05010400u);
                    const uint32_t hi23 = __builtin_amdgcn_perm(r[3][i], r[2][i], 0x07030602u);
                    dst[i] = make_uint4(__builtin_amdgcn_perm(lo23, lo01, 0x05040100u),
                                        __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                        __builtin_amdgcn_perm(hi23, hi01, 0x05040100u),
                                        __builtin_amdgcn_perm(hi23, hi01, 0x07060302u));
                }
            }
            if (t < n) {
                const uint32_t d = t == pos ? reinterpret_cast<const uint32_t*>(s_v + 64)[0] : vd[T];
                DT[(t & 7) * (VP / 8) + (t >> 3)] = h2f((uint16_t)(d & 0xFFFFu));
                DT[(8 + (t & 7)) * (VP / 8) + (t >> 3)] = h2f((uint16_t)(d >> 16));
            }
        });
    }
    lds_barrier();

    // ---- softmax: max (order-free), expf, sequential sum, divide, requantize
    float mx = -INFINITY;
    for (int c = tid; c < n; c += kAdThreads) mx = fmaxf(mx, S[c]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    lds_barrier();
    mx = red[0];
#pragma unroll
    for (int q = 1; q < kAdThreads / kWave; q++) mx = fmaxf(mx, red[q]);
    const bool long_row = n > kAdSeqMax;
    const int npad = (n + kSsThreads - 1) & ~(kSsThreads - 1);
    for (int c = tid; c < (long_row ? npad : n); c += kAdThreads) S[c] = c < n ? expf_ref(S[c] - mx) : 0.0f;
    lds_barrier();
    float sum;
    if (long_row) {
        // the exact parallel sum of the terms; the zero padding leaves a sum
        // of non-negative terms as it is
        sum = block_seq_sum_nonneg(S, npad, ssh);
    } else {
        if (w == 0) {
            const float ss = seq_sum(S, n);
            if (lane == 0) s_sum = ss;
        }
        lds_barrier();
        sum = s_sum;
    }
    for (int c0 = 0; c0 < n; c0 += kAdThreads) {
        const int c = c0 + tid;
        const bool valid = c < n;
        const float p = valid ? S[c] / sum : 0.0f;
        const float pr = q8_roundtrip_lane(p, valid);  // P stored as Act: 32-position blocks
        if (valid) {
            if constexpr (kRes) PT[(c & 7) * sT + (c >> 3)] = pr;
            else S[c] = pr;
        }
    }
    lds_barrier();

    // ---- P.V: thread = (lane l = tid / 64, column m = tid % 64): the chain
    // (l, m) over positions l, l + 8, ... in order.  Chunk ch sits in buffer
    // ch & 1 while chunk ch + 1 is parked in the other and chunk ch + 2 is
    // requested.
    static_assert(kAdThreads == 8 * 64, "one P.V chain per thread");
    const int l = tid >> 6, m = tid & 63;
    const int n8 = n & ~7;
    float a0 = 0.0f;
    if constexpr (kRes) {
        // the chain's positions l + 8 k, k < n8 / 8, four at a time: one
        // dword of codes, one 16-byte read each of deltas and P
        const int kn = n8 >> 3, ng = kn >> 2;
        const float* Pl = PT + l * sT;
        const uint32_t* Cl = CT + l * K4 * 64 + m;
        const float* Dl = DT + ((m >> 5) * 8 + l) * (VP / 8);
        auto four = [&](uint32_t cw, float4 d4, float4 p4) {
            const float dd[4] = {d4.x, d4.y, d4.z, d4.w};
            const float pp[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
            for (int j = 0; j < 4; j++) a0 = pp[j] * ((float)(int)(int8_t)(cw >> (8 * j)) * dd[j]) + a0;
        };
        int k4 = 0;
        for (; k4 + 4 <= ng; k4 += 4) {
            uint32_t cw[4];
            float4 d4[4], p4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                cw[u] = Cl[(k4 + u) * 64];
                d4[u] = reinterpret_cast<const float4*>(Dl)[k4 + u];
                p4[u] = reinterpret_cast<const float4*>(Pl)[k4 + u];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) four(cw[u], d4[u], p4[u]);
        }
        for (; k4 < ng; k4++)
            four(Cl[k4 * 64], reinterpret_cast<const float4*>(Dl)[k4], reinterpret_cast<const float4*>(Pl)[k4]);
        for (int k = ng * 4; k < kn; k++)
            a0 = Pl[k] * ((float)(int)(int8_t)(Cl[(k >> 2) * 64] >> (8 * (k & 3))) * Dl[k]) + a0;
    } else {
        for (int ch = 0; ch < nch; ch++) {
            const uint8_t* B = Vb + (ch & 1) * (kAdVc * kAdVB);
            const int c0 = ch * kAdVc;
            const int cend = min(c0 + kAdVc, n8);
            auto vone = [&](int c) {
                const uint8_t* vrow = B + (c - c0) * kAdVB;
                const float d = h2f(reinterpret_cast<const uint16_t*>(vrow + 64)[m >> 5]);  // block of column m
                return (float)reinterpret_cast<const int8_t*>(vrow)[m] * d;
            };
            int c = c0;
            for (; c + 64 <= cend; c += 64) {
                // eight positions of the chain: loads first, then the adds in order
                float p[8], v[8];
    #pragma unroll
                for (int u = 0; u < 8; u++) {
                    p[u] = S[c + 8 * u + l];
                    v[u] = vone(c + 8 * u + l);
                }
    #pragma unroll
                for (int u = 0; u < 8; u++) a0 = p[u] * v[u] + a0;
            }
            for (; c < cend; c += 8) a0 = S[c + l] * vone(c + l) + a0;
            if (ch + 1 < nch) {
                store_vchunk(vch, Vb + ((ch + 1) & 1) * (kAdVc * kAdVB), ch + 1, pos, s_v);
                if (ch + 2 < nch) load_vchunk(vch, vslice, vc + kvd, ch + 2, kv_pitch, g, kv_rows);
            }
            lds_barrier();
        }
    }
    acc[l * 64 + m] = a0;
    lds_barrier();
    if (w == 0) {
        // lanes left to right, then the tail positions [n8, n) in order (all
        // in the last chunk, still in its buffer)
        const int j = lane;
        float s = acc[j];
#pragma unroll
        for (int q = 1; q < 8; q++) s = s + acc[q * 64 + j];
        if constexpr (kRes) {
            for (int c = n8; c < n; c++) {
                const int lc = c & 7, kc8 = c >> 3;
                const uint32_t cw = CT[(lc * K4 + (kc8 >> 2)) * 64 + j];
                s = s + PT[lc * sT + kc8] *
                            ((float)(int)(int8_t)(cw >> (8 * (kc8 & 3))) * DT[((j >> 5) * 8 + lc) * (VP / 8) + kc8]);
            }
        } else {
            const uint8_t* B = Vb + ((nch - 1) & 1) * (kAdVc * kAdVB);
            const int c0 = (nch - 1) * kAdVc;
            for (int c = n8; c < n; c++) {
                const uint8_t* vrow = B + (c - c0) * kAdVB;
                s = s + S[c] * ((float)reinterpret_cast<const int8_t*>(vrow)[j] *
                                h2f(reinterpret_cast<const uint16_t*>(vrow + 64)[j >> 5]));
            }
        }
        act_store<Q8>(out, h * 64 + j, act_delta_offset(hq * 64), s, true);
    }
}

// ---- fp16 activations -------------------------------------------------------
//
// k_attn_dec's structure for fp16 rows (Zephyr, and the fp16 variants of the
// other models), with the arithmetic of k_qkv_post<F16> and k_attn<F16>: the
// Linear outputs rounded to fp16 (+ fp16 bias, rounded: bias_add_inplace,
// gten/ops.cpp:639-666), OpenELM's QK norm, RoPE, stored as fp16; scores as
// the fp16 dot (eight fp32 lanes = element mod 8, summed left to right,
// gten/ops.cpp:208-242), softmax as above with P rounded to fp16, P.V and
// the output as k_attn_dec.  K rows and q are fp16 pairs (the products go
// through v_fma_mix, exact like the fp32 products of fp16 values).
constexpr int kAdVB16 = 128;  // LDS bytes per staged V position: 64 fp16 values
constexpr int kAdVParts16 = kAdVc * 8 / kAdThreads;
static_assert(kAdVParts16 >= 1 && kAdVParts16 * kAdThreads == kAdVc * 8, "fp16 V chunk parts");

struct KRow16 {
    uint4 q[8];
};

__device__ __forceinline__ KRow16 load_krow16(const uint8_t* kslice, int c, int kv_pitch)
{
    KRow16 r;
    const uint4* p = reinterpret_cast<const uint4*>(kslice + (size_t)c * kv_pitch);
#pragma unroll
    for (int v = 0; v < 8; v++) r.q[v] = p[v];
    return r;
}

__device__ __forceinline__ float score16(const uint4 (&qv)[8], const KRow16& k, float scale)
{
    float a8[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int v = 0; v < 8; v++) {
        const uint32_t wq[4] = {qv[v].x, qv[v].y, qv[v].z, qv[v].w};
        const uint32_t wk[4] = {k.q[v].x, k.q[v].y, k.q[v].z, k.q[v].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            a8[2 * e] = __builtin_fmaf(h2f((uint16_t)(wq[e] & 0xFFFFu)), h2f((uint16_t)(wk[e] & 0xFFFFu)), a8[2 * e]);
            a8[2 * e + 1] = __builtin_fmaf(h2f((uint16_t)(wq[e] >> 16)), h2f((uint16_t)(wk[e] >> 16)), a8[2 * e + 1]);
        }
    }
    const float s = a8[0] + a8[1] + a8[2] + a8[3] + a8[4] + a8[5] + a8[6] + a8[7];
    return s * scale;
}

struct VChunk16 {
    uint32_t p[kAdVParts16][4];
};

// 16-byte parts tid + i kAdThreads of chunk ch (position = part / 8).
__device__ __forceinline__ void load_vchunk16(VChunk16& v, const uint8_t* vslice, int ch, int kv_pitch, int kv_rows)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAdVParts16; i++) {
        const int idx = tid + i * kAdThreads;
        const int c = min(ch * kAdVc + (idx >> 3), kv_rows - 1);
        const uint4 t4 = reinterpret_cast<const uint4*>(vslice + (size_t)c * kv_pitch)[idx & 7];
        v.p[i][0] = t4.x;
        v.p[i][1] = t4.y;
        v.p[i][2] = t4.z;
        v.p[i][3] = t4.w;
    }
}

__device__ __forceinline__ void store_vchunk16(const VChunk16& v, uint8_t* buf, int ch, int pos, const uint16_t* s_v)
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kAdVParts16; i++) {
        const int idx = tid + i * kAdThreads;
        const int cl = idx >> 3, part = idx & 7;
        uint4 t4 = make_uint4(v.p[i][0], v.p[i][1], v.p[i][2], v.p[i][3]);
        if (ch * kAdVc + cl == pos) t4 = reinterpret_cast<const uint4*>(s_v)[part];
        reinterpret_cast<uint4*>(buf + cl * kAdVB16)[part] = t4;
    }
}

// VP > 0: the V slice resident in shared memory as k_attn_dec's, with fp16
// pairs: dword (l, k2, column) holds the column's values at positions
// 16 k2 + l (low half) and 16 k2 + l + 8 (high half).
template <bool BIAS, bool QKNORM, int MK, int VP>
__global__ __launch_bounds__(kAdThreads) void k_attn_dec_f16(
    const float* __restrict__ raw, int hq, int hkv, const uint16_t* __restrict__ bq, const uint16_t* __restrict__ bk,
    const uint16_t* __restrict__ bv, const uint16_t* __restrict__ qn_w, const uint16_t* __restrict__ kn_w,
    const float2* __restrict__ table, int d_half, int pos_host, const int* __restrict__ dpos, uint8_t* __restrict__ kc,
    uint8_t* __restrict__ vc, int kv_pitch, uint8_t* __restrict__ out, float scale, int kv_rows)
{
    extern __shared__ __align__(16) float sm[];
    __shared__ __align__(16) uint16_t s_q[64], s_k[64], s_v[64];
    __shared__ __align__(16) float s_nrm[2][64];
    __shared__ float red[kAdThreads / kWave];
    __shared__ float s_sum;
    __shared__ SsShared ssh;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // heads of one kv group on one XCD, as k_attn_dec
    const int h = hq % 8 == 0 ? (int)(blockIdx.x % 8) * (hq / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int gs = hq / hkv, g = h / gs;
    const int col = w == 0 ? h * 64 : (w == 1 ? hq * 64 + g * 64 : hq * 64 + hkv * 64 + g * 64);
    const float raw_x = w < 3 ? raw[col + lane] : 0.0f;
    float bias = 0.0f;
    if (BIAS && w < 3) bias = h2f((w == 0 ? bq + h * 64 : (w == 1 ? bk + g * 64 : bv + g * 64))[lane]);
    const int pair = lane < d_half ? lane : lane - d_half;
    const bool rope_lane_in = w < 2 && lane < 2 * d_half;
    const uint8_t* kslice = kc + g * 128;
    const uint8_t* vslice = vc + g * 128;
    constexpr bool kRes = VP > 0;
    static_assert(VP % 16 == 0, "resident V: whole 16-position groups");
    VChunk16 vch;
    if constexpr (!kRes) load_vchunk16(vch, vslice, 0, kv_pitch, kv_rows);
    const int pos = dpos ? load_pos(dpos) : pos_host;
    float2 rp = make_float2(0.0f, 0.0f);
    if (rope_lane_in) rp = table[(size_t)pos * d_half + pair];
    __builtin_amdgcn_sched_barrier(0);
    const int n = pos + 1;
    const int spad = (kv_rows + kSsThreads - 1) & ~(kSsThreads - 1);
    const int sT = spad / 8 + 4;
    float* S = sm;
    float* PT = S + spad;
    float* acc = kRes ? PT + 8 * sT : S + spad;
    uint8_t* Vb = reinterpret_cast<uint8_t*>(acc + 512);
    uint32_t* CT = reinterpret_cast<uint32_t*>(acc + 512);
    constexpr int K2 = VP / 16, TPT = (4 * VP + kAdThreads - 1) / kAdThreads;

    // ---- K rows (positions < pos) into registers
    KRow16 kr[MK];
    static_for<0, MK>([&](auto I) {
        const int c = tid + I * kAdThreads;
        kr[I] = load_krow16(kslice, c < pos ? c : 0, kv_pitch);
    });

    // ---- q_h (wave 0), k_g (wave 1), v_g (wave 2) of the new position
    if (w < 3) {
        float x = f16_roundtrip(raw_x);  // the Linear output as stored
        if (BIAS) x = f16_roundtrip(x + bias);
        if (w < 2) {
            if (QKNORM) {
                float* buf = s_nrm[w];
                buf[lane] = x * x;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
                const float rms = sqrtf(seq_sum(buf, 64) / 64.0f);
                x = f16_roundtrip(x / (rms + 1e-6f) * h2f((w == 0 ? qn_w : kn_w)[lane]));
            }
            x = rope_lane_pair(x, lane, d_half, rp);
        }
        const uint16_t hx = f2h(x);
        uint16_t* st = w == 0 ? s_q : (w == 1 ? s_k : s_v);
        st[lane] = hx;
        if (w > 0 && h % gs == 0)
            reinterpret_cast<uint16_t*>((w == 1 ? kc : vc) + (size_t)pos * kv_pitch)[g * 64 + lane] = hx;
    }
    // resident V: item t = (k2, l, part q) covers rows 16 k2 + l and + 8,
    // bytes 16 q.. (columns 8 q..8 q + 7)
    uint32_t vw[kRes ? TPT : 1][2][4];
    if constexpr (kRes) {
        static_for<0, TPT>([&](auto T) {
            const int t = tid + T * kAdThreads;
            const int q = t & 7, l = (t >> 3) & 7, k2 = t >> 6;
            if (t < 4 * VP && 16 * k2 + l < n) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int c = min(16 * k2 + 8 * j + l, kv_rows - 1);
                    const uint4 x = reinterpret_cast<const uint4*>(vslice + (size_t)c * kv_pitch)[q];
                    vw[T][j][0] = x.x;
                    vw[T][j][1] = x.y;
                    vw[T][j][2] = x.z;
                    vw[T][j][3] = x.w;
                }
            }
        });
    }
    lds_barrier();

    const int nch = (n + kAdVc - 1) / kAdVc;
    if constexpr (!kRes) {
        store_vchunk16(vch, Vb, 0, pos, s_v);
        if (nch > 1) load_vchunk16(vch, vslice, 1, kv_pitch, kv_rows);
    }

    // ---- scores of positions c <= pos (thread = position)
    {
        uint4 qv[8];
#pragma unroll
        for (int v = 0; v < 8; v++) qv[v] = reinterpret_cast<const uint4*>(s_q)[v];
        static_for<0, MK>([&](auto I) {
            const int c = tid + I * kAdThreads;
            if (c < pos) S[c] = score16(qv, kr[I], scale);
        });
        int c = tid + MK * kAdThreads;
        if (c < pos) {
            KRow16 cur = load_krow16(kslice, c, kv_pitch);
            for (;;) {
                const int cn = c + kAdThreads;
                KRow16 nxt = cur;
                if (cn < pos) nxt = load_krow16(kslice, cn, kv_pitch);
                S[c] = score16(qv, cur, scale);
                if (cn >= pos) break;
                cur = nxt;
                c = cn;
            }
        }
        if (tid == (pos & (kAdThreads - 1))) {
            KRow16 kk;
#pragma unroll
            for (int v = 0; v < 8; v++) kk.q[v] = reinterpret_cast<const uint4*>(s_k)[v];
            S[pos] = score16(qv, kk, scale);
        }
    }
    if constexpr (kRes) {
        // ---- resident V into shared memory: two rows' dwords interleaved by
        // halves; the new position's row comes from s_v (all vector loads
        // waited for here, as in k_attn_dec)
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        static_for<0, TPT>([&](auto T) {
            const int t = tid + T * kAdThreads;
            const int q = t & 7, l = (t >> 3) & 7, k2 = t >> 6;
            if (t < 4 * VP && 16 * k2 + l < n) {
                uint32_t r[2][4];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const bool cur = 16 * k2 + 8 * j + l == pos;
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        r[j][i] = cur ? reinterpret_cast<const uint32_t*>(s_v)[4 * q + i] : vw[T][j][i];
                }
                uint4* dst = reinterpret_cast<uint4*>(CT + (l * K2 + k2) * 64 + 8 * q);
                dst[0] = make_uint4(__builtin_amdgcn_perm(r[1][0], r[0][0], 0x05040100u),
                                    __builtin_amdgcn_perm(r[1][0], r[0][0], 0x07060302u),
                                    __builtin_amdgcn_perm(r[1][1], r[0][1], 0x05040100u),
                                    __builtin_amdgcn_perm(r[1][1], r[0][1], 0x07060302u));
                dst[1] = make_uint4(__builtin_amdgcn_perm(r[1][2], r[0][2], 0x05040100u),
                                    __builtin_amdgcn_perm(r[1][2], r[0][2], 0x07060302u),
                                    __builtin_amdgcn_perm(r[1][3], r[0][3], 0x05040100u),
                                    __builtin_amdgcn_perm(r[1][3], r[0][3], 0x07060302u));
            }
        });
    }
    lds_barrier();

    // ---- softmax: max (order-free), expf, sequential sum, divide, fp16
    float mx = -INFINITY;
    for (int c = tid; c < n; c += kAdThreads) mx = fmaxf(mx, S[c]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    lds_barrier();
    mx = red[0];
#pragma unroll
    for (int q = 1; q < kAdThreads / kWave; q++) mx = fmaxf(mx, red[q]);
    const bool long_row = n > kAdSeqMax;
    const int npad = (n + kSsThreads - 1) & ~(kSsThreads - 1);
    for (int c = tid; c < (long_row ? npad : n); c += kAdThreads) S[c] = c < n ? expf_ref(S[c] - mx) : 0.0f;
    lds_barrier();
    float sum;
    if (long_row) {
        sum = block_seq_sum_nonneg(S, npad, ssh);
    } else {
        if (w == 0) {
            const float ss = seq_sum(S, n);
            if (lane == 0) s_sum = ss;
        }
        lds_barrier();
        sum = s_sum;
    }
    for (int c = tid; c < n; c += kAdThreads) {
        const float p = f16_roundtrip(S[c] / sum);  // P stored as an fp16 row
        if constexpr (kRes) PT[(c & 7) * sT + (c >> 3)] = p;
        else S[c] = p;
    }
    lds_barrier();

    // ---- P.V: as k_attn_dec, the chain (l, m) over positions l, l + 8, ...
    const int l = tid >> 6, m = tid & 63;
    const int n8 = n & ~7;
    float a0 = 0.0f;
    if constexpr (kRes) {
        const int kn = n8 >> 3, ng = kn >> 2;
        const float* Pl = PT + l * sT;
        const uint32_t* Cl = CT + l * K2 * 64 + m;
        for (int k4 = 0; k4 < ng; k4++) {
            const uint32_t w0 = Cl[(2 * k4) * 64], w1 = Cl[(2 * k4 + 1) * 64];
            const float4 p4 = reinterpret_cast<const float4*>(Pl)[k4];
            a0 = p4.x * h2f((uint16_t)(w0 & 0xFFFFu)) + a0;
            a0 = p4.y * h2f((uint16_t)(w0 >> 16)) + a0;
            a0 = p4.z * h2f((uint16_t)(w1 & 0xFFFFu)) + a0;
            a0 = p4.w * h2f((uint16_t)(w1 >> 16)) + a0;
        }
        for (int k = ng * 4; k < kn; k++) {
            const uint32_t wk = Cl[(k >> 1) * 64];
            a0 = Pl[k] * h2f((uint16_t)((k & 1) ? wk >> 16 : wk & 0xFFFFu)) + a0;
        }
    } else {
        for (int ch = 0; ch < nch; ch++) {
            const uint8_t* B = Vb + (ch & 1) * (kAdVc * kAdVB16);
            const int c0 = ch * kAdVc;
            const int cend = min(c0 + kAdVc, n8);
            auto vone = [&](int c) { return h2f(reinterpret_cast<const uint16_t*>(B + (c - c0) * kAdVB16)[m]); };
            int c = c0;
            for (; c + 64 <= cend; c += 64) {
                float p[8], v[8];
    #pragma unroll
                for (int u = 0; u < 8; u++) {
                    p[u] = S[c + 8 * u + l];
                    v[u] = vone(c + 8 * u + l);
                }
    #pragma unroll
                for (int u = 0; u < 8; u++) a0 = p[u] * v[u] + a0;
            }
            for (; c < cend; c += 8) a0 = S[c + l] * vone(c + l) + a0;
            if (ch + 1 < nch) {
                store_vchunk16(vch, Vb + ((ch + 1) & 1) * (kAdVc * kAdVB16), ch + 1, pos, s_v);
                if (ch + 2 < nch) load_vchunk16(vch, vslice, ch + 2, kv_pitch, kv_rows);
            }
            lds_barrier();
        }
    }
    acc[l * 64 + m] = a0;
    lds_barrier();
    if (w == 0) {
        const int j = lane;
        float s = acc[j];
#pragma unroll
        for (int q = 1; q < 8; q++) s = s + acc[q * 64 + j];
        if constexpr (kRes) {
            for (int c = n8; c < n; c++) {
                const int lc = c & 7, kc8 = c >> 3;
                const uint32_t wk = CT[(lc * K2 + (kc8 >> 1)) * 64 + j];
                s = s + PT[lc * sT + kc8] * h2f((uint16_t)((kc8 & 1) ? wk >> 16 : wk & 0xFFFFu));
            }
        } else {
            const uint8_t* B = Vb + ((nch - 1) & 1) * (kAdVc * kAdVB16);
            const int c0 = (nch - 1) * kAdVc;
            for (int c = n8; c < n; c++)
                s = s + S[c] * h2f(reinterpret_cast<const uint16_t*>(B + (c - c0) * kAdVB16)[j]);
        }
        reinterpret_cast<uint16_t*>(out)[h * 64 + j] = f2h(s);
    }
}

int attn_decode_f16_launch(const float* raw, int hq, int hkv, const uint16_t* bq, const uint16_t* bk,
                           const uint16_t* bv, const uint16_t* qn_w, const uint16_t* kn_w, const float* table,
                           int d_half, int pos, const int* dpos, uint8_t* kc, uint8_t* vc, int kv_pitch, uint8_t* out,
                           int max_ctx, hipStream_t st)
{
    if (hkv <= 0 || hq % hkv) return fail(NC_ERR_ARG, "attention: %d query heads over %d kv heads", hq, hkv);
    if (max_ctx <= 0 || max_ctx > kAttnMaxCtx)
        return fail(NC_ERR_ARG, "attention: context %d (at most %d positions)", max_ctx, kAttnMaxCtx);
    if (!dpos && (pos < 0 || pos >= max_ctx)) return fail(NC_ERR_ARG, "attention: position %d of %d", pos, max_ctx);
    if ((bq != nullptr) != (bk != nullptr) || (bq != nullptr) != (bv != nullptr))
        return fail(NC_ERR_ARG, "attention: q, k and v biases come together");
    const size_t spad = ((size_t)max_ctx + kSsThreads - 1) & ~(size_t)(kSsThreads - 1);
    // the V slice resident for caches of up to 256 rows (128 bytes a row)
    const bool res = max_ctx <= 256;
    const size_t lds = res ? (spad + 8 * (spad / 8 + 4) + 512) * 4 + 256 * 128
                           : (spad + 512) * 4 + 2 * (size_t)kAdVc * kAdVB16;
    const float scale = 1.0f / sqrtf(64.0f);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(hq), dim3(kAdThreads), lds, st, raw, hq, hkv, bq, bk, bv, qn_w, kn_w,
                           (const float2*)table, d_half, pos, dpos, kc, vc, kv_pitch, out, scale, max_ctx);
    };
    auto by_ctx = [&](auto bias, auto qk) {
        constexpr bool B = decltype(bias)::value, QK = decltype(qk)::value;
        if (res) go(k_attn_dec_f16<B, QK, 1, 256>);
        else if (max_ctx <= kAdThreads) go(k_attn_dec_f16<B, QK, 1, 0>);
        else go(k_attn_dec_f16<B, QK, kAdMaxK, 0>);
    };
    if (bq) {
        if (qn_w) by_ctx(std::true_type{}, std::true_type{});
        else by_ctx(std::true_type{}, std::false_type{});
    } else {
        if (qn_w) by_ctx(std::false_type{}, std::true_type{});
        else by_ctx(std::false_type{}, std::false_type{});
    }
    return launch_status("k_attn_dec_f16");
}

// Resident V positions of k_attn_dec for a cache of max_ctx rows (0: streamed).
static int attn_decode_vp(int max_ctx)
{
    return max_ctx <= 256 ? 256 : max_ctx <= 512 ? 512 : max_ctx <= kAdResMax ? kAdResMax : 0;
}

// Shared memory of k_attn_dec for a cache of max_ctx rows.
static size_t attn_decode_lds(int max_ctx)
{
    const size_t spad = ((size_t)max_ctx + kSsThreads - 1) & ~(size_t)(kSsThreads - 1);
    const size_t vp = (size_t)attn_decode_vp(max_ctx);
    if (vp) return (spad + 8 * (spad / 8 + 4) + 512) * 4 + vp * 64 + vp * 8;
    return (spad + 512) * 4 + 2 * (size_t)kAdVc * kAdVB;
}

bool attn_decode_supported(int hq, int hkv, int max_ctx)
{
    return hkv > 0 && hq % hkv == 0 && max_ctx > 0 && max_ctx <= kAttnMaxCtx;
}

int attn_decode_launch(const float* raw, int hq, int hkv, const uint16_t* bq, const uint16_t* bk, const uint16_t* bv,
                       const uint16_t* qn_w, const uint16_t* kn_w, const float* table, int d_half, int pos,
                       const int* dpos, uint8_t* kc, uint8_t* vc, int kv_pitch, uint8_t* out, int max_ctx,
                       hipStream_t st, const float* rope_cur)
{
    if ((bq || bk || bv) && !(bq && bk && bv)) return fail(NC_ERR_ARG, "attention: q, k and v biases go together");
    if (bq && qn_w) return fail(NC_ERR_ARG, "attention: biases with the q/k norms");
    if (hkv <= 0 || hq % hkv) return fail(NC_ERR_ARG, "attention: %d query heads over %d kv heads", hq, hkv);
    if (max_ctx <= 0 || max_ctx > kAttnMaxCtx)
        return fail(NC_ERR_ARG, "attention: context %d (at most %d positions)", max_ctx, kAttnMaxCtx);
    if (!dpos && (pos < 0 || pos >= max_ctx)) return fail(NC_ERR_ARG, "attention: position %d of %d", pos, max_ctx);
    const size_t lds = attn_decode_lds(max_ctx);
    const float scale = 1.0f / sqrtf(64.0f);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(hq), dim3(kAdThreads), lds, st, raw, hq, hkv, bq, bk, bv, qn_w, kn_w,
                           (const float2*)table, d_half, pos, dpos, kc, vc, kv_pitch, out, scale,
                           (const float2*)rope_cur, max_ctx);
    };
    // K rows requested at the start: one per thread for caches of up to
    // kAdThreads positions, two beyond; the V slice resident up to kAdResMax
    auto by_ctx = [&](auto qk, auto bias) {
        constexpr bool QK = decltype(qk)::value, B = decltype(bias)::value;
        switch (attn_decode_vp(max_ctx)) {
        case 256: go(k_attn_dec<QK, B, 1, 256>); break;
        case 512: go(k_attn_dec<QK, B, 1, 512>); break;
        case kAdResMax: go(k_attn_dec<QK, B, kAdMaxK, kAdResMax>); break;
        default: go(k_attn_dec<QK, B, kAdMaxK, 0>); break;
        }
    };
    if (qn_w) by_ctx(std::true_type{}, std::false_type{});
    else if (bq) by_ctx(std::false_type{}, std::true_type{});
    else by_ctx(std::false_type{}, std::false_type{});
    return launch_status("k_attn_dec");
}

}  // namespace nc
