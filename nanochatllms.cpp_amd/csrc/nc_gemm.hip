// nc_gemm.hip -- prefill matmul of Q8 activation rows with Q4 / Q8 weights
// on the matrix cores, with the reference's arithmetic.
//
// matmul_2d_impl (gten/ops.cpp:579-614) computes each output as the
// reference's block dot product (vec_dot_product_q8 / _q8_q4, ops.cpp:
// 292-490): per 32-value block b, four int32 lane sums L_k(b) over the
// elements {2k, 2k+1, 2k+8, 2k+9} and the same + 16, fp32 terms
// float(L_k) * (d_x * d_w), four fp32 chains acc_k folded in block order,
// and (acc_0 + acc_1) + (acc_2 + acc_3).
//
// The integer lane sums come from v_mfma_i32_16x16x32_i8 (K = 32 = one
// block), with the activation operand expanded by lane: matrix row 4r + k
// holds row r's lane-k codes in K group k and zeros in the other three
// groups, the weight operand holds column n's lane-g codes in K group g (the
// weights are stored lane-permuted, so a lane's eight codes are one dword
// (Q4) or two (Q8)).  Result entry (4r + k, n) is then exactly L_k(r, n),
// and the MFMA output layout puts the four lane sums of one (row, column)
// in one thread: thread (n, r) owns its chains and folds them in block
// order with plain fp32 multiplies and adds -- the reference's rounding
// steps, one per block and lane.  Q4 codes enter raw (0..14): the
// accumulator starts at -7 * (sum of the lane's activation codes), so the
// MFMA yields sum (code - 7) * x, as the reference's decoded values give.
//
// Three quarters of each activation operand are zeros: the matrix cores do
// four times the necessary integer work, which is cheap next to the
// vector-unit fold (13 fp32 operations per output and block).  k_gemm_qh
// (below) takes the same lane sums on the fp16 matrix cores and reads the
// weights' chunk-major copy when the caller has one.
#include <hip/hip_ext.h>

#include <type_traits>

#include "nc_kernels.h"
#include "nc_qdot.h"

namespace nc {

constexpr int kGmChunk = 4;                // activation blocks staged per step (double-buffered)

typedef int v4i __attribute__((ext_vector_type(4)));

// NG 16-wide column groups per wavefront, NW wavefronts per workgroup (all
// on the same rows, side by side in columns), MR groups of 4 rows (one MFMA
// row operand each) per workgroup; the first 4 MR x kGmChunk threads stage
// the activation blocks.  Kept for rows whose blocks do not come in fours and
// for long prompts of tall weights without the chunk-major copy.
template <int WT, int NG, int NW, int MR, int PF>
__global__ __launch_bounds__(64 * NW) void k_gemm_q(const uint8_t* __restrict__ x, int x_pitch, int n_rows,
                                                      const uint32_t* __restrict__ wq,
                                                      const uint16_t* __restrict__ wd, float* __restrict__ out,
                                                      int out_pitch, int N, int nb)
{
    constexpr int WV = WT == Q4 ? 1 : 2;  // code dwords of one lane of a weight block
    constexpr int WD = WT == Q4 ? 4 : 8;  // code dwords per weight block
    constexpr int kGmNg = NG;
    constexpr int kGmCols = 16 * NG * NW;  // columns per workgroup
    constexpr int kGmRows = 4 * MR;        // rows per workgroup
    // staged activation blocks (nc_qdot.h layout): [buffer][block][row]
    __shared__ __align__(16) uint32_t xs[2][kGmChunk][kGmRows][kStage];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int lc = lane & 15, lg = lane >> 4;  // column within a 16-group; K group (AVX lane)
    const int r0 = blockIdx.y * kGmRows;
    const int c0 = blockIdx.x * kGmCols + wv * 16 * NG;
    const int nch = (nb + kGmChunk - 1) / kGmChunk;

    // staging: thread t < kGmRows x kGmChunk stages (row t % kGmRows, block
    // t / kGmRows) of each chunk; rows past the end repeat the last row
    // (their outputs are not stored)
    constexpr int kStagers = kGmRows * kGmChunk;
    static_assert(kStagers <= 64 * NW, "every staged (row, block) needs its own thread");
    const int srow = tid % kGmRows, sblk = (tid / kGmRows) & (kGmChunk - 1);
    const uint8_t* xrow = x + (size_t)min(r0 + srow, n_rows - 1) * x_pitch;
    auto stage_load = [&](int ch) { return load_x_block(xrow, nb, min(ch * kGmChunk + sblk, nb - 1)); };

    // this thread's weight columns (columns past the end repeat the last)
    size_t wrow[kGmNg];
#pragma unroll
    for (int n = 0; n < kGmNg; n++) wrow[n] = (size_t)min(c0 + 16 * n + lc, N - 1) * nb;
    auto w_load = [&](int ch, uint32_t (&w)[kGmChunk][kGmNg][WV], uint16_t (&d)[kGmChunk][kGmNg]) {
#pragma unroll
        for (int j = 0; j < kGmChunk; j++) {
            const int b = min(ch * kGmChunk + j, nb - 1);
#pragma unroll
            for (int n = 0; n < kGmNg; n++) {
                const uint32_t* blk = wq + (wrow[n] + b) * WD;
#pragma unroll
                for (int v = 0; v < WV; v++) w[j][n][v] = blk[WV * lg + v];
                d[j][n] = wd[wrow[n] + b];
            }
        }
    };

    float acc[MR][kGmNg][4];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int n = 0; n < kGmNg; n++)
#pragma unroll
            for (int k = 0; k < 4; k++) acc[m][n][k] = 0.0f;

    // weights and activation blocks: a ring of PF chunks in registers;
    // chunk ch sits in slot ch % PF from its request (PF chunks ahead) until
    // it is used, so HBM latency hides behind PF chunks of work, and a slot
    // is refilled straight after use (no register copies, which would wait
    // for the loads).  Both are requested together because the vector
    // memory counter completes in order: the activation blocks staged at
    // the end of chunk ch (chunk ch + 1's) were requested PF - 1 chunks
    // earlier, so waiting for them waits only for loads that old.  Every
    // request is issued (chunks past the end re-read the last blocks), so
    // the waits are exact counts.
    uint32_t wr[PF][kGmChunk][kGmNg][WV];
    uint16_t dr[PF][kGmChunk][kGmNg];
    XRaw xq[PF];
#pragma unroll
    for (int p = 0; p < PF; p++) {
        w_load(p, wr[p], dr[p]);
        xq[p] = stage_load(min(p, nch - 1));
    }
    if (tid < kStagers) stage_x_block(xq[0], xs[0][sblk][srow]);
    lds_barrier();
    for (int cb = 0; cb < nch; cb += PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int ch = cb + p;
            if (ch >= nch) break;  // uniform
            const int buf = ch & 1;
            {
#pragma unroll
            for (int j = 0; j < kGmChunk; j++) {
                if (ch * kGmChunk + j >= nb) break;  // uniform
                // weight operands: column lc of group n, lane lg's eight codes
                long B[kGmNg];
                float dw[kGmNg];
#pragma unroll
                for (int n = 0; n < kGmNg; n++) {
                    if (WT == Q4) {
                        const uint32_t P = wr[p][j][n][0];
                        // high nibbles pair with codes {2k,2k+1,2k+8,2k+9},
                        // low nibbles with those + 16 (the staged xa_k, xb_k
                        // order)
                        B[n] = (long)(uint64_t)(((P >> 4) & 0x0F0F0F0Fu) | ((uint64_t)(P & 0x0F0F0F0Fu) << 32));
                    } else {
                        B[n] = (long)(uint64_t)(wr[p][j][n][0] | ((uint64_t)wr[p][j][n][1] << 32));
                    }
                    dw[n] = h2f(dr[p][j][n]);
                }
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    // activation operand: matrix row lc = 4 r' + k of row
                    // group m holds row (4m + r')'s lane-k codes in K group
                    // k only
                    const uint32_t* sa = xs[buf][j][4 * m + (lc >> 2)];
                    const uint2 v = *reinterpret_cast<const uint2*>(sa + 2 * lg);
                    const bool own = lg == (lc & 3);
                    const long A = (long)(uint64_t)((own ? v.x : 0u) | ((uint64_t)(own ? v.y : 0u) << 32));
                    // this thread's outputs: row 4m + lg, lane sums k = 0..3
                    const uint32_t* sr = xs[buf][j][4 * m + lg];
                    const uint4 cs = *reinterpret_cast<const uint4*>(sr + 8);
                    const v4i cinit = WT == Q4 ? v4i{(int)cs.x, (int)cs.y, (int)cs.z, (int)cs.w} : v4i{0, 0, 0, 0};
                    const float dx = __uint_as_float(sr[12]);
#pragma unroll
                    for (int n = 0; n < kGmNg; n++) {
                        const v4i L = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[n], cinit, 0, 0, 0);
                        const float dd = dx * dw[n];
#pragma unroll
                        for (int k = 0; k < 4; k++) acc[m][n][k] = acc[m][n][k] + (float)L[k] * dd;
                    }
                }
            }
            }
            // the slot's next chunk, then chunk ch + 1's activation blocks
            // into the other staging buffer
            w_load(ch + PF, wr[p], dr[p]);
            xq[p] = stage_load(min(ch + PF, nch - 1));
            if (ch + 1 < nch && tid < kStagers) stage_x_block(xq[(p + 1) % PF], xs[buf ^ 1][sblk][srow]);
            lds_barrier();
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) {
        const int row = r0 + 4 * m + lg;
#pragma unroll
        for (int n = 0; n < kGmNg; n++) {
            const int col = c0 + 16 * n + lc;
            if (row < n_rows && col < N)
                out[(size_t)row * out_pitch + col] = (acc[m][n][0] + acc[m][n][1]) + (acc[m][n][2] + acc[m][n][3]);
        }
    }
}

// ---------------------------------------------------------------------------
// The same products with the lane sums taken on the fp16 matrix cores
// (v_mfma_f32_16x16x32_f16): codes enter as fp16 integers (activation codes
// -127..127, Q4 weights code - 7 in -7..8, Q8 weights -127..127), so each
// product is an integer below 2^14 and each lane sum of eight products an
// integer below 2^17.  Every partial sum the matrix core forms is then an
// integer exactly representable in fp32, and the fp32 result is exactly
// float(L_k): the conversion the integer path needs per lane and block is
// gone, and the fold is 9 fp32 operations per (row, column, block) instead
// of 13.
//
// The activation operand is staged once per workgroup already expanded: for
// block j and row group m, lane l = (4r + k) + 16 g holds row 4m + r's lane-k
// codes as fp16 when g == k, and zeros otherwise (the zero entries are written
// once at kernel start and never touched again).  A lane reads its 16 bytes
// with one LDS load; rows of a group share them across the NW wavefronts.
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// Four bytes b0..b3 of `u` (each below 256) as fp16 1024 + b, two per dword:
// [b0, b1] and [b2, b3] (v_perm_b32 with the exponent byte 0x64 from a
// constant).
__device__ __forceinline__ void bytes_to_h1024(uint32_t u, uint32_t& lo, uint32_t& hi)
{
    lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
}

// The same, then plus `bias` (fp16, both halves): exact integers.
__device__ __forceinline__ void bytes_to_h(uint32_t u, uint32_t bias2, uint32_t& lo, uint32_t& hi)
{
    uint32_t a, b;
    bytes_to_h1024(u, a, b);
    const h2_t bb = __builtin_bit_cast(h2_t, bias2);
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, a) + bb);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, b) + bb);
}
constexpr uint32_t kHm1152 = 0xE480E480u;  // fp16 -1152, twice: (1024 + c + 128) - 1152 = c
constexpr uint32_t kHm1031 = 0xE407E407u;  // fp16 -1031, twice: (1024 + n) - 1031 = n - 7

// Four signed int8 codes -> four fp16 values (two dwords).
__device__ __forceinline__ void s8x4_to_h(uint32_t v, uint32_t& lo, uint32_t& hi)
{
    bytes_to_h(v ^ 0x80808080u, kHm1152, lo, hi);
}

// NW wavefronts per workgroup share the staged activation blocks of 4 MR
// rows and own 16 weight columns each; a chunk is CH blocks (one LDS barrier
// per chunk), and PF chunks of weights and activation blocks are in flight.
// Within a chunk the MFMAs of block j + 1 are issued before the folds of
// block j, so no fold waits on the MFMA just issued.  CL: the weights are
// read from their chunk-major copy (k_chunk_layout), where a wavefront's
// codes of four blocks are one contiguous 1 KB (Q4) and a thread's are one
// 16-byte load, instead of four 4-byte loads from 16 rows each.  WPE: the
// wavefronts per SIMD the registers are allotted for (the fold is
// vector-unit work and needs wavefronts beside each other to cover its
// latencies).
template <int WT, int MR, int NW, int CH, int PF, bool CL, int WPE = 1>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE))) void k_gemm_qh(
        const uint8_t* __restrict__ x, int x_pitch, int n_rows, const uint32_t* __restrict__ wq,
        const uint16_t* __restrict__ wd, float* __restrict__ out, int out_pitch, int N, int nb)
{
    constexpr int WV = WT == Q4 ? 1 : 2;  // code dwords of one lane of a weight block
    constexpr int WD = WT == Q4 ? 4 : 8;  // code dwords per weight block
    constexpr int kRows = 4 * MR;         // rows per workgroup
    constexpr int kThreads = 64 * NW;
    static_assert(CH == 4 || CH == 8, "chunk of 4 or 8 blocks (one 8- or 16-byte delta load)");
    // expanded activation operands [buffer][block][row group][lane] and the
    // rows' deltas [buffer][block][row]
    __shared__ __align__(16) uint4 xa[2][CH][MR][64];
    __shared__ float xd[2][CH][kRows];
    // CI (the long-prompt Q4 shape: chunk-major copy, at most 8 rows, one
    // chunk in flight): the products' accumulator start per (block, row,
    // lane k), -1031 x (sum of the lane's eight activation codes), and raw
    // weight codes 1024 + n (four conversions fewer per block; the other
    // shapes have no registers for the starts)
    constexpr bool CI = WT == Q4 && CL && MR <= 2 && PF == 1;
    __shared__ __align__(16) float xc[CI ? 2 : 1][CH][kRows][4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int lc = lane & 15, lg = lane >> 4;
    const int r0 = blockIdx.y * kRows;
    const int col = min(blockIdx.x * 16 * NW + wv * 16 + lc, N - 1);  // this thread's weight column
    const int nch = nb / CH;

    // zero entries: lane l = lc + 16 lg with lg != lc % 4, never staged
    for (int e = tid; e < 2 * CH * MR * 64; e += kThreads)
        if (((e & 15) & 3) != ((e >> 4) & 3)) (&xa[0][0][0][0])[e] = make_uint4(0, 0, 0, 0);

    // staging, spread over every thread: a task is one AVX lane k of one
    // (row, block) of the chunk -- its eight codes as fp16 (16 bytes) -- and
    // lane 0's task also stages the block's delta.  Rows past the end repeat
    // the last row (their outputs are not stored).
    constexpr int kTasks = 4 * kRows * CH;
    constexpr int TPT = (kTasks + kThreads - 1) / kThreads;  // tasks per thread
    struct XLane {
        uint32_t d[4];  // dwords k/2, 2 + k/2, 4 + k/2, 6 + k/2 of the block
        uint16_t d16;
    };
    int t_row[TPT], t_blk[TPT], t_k[TPT];
    const uint8_t* t_src[TPT];
#pragma unroll
    for (int i = 0; i < TPT; i++) {
        const int t = min(tid + i * kThreads, kTasks - 1);  // surplus slots repeat the last task
        t_k[i] = t & 3;
        t_row[i] = (t >> 2) % kRows;
        t_blk[i] = (t >> 2) / kRows;
        t_src[i] = x + (size_t)min(r0 + t_row[i], n_rows - 1) * x_pitch;
    }
    auto x_load = [&](int ch, XLane (&q)[TPT]) {
        const int b0 = min(ch, nch - 1) * CH;
#pragma unroll
        for (int i = 0; i < TPT; i++) {
            const int b = b0 + t_blk[i];
            const uint32_t* blk = reinterpret_cast<const uint32_t*>(t_src[i] + (size_t)b * 32);
            const int h = t_k[i] >> 1;
#pragma unroll
            for (int v = 0; v < 4; v++) q[i].d[v] = blk[2 * v + h];
            q[i].d16 = reinterpret_cast<const uint16_t*>(t_src[i] + (size_t)nb * 32)[b];
        }
    };
    auto stage = [&](const XLane (&q)[TPT], int buf) {
#pragma unroll
        for (int i = 0; i < TPT; i++) {
            if (tid + i * kThreads >= kTasks) break;  // uniform per wave: kTasks is a multiple of 64
            const int k = t_k[i], r = t_row[i], j = t_blk[i];
            const uint32_t a = pick_pair(q[i].d[0], q[i].d[1], k & 1);
            const uint32_t bq = pick_pair(q[i].d[2], q[i].d[3], k & 1);
            uint4 hv;
            s8x4_to_h(a, hv.x, hv.y);
            s8x4_to_h(bq, hv.z, hv.w);
            xa[buf][j][r >> 2][(r & 3) * 4 + k + 16 * k] = hv;
            if (k == 0) xd[buf][j][r] = h2f(q[i].d16);
            if constexpr (CI)
                xc[buf][j][r][k] = -1031.0f * (float)(__builtin_amdgcn_sdot4((int)a, 0x01010101, 0, false) +
                                                       __builtin_amdgcn_sdot4((int)bq, 0x01010101, 0, false));
        }
    };

    const uint32_t* wcol = wq + (size_t)col * nb * WD + WV * lg;
    const uint16_t* dcol = wd + (size_t)col * nb;
    struct WChunk {
        uint32_t c[CH][WV];
        uint32_t d[CH / 2];  // the chunk's fp16 deltas, two per dword
    };
    auto w_load = [&](int ch, WChunk& w) {
        const int b0 = min(ch, nch - 1) * CH;
        if constexpr (CL) {
            // codes [nb/4][N][4 lanes][4 blocks x WV dwords], deltas [nb/4][N][4]
#pragma unroll
            for (int h = 0; h < CH / 4; h++) {
                const size_t c4 = (size_t)(b0 / 4 + h) * N + col;
                const uint4* src = reinterpret_cast<const uint4*>(wq + (c4 * 4 + lg) * 4 * WV);
#pragma unroll
                for (int q = 0; q < WV; q++) {
                    const uint4 t = src[q];
                    const uint32_t tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) w.c[4 * h + (4 * q + e) / WV][(4 * q + e) % WV] = tv[e];
                }
                const uint2 d = *reinterpret_cast<const uint2*>(wd + c4 * 4);
                w.d[2 * h] = d.x;
                w.d[2 * h + 1] = d.y;
            }
        } else {
#pragma unroll
            for (int j = 0; j < CH; j++)
#pragma unroll
                for (int v = 0; v < WV; v++) w.c[j][v] = wcol[(size_t)(b0 + j) * WD + v];
            if constexpr (CH == 4) {
                const uint2 d = *reinterpret_cast<const uint2*>(dcol + b0);
                w.d[0] = d.x;
                w.d[1] = d.y;
            } else {
                const uint4 d = *reinterpret_cast<const uint4*>(dcol + b0);
                w.d[0] = d.x;
                w.d[1] = d.y;
                w.d[2] = d.z;
                w.d[3] = d.w;
            }
        }
    };

    float acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int k = 0; k < 4; k++) acc[m][k] = 0.0f;

    // one block's B operand (fp16 codes) and delta
    auto b_operand = [&](const WChunk& w, int j, h8_t& Bh, float& dw) {
        uint4 B;
        if (CI) {
            // high nibbles pair with the lane's codes {2k,2k+1,2k+8,2k+9},
            // low nibbles with those + 16; raw 1024 + n (the accumulator
            // start takes off 1031 x the activation codes' sum, so the
            // result is sum (n - 7) x: every value on the way an integer
            // below 2^22)
            const uint32_t P = w.c[j][0];
            bytes_to_h1024((P >> 4) & 0x0F0F0F0Fu, B.x, B.y);
            bytes_to_h1024(P & 0x0F0F0F0Fu, B.z, B.w);
        } else if (WT == Q4) {
            // the same nibbles as code - 7
            const uint32_t P = w.c[j][0];
            bytes_to_h((P >> 4) & 0x0F0F0F0Fu, kHm1031, B.x, B.y);
            bytes_to_h(P & 0x0F0F0F0Fu, kHm1031, B.z, B.w);
        } else {
            s8x4_to_h(w.c[j][0], B.x, B.y);
            s8x4_to_h(w.c[j][1], B.z, B.w);
        }
        Bh = __builtin_bit_cast(h8_t, B);
        dw = h2f((uint16_t)(w.d[j >> 1] >> (16 * (j & 1))));
    };

    // weights and activation blocks in a ring of PF chunks (requested PF
    // chunks ahead, every request issued so the waits are exact counts)
    WChunk wr[PF];
    XLane xq[PF][TPT];
#pragma unroll
    for (int p = 0; p < PF; p++) {
        w_load(p, wr[p]);
        x_load(p, xq[p]);
    }
    stage(xq[0], 0);
    lds_barrier();
    for (int cb = 0; cb < nch; cb += PF) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int ch = cb + p;
            if (ch >= nch) break;  // uniform
            const int buf = ch & 1;
            // the chunk's row deltas, and the activation operands two
            // blocks ahead in a ring of two (block j + 2 is read into block
            // j's slot once block j's products are issued), which keeps the
            // registers within three wavefronts per SIMD
            uint4 Ar[2][MR];
            f4_t Cr[2][MR];  // CI: accumulator starts, in the same ring
            float dxr[CH][MR];
            auto c_init = [&](int j, int m) {
                if constexpr (CI) return *reinterpret_cast<const f4_t*>(&xc[buf][j][4 * m + lg][0]);
                else return f4_t{0.0f, 0.0f, 0.0f, 0.0f};
            };
#pragma unroll
            for (int j = 0; j < CH; j++)
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    if (j < 2) {
                        Ar[j][m] = xa[buf][j][m][lane];
                        Cr[j][m] = c_init(j, m);
                    }
                    dxr[j][m] = xd[buf][j][4 * m + lg];
                }
            f4_t L[2][MR];
            float dw[2];
            {
                h8_t Bh;
                b_operand(wr[p], 0, Bh, dw[0]);
#pragma unroll
                for (int m = 0; m < MR; m++)
                    L[0][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, Ar[0][m]), Bh, Cr[0][m],
                                                                      0, 0, 0);
            }
#pragma unroll
            for (int j = 0; j < CH; j++) {
                const int cur = j & 1;
                if (j + 1 < CH) {
                    h8_t Bh;
                    b_operand(wr[p], j + 1, Bh, dw[cur ^ 1]);
#pragma unroll
                    for (int m = 0; m < MR; m++)
                        L[cur ^ 1][m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(h8_t, Ar[cur ^ 1][m]), Bh, Cr[cur ^ 1][m], 0, 0, 0);
                }
                if (j + 2 < CH) {
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        Ar[cur][m] = xa[buf][j + 2][m][lane];
                        Cr[cur][m] = c_init(j + 2, m);
                    }
                }
                // block j's folds in block order: row 4m + lg, lane sums k
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const float dd = dxr[j][m] * dw[cur];
#pragma unroll
                    for (int k = 0; k < 4; k++) acc[m][k] = acc[m][k] + L[cur][m][k] * dd;
                }
            }
            w_load(ch + PF, wr[p]);
            x_load(ch + PF, xq[p]);
            if (ch + 1 < nch) stage(xq[(p + 1) % PF], buf ^ 1);
            lds_barrier();
        }
    }
    const int oc = blockIdx.x * 16 * NW + wv * 16 + lc;
#pragma unroll
    for (int m = 0; m < MR; m++) {
        const int row = r0 + 4 * m + lg;
        if (row < n_rows && oc < N)
            out[(size_t)row * out_pitch + oc] = (acc[m][0] + acc[m][1]) + (acc[m][2] + acc[m][3]);
    }
}

// The chunk-major copy of a Q4 / Q8 weight [N, K] (K % 128 == 0) that the
// prefill matmul reads: codes [K/128][N][4 lanes][4 blocks][WV dwords] --
// for each group of four blocks, each row's lane-k code dwords of the four
// blocks side by side -- and deltas [K/128][N][4].
template <int WT>
__global__ void k_chunk_layout(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N, int nb,
                               uint32_t* __restrict__ cq, uint16_t* __restrict__ cd)
{
    constexpr int WV = WT == Q4 ? 1 : 2, WD = WV * 4;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one (row, block) each
    if (t >= (int64_t)N * nb) return;
    const int n = (int)(t / nb), b = (int)(t - (int64_t)n * nb);
    const size_t c4 = (size_t)(b >> 2) * N + n;
    const uint32_t* src = wq + t * WD;
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
        for (int v = 0; v < WV; v++) cq[((c4 * 4 + k) * 4 + (b & 3)) * WV + v] = src[WV * k + v];
    cd[c4 * 4 + (b & 3)] = wd[t];
}

bool chunk_layout_supported(const nc_tensor* w)
{
    return (w->dtype == NC_Q4 || w->dtype == NC_Q8) && w->cols > 0 && w->cols % 128 == 0 && w->rows > 0;
}

int chunk_layout_launch(const nc_tensor* w, void* codes, void* deltas, hipStream_t st)
{
    if (!chunk_layout_supported(w)) return fail(NC_ERR_ARG, "chunk layout: [%d x %d] dtype %d", w->rows, w->cols, w->dtype);
    const int nb = w->cols / 32;
    const int64_t n = (int64_t)w->rows * nb;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (w->dtype == NC_Q4)
        hipLaunchKernelGGL(k_chunk_layout<Q4>, grid, dim3(256), 0, st, (const uint32_t*)w->data,
                           (const uint16_t*)w->deltas, w->rows, nb, (uint32_t*)codes, (uint16_t*)deltas);
    else
        hipLaunchKernelGGL(k_chunk_layout<Q8>, grid, dim3(256), 0, st, (const uint32_t*)w->data,
                           (const uint16_t*)w->deltas, w->rows, nb, (uint32_t*)codes, (uint16_t*)deltas);
    return launch_status("k_chunk_layout");
}

// Workgroup shapes, measured on MI355X with Q4 weights (us per launch,
// exact results in every shape).  k_gemm_q: NG 16-wide column groups per
// wavefront, NW wavefronts per workgroup sharing one staging of 4 MR rows,
// PF weight chunks in flight (MF: a variant that issued a chunk's MFMAs
// before its folds, since replaced by k_gemm_qh).
//   64 rows:   q|k|v (2560 x 2048) 30.6 -> 22.1 with (1, 1, 4, 3, MF);
//              o 28.5 -> 21.2, down (2048 x 5632) 67.0 -> 49.8 the same;
//              gate|up (11264 x 2048) 81.6 -> 56.4 with (1, 2, 8, 4)
//   512 rows:  (1, 2, 8, 4): q|k|v 138 -> 74, o 93 -> 62, down 196 -> 138;
//              gate|up 503 -> 265 with (2, 2, 8, 3)
// k_gemm_qh over the chunk-major copy (MR, NW, CH, PF), every launch after
// a 512 MB write that evicts L2 and the memory-side cache, as a prefill
// meets its weights (k_gemm_q in brackets):
//   64 rows, (2, 4, 8, 2):  q|k|v (2560 x 2048) 18.2 [24.5]; o 14.2 [22.2];
//              down (2048 x 5632) 29.5 [47.3]; Q8 q|k|v 20.5 [24.7], down
//              32.6 [48.8]
//   gate|up (11264 x 2048, 64 rows) and every 512-row shape, (4, 4, 4, 2):
//              gate|up 40.0 [61.5], Q8 48.6 [64.5]; MiniCPM q|k|v (6912 x
//              2304) 162 [210], o 63 [81], gate|up (11520 x 2304) 266
//              [318], down (2304 x 5760) 145 [186]
// Where the time goes (the same shapes with parts of the work left out of a
// copy of the kernel): at 64 rows the fold was a few percent, the weight
// loads a quarter and the activation staging another quarter -- a launch
// is bound by load latency and request count, not by the arithmetic.  The
// chunk-major copy turns four 4-byte loads from 16 rows into one 16-byte
// load per thread and chunk; at 512 rows the staging was the largest part
// (28%) while one wavefront of four did it, so every thread now stages one
// AVX lane of one (row, block).
constexpr int kGemmWideRows = 256;
constexpr int kGemmTallCols = 8192;
constexpr int kGemmShortRows = 80;  // prompts up to this many rows take the short-prompt shapes

int gemm_q_raw(const uint8_t* x, int x_pitch, int n_rows, const nc_tensor* w, float* out, int out_pitch,
               hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop, const nc_tensor* wc)
{
    if (w->dtype != NC_Q4 && w->dtype != NC_Q8) return fail(NC_ERR_ARG, "gemm: Q4/Q8 weights only");
    if (w->cols % 32 || w->cols <= 0 || w->rows <= 0 || n_rows <= 0)
        return fail(NC_ERR_ARG, "gemm: [%d x %d] weights, %d rows", w->rows, w->cols, n_rows);
    const int N = w->rows, nb = w->cols / 32;
    auto go = [&](auto kern, int mr, int ng, int nw, const nc_tensor* wt = nullptr) {
        if (!wt) wt = w;
        const dim3 grid((N + 16 * ng * nw - 1) / (16 * ng * nw), (n_rows + 4 * mr - 1) / (4 * mr));
        if (ev_start)
            hipExtLaunchKernelGGL(kern, grid, dim3(64 * nw), 0, st, ev_start, ev_stop, 0, x, x_pitch, n_rows,
                                  (const uint32_t*)wt->data, (const uint16_t*)wt->deltas, out, out_pitch, N, nb);
        else
            hipLaunchKernelGGL(kern, grid, dim3(64 * nw), 0, st, x, x_pitch, n_rows, (const uint32_t*)wt->data,
                               (const uint16_t*)wt->deltas, out, out_pitch, N, nb);
    };
    const bool wide = n_rows >= kGemmWideRows, tall = N >= kGemmTallCols;
    // the chunk-major copy, when the caller has one (shapes measured with
    // cold caches, as a prefill meets its weights)
    if (wc) {
        if (wc->dtype != w->dtype || wc->rows != N || wc->cols != w->cols || !chunk_layout_supported(wc))
            return fail(NC_ERR_ARG, "gemm: chunk copy [%d x %d] of a [%d x %d] weight", wc->rows, wc->cols, N, w->cols);
        auto goc = [&](auto kern, int mr, int nw) { go(kern, mr, 1, nw, wc); };
        auto by_type_c = [&](auto wt) {
            constexpr int WT = decltype(wt)::value;
            // chunks of 8 blocks need nb % 8 == 0 (the copy itself is in
            // 4-block chunks).  Long Q4 prompts: 8 rows per workgroup, one
            // chunk in flight, five wavefronts per SIMD (84 VGPRs); medium
            // ones (81-255 rows): 8 rows, two chunks in flight, four
            // wavefronts (120 VGPRs).
            if (wide && WT == Q4) goc(k_gemm_qh<WT, 2, 4, 4, 1, true, 5>, 2, 4);
            else if (n_rows > kGemmShortRows && WT == Q4) goc(k_gemm_qh<WT, 2, 4, 4, 2, true, 4>, 2, 4);
            else if (wide || tall || n_rows > kGemmShortRows || nb % 8)
                goc(k_gemm_qh<WT, 4, 4, 4, 2, true, WT == Q4 ? 3 : 1>, 4, 4);
            else goc(k_gemm_qh<WT, 2, 4, 8, 2, true>, 2, 4);
        };
        if (w->dtype == NC_Q4) by_type_c(std::integral_constant<int, Q4>{});
        else by_type_c(std::integral_constant<int, Q8>{});
        return launch_status("k_gemm_qh (chunk layout)");
    }
    // the fp16 matrix-core kernel: chunks of 4 (8) blocks, 8- (16-) byte
    // delta loads
    const bool qh4 = nb % 4 == 0 && ((uintptr_t)w->deltas & 7) == 0;
    const bool qh8 = nb % 8 == 0 && ((uintptr_t)w->deltas & 15) == 0;
    auto goh = [&](auto kern, int mr, int nw) { go(kern, mr, 1, nw); };
    auto by_type = [&](auto wt) {
        constexpr int WT = decltype(wt)::value;
        if (wide && tall) go(k_gemm_q<WT, 2, 2, 8, 3>, 8, 2, 2);
        else if (qh4 && (wide || tall || n_rows > kGemmShortRows || !qh8)) goh(k_gemm_qh<WT, 4, 4, 4, 2, false>, 4, 4);
        else if (qh8 && n_rows <= 16) goh(k_gemm_qh<WT, 2, 2, 8, 3, false>, 2, 2);
        else if (qh8 && (N <= 2048 || nb >= 128)) goh(k_gemm_qh<WT, 2, 4, 8, 2, false>, 2, 4);
        else if (qh8) goh(k_gemm_qh<WT, 4, 4, 4, 2, false>, 4, 4);
        else if (wide || (tall && n_rows >= 32)) go(k_gemm_q<WT, 1, 2, 8, 4>, 8, 1, 2);
        else go(k_gemm_q<WT, 1, 1, 4, 3>, 4, 1, 1);
    };
    if (w->dtype == NC_Q4) by_type(std::integral_constant<int, Q4>{});
    else by_type(std::integral_constant<int, Q8>{});
    return launch_status("k_gemm_q / k_gemm_qh");
}

}  // namespace nc
