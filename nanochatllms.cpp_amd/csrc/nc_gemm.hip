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
// vector-unit fold (13 fp32 operations per output and block).
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
// the activation blocks.
template <int WT, int NG, int NW, int MR, int PF, bool MF = false>
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
            if constexpr (MF) {
                // the chunk's MFMAs first (nb % kGmChunk == 0), then its folds
                // in block order: no fold waits on the MFMA just issued
                v4i L[kGmChunk][MR][kGmNg];
                float dd[kGmChunk][MR][kGmNg];
#pragma unroll
                for (int j = 0; j < kGmChunk; j++) {
                    long B[kGmNg];
                    float dw[kGmNg];
#pragma unroll
                    for (int n = 0; n < kGmNg; n++) {
                        if (WT == Q4) {
                            const uint32_t P = wr[p][j][n][0];
                            B[n] = (long)(uint64_t)(((P >> 4) & 0x0F0F0F0Fu) | ((uint64_t)(P & 0x0F0F0F0Fu) << 32));
                        } else {
                            B[n] = (long)(uint64_t)(wr[p][j][n][0] | ((uint64_t)wr[p][j][n][1] << 32));
                        }
                        dw[n] = h2f(dr[p][j][n]);
                    }
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        const uint32_t* sa = xs[buf][j][4 * m + (lc >> 2)];
                        const uint2 v = *reinterpret_cast<const uint2*>(sa + 2 * lg);
                        const bool own = lg == (lc & 3);
                        const long A = (long)(uint64_t)((own ? v.x : 0u) | ((uint64_t)(own ? v.y : 0u) << 32));
                        const uint32_t* sr = xs[buf][j][4 * m + lg];
                        const uint4 cs = *reinterpret_cast<const uint4*>(sr + 8);
                        const v4i cinit = WT == Q4 ? v4i{(int)cs.x, (int)cs.y, (int)cs.z, (int)cs.w} : v4i{0, 0, 0, 0};
                        const float dx = __uint_as_float(sr[12]);
#pragma unroll
                        for (int n = 0; n < kGmNg; n++) {
                            L[j][m][n] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B[n], cinit, 0, 0, 0);
                            dd[j][m][n] = dx * dw[n];
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < kGmChunk; j++)
#pragma unroll
                    for (int m = 0; m < MR; m++)
#pragma unroll
                        for (int n = 0; n < kGmNg; n++)
#pragma unroll
                            for (int k = 0; k < 4; k++)
                                acc[m][n][k] = acc[m][n][k] + (float)L[j][m][n][k] * dd[j][m][n];
            } else {
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

// Workgroup shapes, measured on MI355X with Q4 weights (us per launch,
// exact results in every shape): NG 16-wide column groups per wavefront,
// NW wavefronts per workgroup sharing one staging of 4 MR rows, PF weight
// chunks in flight, MF MFMAs first.
//   64 rows:   q|k|v (2560 x 2048) 30.6 -> 22.1 with (1, 1, 4, 3, MF);
//              o 28.5 -> 21.2, down (2048 x 5632) 67.0 -> 49.8 the same;
//              gate|up (11264 x 2048) 81.6 -> 56.4 with (1, 2, 8, 4)
//   512 rows:  (1, 2, 8, 4): q|k|v 138 -> 74, o 93 -> 62, down 196 -> 138;
//              gate|up 503 -> 265 with (2, 2, 8, 3)
// Wider shapes re-read the staged rows from LDS fewer times per weight
// column but leave fewer wavefronts for short prompts; MFMAs first lets a
// chunk's folds run without waiting on each MFMA result, and needs the
// chunk's four blocks to exist (nb % 4 == 0).
constexpr int kGemmWideRows = 256;
constexpr int kGemmTallCols = 8192;

int gemm_q_raw(const uint8_t* x, int x_pitch, int n_rows, const nc_tensor* w, float* out, int out_pitch,
               hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop)
{
    if (w->dtype != NC_Q4 && w->dtype != NC_Q8) return fail(NC_ERR_ARG, "gemm: Q4/Q8 weights only");
    if (w->cols % 32 || w->cols <= 0 || w->rows <= 0 || n_rows <= 0)
        return fail(NC_ERR_ARG, "gemm: [%d x %d] weights, %d rows", w->rows, w->cols, n_rows);
    const int N = w->rows, nb = w->cols / 32;
    auto go = [&](auto kern, int mr, int ng, int nw) {
        const dim3 grid((N + 16 * ng * nw - 1) / (16 * ng * nw), (n_rows + 4 * mr - 1) / (4 * mr));
        if (ev_start)
            hipExtLaunchKernelGGL(kern, grid, dim3(64 * nw), 0, st, ev_start, ev_stop, 0, x, x_pitch, n_rows,
                                  (const uint32_t*)w->data, (const uint16_t*)w->deltas, out, out_pitch, N, nb);
        else
            hipLaunchKernelGGL(kern, grid, dim3(64 * nw), 0, st, x, x_pitch, n_rows, (const uint32_t*)w->data,
                               (const uint16_t*)w->deltas, out, out_pitch, N, nb);
    };
    const bool wide = n_rows >= kGemmWideRows, tall = N >= kGemmTallCols;
    auto by_type = [&](auto wt) {
        constexpr int WT = decltype(wt)::value;
        if (wide && tall) go(k_gemm_q<WT, 2, 2, 8, 3>, 8, 2, 2);
        else if (wide || (tall && n_rows >= 32)) go(k_gemm_q<WT, 1, 2, 8, 4>, 8, 1, 2);
        else if (nb % kGmChunk == 0) go(k_gemm_q<WT, 1, 1, 4, 3, true>, 4, 1, 1);
        else go(k_gemm_q<WT, 1, 1, 4, 3>, 4, 1, 1);
    };
    if (w->dtype == NC_Q4) by_type(std::integral_constant<int, Q4>{});
    else by_type(std::integral_constant<int, Q8>{});
    return launch_status("k_gemm_q");
}

}  // namespace nc
