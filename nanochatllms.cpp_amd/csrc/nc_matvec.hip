// nc_matvec.hip -- decode/prefill matrix-vector products for gfx950.
//
// Replaces matmul_2d_impl + vec_dot_product_{q8,q8_q4,f16} (gten/ops.cpp:
// 208-242, 292-490, 579-614).  The reference's AVX dot products fix a
// summation order that these kernels keep exactly:
//   Q8/Q4: per 32-value block i, four int32 lane sums L_k(i) over the
//          elements j with (j mod 8) in {2k, 2k+1}; t_k(i) = float(L_k) *
//          (d_x * d_w); acc_k = ((0 + t_k(0)) + t_k(1)) + ... in block order;
//          result (acc_0 + acc_1) + (acc_2 + acc_3).
//   F16:   eight fp32 lanes (lane = index mod 8), acc_j = x*w + acc_j over
//          the 8-wide chunks in order, result f0 + f1 + ... + f7 left to right.
//
// Q8/Q4 kernel: a 256-thread workgroup owns R weight rows.  Every thread
// loads whole weight blocks (16 B of Q4 codes or 32 B of Q8 codes, lane-
// permuted at upload so each lane's 8 codes sit in one or two dwords),
// computes the four exact integer lane sums with v_dot4 and the four fp32
// terms, and parks the terms in LDS; then 4R threads each fold one
// (row, lane) chain in block order.  Loads and integer work are spread over
// every block of the workgroup's rows; only the cheap fp32 fold is serial.
// The activation row is staged once per workgroup in LDS with the lane
// permutation, its per-lane code sums (for the Q4 "-7" offset) and delta.
// Weights are held in registers across activation rows, so prefill reads
// every weight once per launch.
//
// F16 kernel: thread = (row, lane j); each thread reads 16-byte runs of its
// own lane (the weight layout interleaves 64-column groups over 8-row
// groups, so a wavefront reads 1 KiB contiguous) and folds its chain in
// order; the eight lanes of a row meet through wavefront shuffles.
#include <hip/hip_ext.h>

#include <type_traits>

#include "nc_kernels.h"
#include "nc_qdot.h"
#include "nc_seqsum.h"

namespace nc {

constexpr int kMvThreads = 256;
constexpr int kMvMaxItems = 4;  // weight blocks per thread held in registers

template <int WT, int R>
__global__ __launch_bounds__(kMvThreads) void k_matvec_q(const uint8_t* __restrict__ x, int x_pitch, int n_xrows,
                                                        const uint32_t* __restrict__ wq,
                                                        const uint16_t* __restrict__ wd, float* __restrict__ out,
                                                        int out_pitch, int N, int nb)
{
    constexpr int WD = WT == Q4 ? 4 : 8;  // code dwords per block
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t* xs = lds;
    const int tp = ((nb + 3) & ~3) + 4;
    float* T = reinterpret_cast<float*>(lds + nb * kStage);
    const int tid = threadIdx.x;
    const int row0 = blockIdx.x * R;
    const int nitems = R * nb;

    // the first activation row's block is requested first, then every weight
    // load of this thread (unconditionally, at a clamped index), so both
    // latencies overlap; x is consumed first
    XRaw x0{};
    if (tid < nb) x0 = load_x_block(x, nb, tid);
    uint4 w[kMvMaxItems][WD / 4];
    uint16_t dw16[kMvMaxItems];
    int tix[kMvMaxItems], bix[kMvMaxItems];
#pragma unroll
    for (int it = 0; it < kMvMaxItems; it++) {
        const int j = tid + it * kMvThreads;
        const int r = j / nb, i = j - r * nb;
        const bool ok = j < nitems && row0 + r < N;
        tix[it] = ok ? r * 4 * tp + i : -1;
        bix[it] = i;
        const size_t b = ok ? (size_t)(row0 + r) * nb + i : 0;
        const uint4* src = reinterpret_cast<const uint4*>(wq + b * WD);
#pragma unroll
        for (int v = 0; v < WD / 4; v++) w[it][v] = load_stream(src + v);
        dw16[it] = load_stream(wd + b);
    }
    for (int p = 0; p < n_xrows; p++) {
        const uint8_t* xr = x + (size_t)p * x_pitch;
        if (tid < nb) stage_x_block(p == 0 ? x0 : load_x_block(xr, nb, tid), xs + tid * kStage);
        __syncthreads();
#pragma unroll
        for (int it = 0; it < kMvMaxItems; it++) {
            if (tix[it] < 0) continue;
            float tv[4];
            q_block_terms<WT>(xs + bix[it] * kStage, w[it], dw16[it], tv);
            float* t = T + tix[it];
#pragma unroll
            for (int k = 0; k < 4; k++) t[k * tp] = tv[k];
        }
        __syncthreads();
        if (tid < kWave) {
            float acc = 0.0f;
            if (tid < 4 * R) acc = seq_sum<16>(T + tid * tp, nb);
            const int g = tid & ~3;
            const float a0 = __shfl(acc, g), a1 = __shfl(acc, g + 1), a2 = __shfl(acc, g + 2), a3 = __shfl(acc, g + 3);
            const float res = (a0 + a1) + (a2 + a3);
            const int row = row0 + (tid >> 2);
            if (tid < 4 * R && (tid & 3) == 0 && row < N) out[(size_t)p * out_pitch + row] = res;
        }
        __syncthreads();
    }
}

// F16: 8 rows x 8 lanes per wavefront, 32 rows per workgroup.
__global__ __launch_bounds__(kMvThreads) void k_matvec_f16(const uint8_t* __restrict__ x, int x_pitch, int n_xrows,
                                                          const uint16_t* __restrict__ w, float* __restrict__ out,
                                                          int out_pitch, int N, int K)
{
    extern __shared__ __align__(16) float xsf[];  // [K/64][8 lanes][8]
    const int tid = threadIdx.x;
    const int j = tid & 7;
    const int row = blockIdx.x * 32 + (tid >> 3);
    const int G = K / 64;
    const int npad = (N + 7) & ~7;
    const uint4* wrow = reinterpret_cast<const uint4*>(w) + (size_t)row * 8 + j;  // group 0
    const size_t gstride = (size_t)npad * 8;                                        // uint4s per group

    for (int p = 0; p < n_xrows; p++) {
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(x + (size_t)p * x_pitch);
        for (int e = tid; e < K; e += kMvThreads) {
            const int g = e >> 6, m = (e >> 3) & 7, jj = e & 7;
            xsf[(g * 8 + jj) * 8 + m] = h2f(xr[e]);
        }
        __syncthreads();
        float acc = 0.0f;
        if (row < N) {
            for (int g = 0; g < G; g++) {
                const uint4 u = wrow[(size_t)g * gstride];
                const float4 xa = *reinterpret_cast<const float4*>(xsf + (g * 8 + j) * 8);
                const float4 xb = *reinterpret_cast<const float4*>(xsf + (g * 8 + j) * 8 + 4);
                const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                for (int m = 0; m < 8; m++) {
                    const uint16_t h = (uint16_t)(m & 1 ? wv[m >> 1] >> 16 : wv[m >> 1] & 0xFFFFu);
                    acc = __builtin_fmaf(xv[m], h2f(h), acc);  // exact product: same as mul then add
                }
            }
        }
        const int base = tid & ~7;
        float s = __shfl(acc, base);
#pragma unroll
        for (int l = 1; l < 8; l++) s = s + __shfl(acc, base + l);
        if (j == 0 && row < N) out[(size_t)p * out_pitch + row] = s;
        __syncthreads();
    }
}

// F16, many activation rows (prefill): a 256-thread workgroup owns 32
// weight rows (thread (row, lane j) as in k_matvec_f16) and runs the
// activation rows kF16TileRows at a time, so each weight is read once per
// tile instead of once per row.  Every (activation row, weight row, lane)
// chain folds its lane's products over the 64-column groups in order, as the
// reference's 8-lane fp32 dot does; the activation tile is staged in LDS
// kF16TileGroups groups at a time.
constexpr int kF16TileRows = 16;
constexpr int kF16TileGroups = 8;  // 512 columns per stage

__global__ __launch_bounds__(kMvThreads) void k_matvec_f16_tile(const uint8_t* __restrict__ x, int x_pitch,
                                                               int n_xrows, const uint16_t* __restrict__ w,
                                                               float* __restrict__ out, int out_pitch, int N, int K)
{
    // xs[p][gl][j][m] = x[p0 + p][64 (g0 + gl) + 8 m + j]
    __shared__ __align__(16) float xs[kF16TileRows][kF16TileGroups][8][8];
    const int tid = threadIdx.x;
    const int j = tid & 7;
    const int row = blockIdx.x * 32 + (tid >> 3);
    const int G = K / 64;
    const int npad = (N + 7) & ~7;
    const int rowc = row < N ? row : N - 1;  // rows past N read a valid row and store nothing
    const uint4* wrow = reinterpret_cast<const uint4*>(w) + (size_t)rowc * 8 + j;  // group 0
    const size_t gstride = (size_t)npad * 8;                                         // uint4s per group

    for (int p0 = 0; p0 < n_xrows; p0 += kF16TileRows) {
        const int np = min(kF16TileRows, n_xrows - p0);
        float acc[kF16TileRows];
#pragma unroll
        for (int p = 0; p < kF16TileRows; p++) acc[p] = 0.0f;
        for (int g0 = 0; g0 < G; g0 += kF16TileGroups) {
            const int ng = min(kF16TileGroups, G - g0);
            // this stage's weights first, then the activation tile
            uint4 wv4[kF16TileGroups];
#pragma unroll
            for (int gl = 0; gl < kF16TileGroups; gl++) wv4[gl] = wrow[(size_t)(g0 + (gl < ng ? gl : 0)) * gstride];
            __syncthreads();  // the previous stage's tile is no longer read
            // 8-value chunks: chunk c of row p covers columns 64 g0 + 8 c .. + 7
            for (int q = tid; q < kF16TileRows * kF16TileGroups * 8; q += kMvThreads) {
                const int p = q / (kF16TileGroups * 8), c = q % (kF16TileGroups * 8);
                const int gl = c >> 3, m = c & 7;
                float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                if (p < np && gl < ng) {
                    const uint4 u = *reinterpret_cast<const uint4*>(x + (size_t)(p0 + p) * x_pitch +
                                                                   ((size_t)(g0 + gl) * 64 + 8 * m) * 2);
                    const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int t = 0; t < 8; t++) v[t] = h2f((uint16_t)(t & 1 ? h[t >> 1] >> 16 : h[t >> 1] & 0xFFFFu));
                }
#pragma unroll
                for (int t = 0; t < 8; t++) xs[p][gl][t][m] = v[t];
            }
            __syncthreads();
#pragma unroll
            for (int gl = 0; gl < kF16TileGroups; gl++) {
                if (gl >= ng) break;
                const uint32_t wq[4] = {wv4[gl].x, wv4[gl].y, wv4[gl].z, wv4[gl].w};
                float wf[8];
#pragma unroll
                for (int m = 0; m < 8; m++) wf[m] = h2f((uint16_t)(m & 1 ? wq[m >> 1] >> 16 : wq[m >> 1] & 0xFFFFu));
#pragma unroll
                for (int p = 0; p < kF16TileRows; p++) {
                    const float4 xa = *reinterpret_cast<const float4*>(&xs[p][gl][j][0]);
                    const float4 xb = *reinterpret_cast<const float4*>(&xs[p][gl][j][4]);
                    const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                    for (int m = 0; m < 8; m++) acc[p] = __builtin_fmaf(xv[m], wf[m], acc[p]);  // exact product
                }
            }
        }
        // lanes 0..7 of each row summed left to right
        const int base = tid & ~7;
#pragma unroll
        for (int p = 0; p < kF16TileRows; p++) {
            float sum = __shfl(acc[p], base);
#pragma unroll
            for (int l = 1; l < 8; l++) sum = sum + __shfl(acc[p], base + l);
            if (j == 0 && row < N && p < np) out[(size_t)(p0 + p) * out_pitch + row] = sum;
        }
    }
}

// F16, prefill (several activation rows): the lane chains of
// k_matvec_f16_row with register tiles.  A 256-thread workgroup owns 32 R
// weight rows and P activation rows; thread (row group rr, lane j) runs lane
// j's chain for its R weight rows and the P activation rows (R x P chains),
// over the 64-column groups in order.  Per chunk of GC groups it holds the
// R weight rows' lane-j values in registers (the next chunk's requested
// before this one is folded) and reads the P rows' lane-j values of each
// group from LDS (fp32, staged per chunk, double-buffered): R P 8 fused
// multiply-adds per 2 P LDS reads.  The products of two fp16 values are
// exact in fp32, so each fused multiply-add is the reference's multiply
// then add.  Workgroups of one weight block sit on one XCD when the grid's
// x extent is a multiple of 8.
template <int R, int P, int GC>
__global__ __launch_bounds__(256) void k_mm_f16(const uint8_t* __restrict__ x, int x_pitch, int n_xrows,
                                              const uint16_t* __restrict__ w, float* __restrict__ out, int out_pitch,
                                              int N, int K)
{
    static_assert(P * GC * 8 <= 256, "one staged chunk per thread at most");
    __shared__ __align__(16) float xs[2][P][GC][8][8];  // [buffer][row][group][lane j][m]
    const int tid = threadIdx.x, j = tid & 7, rr = tid >> 3;
    const int G = K / 64, nck = (G + GC - 1) / GC;
    const size_t gstride = (size_t)((N + 7) & ~7) * 8;  // uint4s per group
    const int wr0 = (int)blockIdx.x * (32 * R) + rr * R;
    const int p0 = (int)blockIdx.y * P;
    const uint4* wrow[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int rowc = min(wr0 + r, N - 1);  // rows past N read a valid row and store nothing
        wrow[r] = reinterpret_cast<const uint4*>(w) + (size_t)rowc * 8 + j;
    }
    // staging: thread q < P GC 8 converts the 8 values of (row q / (8 GC),
    // group (q / 8) % GC, m = q % 8) of a chunk
    auto stage = [&](int ck, int buf) {
        if (tid < P * GC * 8) {
            const int p = tid / (GC * 8), gl = (tid >> 3) % GC, m = tid & 7;
            const int g = ck * GC + gl;
            float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (p0 + p < n_xrows && g < G) {
                const uint4 u =
                    *reinterpret_cast<const uint4*>(x + (size_t)(p0 + p) * x_pitch + ((size_t)g * 64 + 8 * m) * 2);
                const uint32_t h[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int t = 0; t < 8; t++) v[t] = h2f((uint16_t)(t & 1 ? h[t >> 1] >> 16 : h[t >> 1] & 0xFFFFu));
            }
#pragma unroll
            for (int t = 0; t < 8; t++) xs[buf][p][gl][t][m] = v[t];
        }
    };
    auto wload = [&](int ck, uint4 (&dst)[GC][R]) {
#pragma unroll
        for (int gl = 0; gl < GC; gl++) {
            const int g = min(ck * GC + gl, G - 1);
#pragma unroll
            for (int r = 0; r < R; r++) dst[gl][r] = load_stream(wrow[r] + (size_t)g * gstride);
        }
    };
    float acc[R][P];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int p = 0; p < P; p++) acc[r][p] = 0.0f;
    auto fold = [&](int ck, int buf, const uint4 (&wv)[GC][R]) {
#pragma unroll
        for (int gl = 0; gl < GC; gl++) {
            if (ck * GC + gl >= G) break;  // uniform
            float wf[R][8];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t q[4] = {wv[gl][r].x, wv[gl][r].y, wv[gl][r].z, wv[gl][r].w};
#pragma unroll
                for (int m = 0; m < 8; m++) wf[r][m] = h2f((uint16_t)(m & 1 ? q[m >> 1] >> 16 : q[m >> 1] & 0xFFFFu));
            }
#pragma unroll
            for (int p = 0; p < P; p++) {
                const float4 xa = *reinterpret_cast<const float4*>(&xs[buf][p][gl][j][0]);
                const float4 xb = *reinterpret_cast<const float4*>(&xs[buf][p][gl][j][4]);
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                for (int m = 0; m < 8; m++)
#pragma unroll
                    for (int r = 0; r < R; r++) acc[r][p] = __builtin_fmaf(xv[m], wf[r][m], acc[r][p]);
            }
        }
    };
    uint4 wa[GC][R], wb[GC][R];
    wload(0, wa);
    stage(0, 0);
    __syncthreads();
    // chunks in pairs, so the two weight sets keep compile-time names
    for (int ck = 0; ck < nck; ck += 2) {
        if (ck + 1 < nck) {
            wload(ck + 1, wb);
            stage(ck + 1, 1);
        }
        fold(ck, 0, wa);
        __syncthreads();
        if (ck + 1 >= nck) break;  // uniform
        if (ck + 2 < nck) {
            wload(ck + 2, wa);
            stage(ck + 2, 0);
        }
        fold(ck + 1, 1, wb);
        __syncthreads();
    }
    // lanes 0..7 of each (weight row, activation row) summed left to right
    const int base = tid & ~7;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int p = 0; p < P; p++) {
            float s = __shfl(acc[r][p], base);
#pragma unroll
            for (int l = 1; l < 8; l++) s = s + __shfl(acc[r][p], base + l);
            if (j == 0 && wr0 + r < N && p0 + p < n_xrows) out[(size_t)(p0 + p) * out_pitch + wr0 + r] = s;
        }
}

// F16, one activation row (decode): a 64-thread workgroup owns 8 rows, thread
// (row, lane j) folds lane j's chain over the 64-column groups in order
// exactly as k_matvec_f16 does, but keeps two batches of kF16Batch weight
// runs in flight (the next batch is requested before the current one is
// folded), so the fold is not serialised behind one load per group.
constexpr int kF16Batch = 16;
constexpr int kMmF16Rows = 8;  // activation rows per k_mm_f16 workgroup; matvec_raw takes it from this many rows

__global__ __launch_bounds__(64) void k_matvec_f16_row(const uint8_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      float* __restrict__ out, int N, int K)
{
    extern __shared__ __align__(16) float xsf[];  // [K/64][8 lanes][8]
    const int tid = threadIdx.x;
    const int j = tid & 7;
    const int row = blockIdx.x * 8 + (tid >> 3);
    const int G = K / 64;
    const int npad = (N + 7) & ~7;
    const int rowc = row < N ? row : N - 1;  // rows past N read a valid row and store nothing
    const uint4* wrow = reinterpret_cast<const uint4*>(w) + (size_t)rowc * 8 + j;  // group 0
    const size_t gstride = (size_t)npad * 8;                                         // uint4s per group
    // two weight batches in flight, used in turn: batch A holds groups
    // [g0, g0 + B), batch B the next B groups; each is refilled right after
    // it is folded (no register copies, which would wait for the loads)
    uint4 wa[kF16Batch], wb[kF16Batch];
    auto load = [&](uint4(&dst)[kF16Batch], int gbase) {
#pragma unroll
        for (int b = 0; b < kF16Batch; b++) {
            const int g = gbase + b;
            dst[b] = load_stream(wrow + (size_t)(g < G ? g : 0) * gstride);
        }
    };
    // the activation row first (8 halves per load, K <= 8192), then the
    // weights, so staging the row waits for the row only
    constexpr int kXMax = 8192 / 8 / 64;
    uint4 xv8[kXMax];
#pragma unroll
    for (int i = 0; i < kXMax; i++) {
        const int c = tid + i * 64;  // 8-value chunk
        xv8[i] = c * 8 < K ? reinterpret_cast<const uint4*>(x)[c] : make_uint4(0, 0, 0, 0);
    }
    load(wa, 0);
    load(wb, kF16Batch);
#pragma unroll
    for (int i = 0; i < kXMax; i++) {
        const int c = tid + i * 64;
        if (c * 8 < K) {
            const uint32_t q[4] = {xv8[i].x, xv8[i].y, xv8[i].z, xv8[i].w};
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int e = c * 8 + t;
                const int g = e >> 6, m = (e >> 3) & 7, jj = e & 7;
                xsf[(g * 8 + jj) * 8 + m] = h2f((uint16_t)(t & 1 ? q[t >> 1] >> 16 : q[t >> 1] & 0xFFFFu));
            }
        }
    }
    __syncthreads();
    float acc = 0.0f;
    auto fold = [&](const uint4(&wv4)[kF16Batch], int gbase) {
#pragma unroll
        for (int b = 0; b < kF16Batch; b++) {
            const int g = gbase + b;
            if (g < G) {
                const float4 xa = *reinterpret_cast<const float4*>(xsf + (g * 8 + j) * 8);
                const float4 xb = *reinterpret_cast<const float4*>(xsf + (g * 8 + j) * 8 + 4);
                const uint32_t wv[4] = {wv4[b].x, wv4[b].y, wv4[b].z, wv4[b].w};
                const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                for (int m = 0; m < 8; m++) {
                    const uint16_t h = (uint16_t)(m & 1 ? wv[m >> 1] >> 16 : wv[m >> 1] & 0xFFFFu);
                    acc = __builtin_fmaf(xv[m], h2f(h), acc);  // exact product: same as mul then add
                }
            }
        }
    };
    for (int g0 = 0; g0 < G; g0 += 2 * kF16Batch) {
        fold(wa, g0);
        if (g0 + 2 * kF16Batch < G) load(wa, g0 + 2 * kF16Batch);
        fold(wb, g0 + kF16Batch);
        if (g0 + 3 * kF16Batch < G) load(wb, g0 + 3 * kF16Batch);
    }
    // lanes 0..7 of the row summed left to right
    const int base = tid & ~7;
    float s = __shfl(acc, base);
#pragma unroll
    for (int l = 1; l < 8; l++) s = s + __shfl(acc, base + l);
    if (j == 0 && row < N) out[row] = s;
}

// Fold of one wavefront's 64 lane chains (8 rows x 8 lanes, thread (row,
// lane j) folds lane j's chain over the G 64-column groups in order, as
// k_matvec_f16_row does), fully unrolled so that each fold waits for its
// own loads only.  The weights come through the ring wv of D loads per
// thread (its first D loads issued by the caller; the load for group g + D
// is issued once group g is folded); the activation row is the fp16 copy xs
// in LDS in the [G][8 lanes][8] order, read P groups ahead of its fold (the
// fp16 x fp16 products go through v_fma_mix exactly as through fp32).
template <int G, int D, int P>
__device__ __forceinline__ float dmv_f16_fold(const uint16_t* xs, uint4 (&wv)[D], const uint4* wrow, size_t gstride,
                                              int j)
{
    static_assert(D <= G && P <= G && P <= 15, "ring depths");
    const uint4* xrow = reinterpret_cast<const uint4*>(xs) + j;  // group g at xrow[g * 8]
    uint4 xr[P];
#pragma unroll
    for (int i = 0; i < P; i++) xr[i] = xrow[i * 8];
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < G; g++) {
        const uint4 xc = xr[g % P];
        if (g + P < G) xr[g % P] = xrow[(g + P) * 8];
        const uint4 wc = wv[g % D];
        if (g + D < G) wv[g % D] = load_stream(wrow + (size_t)(g + D) * gstride);
        const uint32_t wq[4] = {wc.x, wc.y, wc.z, wc.w}, xq[4] = {xc.x, xc.y, xc.z, xc.w};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const float a = h2f((uint16_t)(m & 1 ? xq[m >> 1] >> 16 : xq[m >> 1] & 0xFFFFu));
            const float b = h2f((uint16_t)(m & 1 ? wq[m >> 1] >> 16 : wq[m >> 1] & 0xFFFFu));
            acc = __builtin_fmaf(a, b, acc);  // exact product: same as mul then add
        }
        // keep the ring order: this group's adds are done and the reads for
        // g + P and g + D issued here (otherwise the adds sink below every
        // read, which then hold all their registers at once)
        asm volatile("" : "+v"(acc)::"memory");
        __builtin_amdgcn_sched_barrier(0);
    }
    return acc;
}

// Row of wavefront quad q's lane-row sub (8 rows per wavefront): plain, rows
// 8q .. 8q+7; GLU (w a fused gate|up [2f, K] weight, N = 2f), gate rows
// 4q .. 4q+3 and up rows f+4q .. f+4q+3.
template <bool GLU>
__device__ __forceinline__ int dmv_f16_row(int q, int sub, int N)
{
    return GLU ? (sub < 4 ? 4 * q + sub : N / 2 + 4 * q + sub - 4) : 8 * q + sub;
}

// Lanes 0..7 of each row summed left to right.  Plain: the fp32 dots to
// out.  GLU: the fp16 SwiGLU values m[4q + i] = Act(Act(silu(Act(g))) *
// Act(u)) as k_silu_mul does them (tinyllama/tinyllama.cpp:88-97 in the
// fp16 dtype).
template <bool GLU>
__device__ __forceinline__ void dmv_f16_finish(float acc, int lane, int q, int row, int N, float* out,
                                               uint16_t* m_out)
{
    const int base = lane & ~7;
    float s = __shfl(acc, base);
#pragma unroll
    for (int l = 1; l < 8; l++) s = s + __shfl(acc, base + l);
    if (!GLU) {
        if ((lane & 7) == 0 && row < N) out[row] = s;
        return;
    }
    const float gsum = __shfl(s, (lane & 3) * 8), usum = __shfl(s, ((lane & 3) + 4) * 8);
    if (lane < 4 && 4 * q + lane < N / 2) {
        const float g = f16_roundtrip(gsum);
        const float gs = f16_roundtrip(g / (1.0f + expf_ref(-g)));
        const float u = f16_roundtrip(usum);
        m_out[4 * q + lane] = f2h(gs * u);
    }
}

// F16, one activation row (decode), for the group counts G = K / 64 it is
// built for: one wavefront per 8 rows (dmv_f16_fold); the row is staged
// into LDS as fp16 in the fold's order while the weight ring is in flight.
template <int G, int D, int P, bool GLU>
__global__ __launch_bounds__(64) void k_dmv_f16(const uint8_t* __restrict__ x, const uint16_t* __restrict__ w,
                                               float* __restrict__ out, int N, uint16_t* __restrict__ m_out)
{
    constexpr int K = G * 64, XC = K / 8, XPT = (XC + 63) / 64;
    __shared__ __align__(16) uint16_t xs[K];  // [G][8 lanes][8] halves
    const int lane = threadIdx.x;
    const int j = lane & 7, q = blockIdx.x;
    const int row = dmv_f16_row<GLU>(q, lane >> 3, N);
    const int rowc = row < N ? row : N - 1;  // rows past N read a valid row and store nothing
    const size_t gstride = (size_t)((N + 7) & ~7) * 8;  // uint4s per group
    const uint4* wrow = reinterpret_cast<const uint4*>(w) + (size_t)rowc * 8 + j;
    // the activation row first, then the weight ring, so staging waits for the row only
    uint4 xv[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int c = lane + i * 64;  // 8-value chunk: group c >> 3, m = c & 7
        xv[i] = (XC % 64 == 0 || c < XC) ? reinterpret_cast<const uint4*>(x)[c] : make_uint4(0, 0, 0, 0);
    }
    uint4 wv[D];
#pragma unroll
    for (int i = 0; i < D; i++) wv[i] = load_stream(wrow + (size_t)i * gstride);
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int c = lane + i * 64;
        if (XC % 64 == 0 || c < XC) {
            const uint32_t q4[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
            for (int t = 0; t < 8; t++)
                xs[((c >> 3) * 8 + t) * 8 + (c & 7)] = (uint16_t)(t & 1 ? q4[t >> 1] >> 16 : q4[t >> 1] & 0xFFFFu);
        }
    }
    __syncthreads();
    const float acc = dmv_f16_fold<G, D, P>(xs, wv, wrow, gstride, j);
    dmv_f16_finish<GLU>(acc, lane, q, row, N, out, m_out);
}

// The norm of the row fused into the fp16 decode matvec that consumes it
// (Zephyr's layer_norm, gten/ops.cpp:669-698; the fp16 Llama, MiniCPM and
// OpenELM models' rms_norm, gten/ops.cpp:830-903).  Threads 0-255 build the
// row -- ADD: the residual sum h = a + Act(Act(braw) [* bscale], Act) stored
// to h_out by workgroup 0 -- and compute the norm, synchronizing among
// themselves through an LDS counter: layer_norm's mean as the exact
// workgroup sum of the fp16 values (nc_seqsum.h), the variance (or rms_norm's
// sum of squares) as the exact workgroup sum of non-negative terms, then
// y = ((x - mean) / (sqrt(var) + 1e-5)) * w + b, or y = x / (sqrt(ss / n) +
// 1e-6) * w, rounded to fp16 into the fold's LDS order.  The other 512
// threads (8 wavefronts, 64 rows) issue their whole weight ring at once and
// fold once the row is there: a wavefront issuing a large transfer waits at
// the issue until the memory system takes it, so the norm's wavefronts hold
// no weights.  They issue the ring only once the norm's row loads have
// returned (a CU serves its loads in order, and rows queued behind the
// ring's hundreds of KB arrive microseconds late).  Under graph replay
// (dpos) the a and h_out rows sit at the device-held position.
constexpr int kNrmNorm = kSsThreads;  // norm threads
constexpr int kNrmFold = 512;         // fold threads
enum { kNrmLayer = 0, kNrmRms = 1 };

template <int G, int D, int P, int KIND, bool ADD, bool GLU>
__global__ __launch_bounds__(kNrmNorm + kNrmFold) void k_dmv_f16_nrm(
    const uint8_t* __restrict__ a, int a_pitch, const float* __restrict__ braw, float bscale, uint8_t* __restrict__ h_out,
    int h_pitch, const uint16_t* __restrict__ nw, const uint16_t* __restrict__ nb, const uint16_t* __restrict__ w,
    float* __restrict__ out, uint16_t* __restrict__ m_out, int N, const int* __restrict__ dpos)
{
    constexpr int K = G * 64, C = K / kNrmNorm;  // values per norm thread
    static_assert(K % kNrmNorm == 0 && C <= kSsMaxPer, "row width");
    __shared__ __align__(16) float buf[K];
    __shared__ __align__(16) uint16_t xs[K];
    __shared__ SgShared sgh;
    __shared__ SsShared ssh;
    __shared__ int cnt, rows_in;
    const int tid = threadIdx.x;
    if (tid == 0) {
        cnt = 0;
        rows_in = 0;
    }
    lds_barrier();
    if (tid < kNrmNorm) {
        const size_t prow = dpos ? (size_t)load_pos(dpos) : 0;
        const uint16_t* arow = reinterpret_cast<const uint16_t*>(a + prow * a_pitch);
        float x[C], g[C], bb[C];
#pragma unroll
        for (int k = 0; k < C; k++) {
            const int e = tid * C + k;
            x[k] = h2f(arow[e]);
            g[k] = h2f(nw[e]);
            bb[k] = KIND == kNrmLayer ? h2f(nb[e]) : 0.0f;
        }
        float bw[C];
        if (ADD) {
#pragma unroll
            for (int k = 0; k < C; k++) bw[k] = braw[tid * C + k];
        }
        // every row load of this wavefront has returned: the fold's
        // wavefronts may queue their weights
        wait_loads_done();
        if ((tid & (kWave - 1)) == 0) __hip_atomic_fetch_add(&rows_in, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (ADD) {
#pragma unroll
            for (int k = 0; k < C; k++) {
                const int e = tid * C + k;
                float bv = f16_roundtrip(bw[k]);  // the Linear output as an fp16 Act
                if (bscale != 1.0f) bv = f16_roundtrip(bv * bscale);
                const float sm = x[k] + bv;
                x[k] = f16_roundtrip(sm);
                if (blockIdx.x == 0) reinterpret_cast<uint16_t*>(h_out + prow * h_pitch)[e] = f2h(sm);
            }
        }
        SsWaveBarrier<kNrmNorm / kWave> bar{&cnt, 0};
        float mean = 0.0f;
        if (KIND == kNrmLayer) {
#pragma unroll
            for (int k = 0; k < C; k++) buf[tid * C + k] = x[k];
            bar();
            mean = block_seq_sum_grid<C, kNrmNorm>(buf, sgh, nullptr, bar) / (float)K;
#pragma unroll
            for (int k = 0; k < C; k++) buf[tid * C + k] = (x[k] - mean) * (x[k] - mean);
        } else {
#pragma unroll
            for (int k = 0; k < C; k++) buf[tid * C + k] = x[k] * x[k];
        }
        bar();
        const float ss = block_seq_sum_core<C>(buf, K, ssh, nullptr, bar);
        const float denom = KIND == kNrmLayer ? sqrtf(ss / (float)K) + 1e-05f : sqrtf(ss / (float)K) + 1e-6f;
#pragma unroll
        for (int k = 0; k < C; k++) {
            const int e = tid * C + k;
            const float y = KIND == kNrmLayer ? ((x[k] - mean) / denom) * g[k] + bb[k] : x[k] / denom * g[k];
            xs[((e >> 6) * 8 + (e & 7)) * 8 + ((e >> 3) & 7)] = f2h(y);
        }
        lds_barrier();
        return;
    }
    const int ft = tid - kNrmNorm, lane = tid & (kWave - 1);
    const int j = lane & 7, q = (int)blockIdx.x * (kNrmFold / kWave) + ft / kWave;
    const int row = dmv_f16_row<GLU>(q, lane >> 3, N);
    const int rowc = row < N ? row : N - 1;  // rows past N read a valid row and store nothing
    const size_t gstride = (size_t)((N + 7) & ~7) * 8;
    const uint4* wrow = reinterpret_cast<const uint4*>(w) + (size_t)rowc * 8 + j;
    uint4 wv[D];
    while (__hip_atomic_load(&rows_in, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < kNrmNorm / kWave)
        __builtin_amdgcn_s_sleep(2);
#pragma unroll
    for (int i = 0; i < D; i++) wv[i] = load_stream(wrow + (size_t)i * gstride);
    lds_barrier();  // the normalized row is in xs
    const float acc = dmv_f16_fold<G, D, P>(xs, wv, wrow, gstride, j);
    dmv_f16_finish<GLU>(acc, lane, q, row, N, out, m_out);
}

// The group counts k_dmv_f16 is built for (d_model and d_ffn of the fp16
// models: 2048 / 5632 and 2304 / 5760), with the ring depths measured best.
template <bool GLU, class Launch>
bool dmv_f16_dispatch(int G, Launch&& go)
{
    switch (G) {
    case 32: go(k_dmv_f16<32, 32, 8, GLU>); return true;
    case 36: go(k_dmv_f16<36, 36, 8, GLU>); return true;
    case 88: go(k_dmv_f16<88, 32, 8, GLU>); return true;
    case 90: go(k_dmv_f16<90, 32, 8, GLU>); return true;
    default: return false;
    }
}

// out[r, c] = dot(x[r], w[c]) for x rows [0, n_rows) (pointers already at
// the first row), fp32 out with `out_pitch` floats per row.
int matvec_raw(const uint8_t* x, int x_dtype, int x_pitch, int n_rows, const nc_tensor* w, float* out, int out_pitch,
               hipStream_t st, hipEvent_t ev_start, hipEvent_t ev_stop, const nc_tensor* wc)
{
    // with events, the dispatch itself records them (the kernel's own start and end)
#define NC_MV_LAUNCH(KERNEL, GRID, LDS, ...)                                                              \
    do {                                                                                                  \
        if (ev_start)                                                                                     \
            hipExtLaunchKernelGGL(KERNEL, GRID, dim3(kMvThreads), LDS, st, ev_start, ev_stop, 0, __VA_ARGS__); \
        else                                                                                              \
            hipLaunchKernelGGL(KERNEL, GRID, dim3(kMvThreads), LDS, st, __VA_ARGS__);                     \
    } while (0)
    const int N = w->rows, K = w->cols;
    if (w->dtype == NC_Q4 || w->dtype == NC_Q8) {
        if (x_dtype != NC_Q8) return fail(NC_ERR_ARG, "matmul: Q%d weights need Q8 activations", w->dtype == NC_Q4 ? 4 : 8);
        if (K % 32) return fail(NC_ERR_ARG, "matmul: K=%d is not a multiple of 32", K);
        if (n_rows >= kGemmMinRows)
            return gemm_q_raw(x, x_pitch, n_rows, w, out, out_pitch, st, ev_start, ev_stop, wc);
        const int nb = K / 32;
        constexpr int R = 4;
        if (R * nb > kMvThreads * kMvMaxItems) return fail(NC_ERR_ARG, "matmul: K=%d too large", K);
        const int tp = ((nb + 3) & ~3) + 4;
        const size_t lds = (size_t)nb * kStage * 4 + (size_t)R * 4 * tp * 4;
        const dim3 grid((N + R - 1) / R);
        if (w->dtype == NC_Q4)
            NC_MV_LAUNCH((k_matvec_q<Q4, R>), grid, lds, x, x_pitch, n_rows, (const uint32_t*)w->data,
                         (const uint16_t*)w->deltas, out, out_pitch, N, nb);
        else
            NC_MV_LAUNCH((k_matvec_q<Q8, R>), grid, lds, x, x_pitch, n_rows, (const uint32_t*)w->data,
                         (const uint16_t*)w->deltas, out, out_pitch, N, nb);
        return launch_status("k_matvec_q");
    }
    if (w->dtype == NC_F16) {
        if (x_dtype != NC_F16) return fail(NC_ERR_ARG, "matmul: F16 weights need F16 activations");
        if (K % 64) return fail(NC_ERR_ARG, "matmul: F16 path needs K %% 64 == 0, K=%d", K);
        const size_t lds = (size_t)K * 4;
        if (lds > 64 * 1024) return fail(NC_ERR_ARG, "matmul: K=%d too large", K);
        if (n_rows == 1) {
            const dim3 grid((N + 7) / 8);
            auto go = [&](auto kern) {
                if (ev_start)
                    hipExtLaunchKernelGGL(kern, grid, dim3(64), 0, st, ev_start, ev_stop, 0, x,
                                          (const uint16_t*)w->data, out, N, nullptr);
                else
                    hipLaunchKernelGGL(kern, grid, dim3(64), 0, st, x, (const uint16_t*)w->data, out, N, nullptr);
            };
            if (dmv_f16_dispatch<false>(K / 64, go)) return launch_status("k_dmv_f16");
        }
        if (n_rows == 1 && K <= 8192) {
            if (ev_start)
                hipExtLaunchKernelGGL(k_matvec_f16_row, dim3((N + 7) / 8), dim3(64), lds, st, ev_start, ev_stop, 0, x,
                                      (const uint16_t*)w->data, out, N, K);
            else
                hipLaunchKernelGGL(k_matvec_f16_row, dim3((N + 7) / 8), dim3(64), lds, st, x, (const uint16_t*)w->data,
                                   out, N, K);
            return launch_status("k_matvec_f16_row");
        }
        if (n_rows >= kMmF16Rows) {
            // 64 weight rows x 8 activation rows per workgroup (measured best of R x P x GC
            // in {1, 2, 4, 8} x {4, 8, 16} x {1, 2, 4} on Zephyr's 128-row prefill)
            const dim3 grid2((N + 63) / 64, (n_rows + kMmF16Rows - 1) / kMmF16Rows);
            if (ev_start)
                hipExtLaunchKernelGGL((k_mm_f16<2, kMmF16Rows, 2>), grid2, dim3(256), 0, st, ev_start, ev_stop, 0, x,
                                      x_pitch, n_rows, (const uint16_t*)w->data, out, out_pitch, N, K);
            else
                hipLaunchKernelGGL((k_mm_f16<2, kMmF16Rows, 2>), grid2, dim3(256), 0, st, x, x_pitch, n_rows,
                                   (const uint16_t*)w->data, out, out_pitch, N, K);
            return launch_status("k_mm_f16");
        }
        const dim3 grid((N + 31) / 32);
        if (n_rows >= 4) {
            NC_MV_LAUNCH(k_matvec_f16_tile, grid, 0, x, x_pitch, n_rows, (const uint16_t*)w->data, out, out_pitch, N,
                         K);
            return launch_status("k_matvec_f16_tile");
        }
        NC_MV_LAUNCH(k_matvec_f16, grid, lds, x, x_pitch, n_rows, (const uint16_t*)w->data, out, out_pitch, N, K);
        return launch_status("k_matvec_f16");
    }
    return fail(NC_ERR_ARG, "matmul: weight dtype %d", w->dtype);
#undef NC_MV_LAUNCH
}

bool matvec_f16_glu_supported(const nc_tensor* w)
{
    return w->dtype == NC_F16 && w->rows % 8 == 0 && w->cols % 64 == 0 &&
           dmv_f16_dispatch<true>(w->cols / 64, [](auto) {});
}

int matvec_f16_glu(const uint8_t* x, const nc_tensor* w, uint8_t* m_out, hipStream_t st, hipEvent_t ev_start,
                   hipEvent_t ev_stop)
{
    const int N = w->rows, K = w->cols;
    if (!matvec_f16_glu_supported(w))
        return fail(NC_ERR_ARG, "gate|up SwiGLU matvec: [%d x %d] dtype %d", N, K, w->dtype);
    const dim3 grid(N / 8);
    auto go = [&](auto kern) {
        if (ev_start)
            hipExtLaunchKernelGGL(kern, grid, dim3(64), 0, st, ev_start, ev_stop, 0, x, (const uint16_t*)w->data,
                                  nullptr, N, (uint16_t*)m_out);
        else
            hipLaunchKernelGGL(kern, grid, dim3(64), 0, st, x, (const uint16_t*)w->data, nullptr, N,
                               (uint16_t*)m_out);
    };
    dmv_f16_dispatch<true>(K / 64, go);
    return launch_status("k_dmv_f16<GLU>");
}

bool dmv_f16_nrm_supported(const nc_tensor* w, int d, bool glu)
{
    return w->dtype == NC_F16 && w->cols == d && (d == 2048 || d == 2304) && (!glu || w->rows % 8 == 0);
}

int dmv_f16_nrm_launch(int kind, const uint8_t* a, int a_pitch, const float* braw, float bscale, uint8_t* h_out,
                       int h_pitch, const uint16_t* nw, const uint16_t* nb, const nc_tensor* w, float* out,
                       uint8_t* m_out, bool glu, hipStream_t st, const int* dpos, hipEvent_t ev_start,
                       hipEvent_t ev_stop)
{
    const int N = w->rows, K = w->cols;
    if (!dmv_f16_nrm_supported(w, K, glu) || (kind == kNrmLayer && !nb))
        return fail(NC_ERR_ARG, "norm + fp16 matvec: [%d x %d] dtype %d", N, K, w->dtype);
    const int quads = glu ? N / 8 : (N + 7) / 8;  // fold wavefronts: 8 rows each
    const dim3 grid((quads + kNrmFold / kWave - 1) / (kNrmFold / kWave));
    auto go = [&](auto kern) {
        if (ev_start)
            hipExtLaunchKernelGGL(kern, grid, dim3(kNrmNorm + kNrmFold), 0, st, ev_start, ev_stop, 0, a, a_pitch, braw,
                                  bscale, h_out, h_pitch, nw, nb, (const uint16_t*)w->data, out, (uint16_t*)m_out, N,
                                  dpos);
        else
            hipLaunchKernelGGL(kern, grid, dim3(kNrmNorm + kNrmFold), 0, st, a, a_pitch, braw, bscale, h_out, h_pitch,
                               nw, nb, (const uint16_t*)w->data, out, (uint16_t*)m_out, N, dpos);
    };
    const bool add = braw != nullptr;
    // ADD x GLU for each norm kind and row width (32 or 36 groups of 64;
    // rows of 36 groups keep 24 in the register ring, the rest refilled
    // during the fold: a full ring would spill at 768 threads)
    auto pick = [&](auto kd) {
        constexpr int KD = decltype(kd)::value;
        if (K == 2048) {
            if (add && glu) go(k_dmv_f16_nrm<32, 32, 8, KD, true, true>);
            else if (add) go(k_dmv_f16_nrm<32, 32, 8, KD, true, false>);
            else if (glu) go(k_dmv_f16_nrm<32, 32, 8, KD, false, true>);
            else go(k_dmv_f16_nrm<32, 32, 8, KD, false, false>);
        } else {
            if (add && glu) go(k_dmv_f16_nrm<36, 24, 8, KD, true, true>);
            else if (add) go(k_dmv_f16_nrm<36, 24, 8, KD, true, false>);
            else if (glu) go(k_dmv_f16_nrm<36, 24, 8, KD, false, true>);
            else go(k_dmv_f16_nrm<36, 24, 8, KD, false, false>);
        }
    };
    if (kind == kNrmLayer) pick(std::integral_constant<int, kNrmLayer>{});
    else pick(std::integral_constant<int, kNrmRms>{});
    return launch_status("k_dmv_f16_nrm");
}

}  // namespace nc

// ================================================================ C-ABI ==

using namespace nc;

namespace {

// Library-owned fp32 staging for matmul_2d calls whose output is an
// activation dtype (grown on demand, never inside a captured graph).
float* g_stage = nullptr;
size_t g_stage_bytes = 0;

int stage_buffer(size_t bytes, float** out)
{
    if (bytes > g_stage_bytes) {
        if (g_stage) (void)hipFree(g_stage);
        g_stage = nullptr;
        g_stage_bytes = 0;
        hipError_t e = hipMalloc(&g_stage, bytes);
        if (e != hipSuccess) return fail(NC_ERR_NOMEM, "matmul staging (%zu bytes): %s", bytes, hipGetErrorString(e));
        g_stage_bytes = bytes;
    }
    *out = g_stage;
    return NC_OK;
}

}  // namespace

// nc_matmul_2d_noalloc's staging: a file-scope device array.  Every GPU the
// library runs on holds its own copy, at its own address, until the process
// ends.  In host code `scratch` only names a host-side stand-in; the device
// address comes from hipGetSymbolAddress, taken once per device with that
// device current (nc_init, or the entry point's first call on a device) and
// kept in g_scratch.  Kernels get that address as an argument.
static __device__ __align__(256) float scratch[NC_NOALLOC_STAGE_BYTES / sizeof(float)];

namespace {

constexpr size_t kNoAllocStageBytes = NC_NOALLOC_STAGE_BYTES;
constexpr int kMaxDevices = 64;
float* g_scratch[kMaxDevices] = {};

int scratch_for_current(float** out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    int s = noalloc_scratch_setup(dev);
    if (s) return s;
    *out = g_scratch[dev];
    return NC_OK;
}

}  // namespace

namespace nc {

int noalloc_scratch_setup(int dev)
{
    if (dev < 0 || dev >= kMaxDevices) return fail(NC_ERR_ARG, "staging array: device %d", dev);
    if (g_scratch[dev]) return NC_OK;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch[dev] = static_cast<float*>(p);
    return NC_OK;
}

}  // namespace nc

// The same as nc_matmul_2d, with an activation-dtype output staged in the
// device's fixed array instead of library-allocated memory: no allocation
// anywhere on this path.
extern "C" int nc_matmul_2d_noalloc(const nc_tensor* x, const nc_tensor* w, nc_tensor* out, int start, int n_ctx,
                                    void* stream)
{
    NC_CHECK_ARG(x && w && out && x->data && w->data && out->data, "matmul_2d_noalloc: null tensor");
    NC_CHECK_ARG(x->cols == w->cols, "matmul_2d_noalloc: x has %d columns, w has %d", x->cols, w->cols);
    NC_CHECK_ARG(out->cols == w->rows, "matmul_2d_noalloc: out has %d columns, w has %d rows", out->cols, w->rows);
    NC_CHECK_ARG(start >= 0 && start <= n_ctx && n_ctx <= x->rows && n_ctx <= out->rows,
                 "matmul_2d_noalloc: rows [%d, %d)", start, n_ctx);
    const int rows = n_ctx - start;
    if (rows == 0) return NC_OK;
    hipStream_t st = stream_of(stream);
    const uint8_t* xr = (const uint8_t*)x->data + (size_t)start * x->pitch;
    if (out->dtype == NC_F32) {
        NC_CHECK_ARG(out->pitch % 4 == 0, "matmul_2d_noalloc: fp32 pitch %d", out->pitch);
        return matvec_raw(xr, x->dtype, x->pitch, rows, w, (float*)((uint8_t*)out->data + (size_t)start * out->pitch),
                          out->pitch / 4, st);
    }
    const size_t need = (size_t)rows * w->rows * 4;
    NC_CHECK_ARG(need <= kNoAllocStageBytes,
                 "matmul_2d_noalloc: %d rows x %d outputs need %zu staging bytes, more than the %zu-byte array", rows,
                 w->rows, need, kNoAllocStageBytes);
    float* stage = nullptr;
    int s = scratch_for_current(&stage);
    if (s) return s;
    if ((s = matvec_raw(xr, x->dtype, x->pitch, rows, w, stage, w->rows, st))) return s;
    return write_rows(stage, w->rows, (uint8_t*)out->data + (size_t)start * out->pitch, out->pitch, out->dtype, w->rows,
                      rows, st);
}

extern "C" int nc_matmul_2d(const nc_tensor* x, const nc_tensor* w, nc_tensor* out, int start, int n_ctx, void* stream)
{
    NC_CHECK_ARG(x && w && out && x->data && w->data && out->data, "matmul_2d: null tensor");
    NC_CHECK_ARG(x->cols == w->cols, "matmul_2d: x has %d columns, w has %d", x->cols, w->cols);
    NC_CHECK_ARG(out->cols == w->rows, "matmul_2d: out has %d columns, w has %d rows", out->cols, w->rows);
    NC_CHECK_ARG(start >= 0 && start <= n_ctx && n_ctx <= x->rows && n_ctx <= out->rows, "matmul_2d: rows [%d, %d)",
                 start, n_ctx);
    const int rows = n_ctx - start;
    if (rows == 0) return NC_OK;
    hipStream_t st = stream_of(stream);
    const uint8_t* xr = (const uint8_t*)x->data + (size_t)start * x->pitch;
    if (out->dtype == NC_F32) {
        NC_CHECK_ARG(out->pitch % 4 == 0, "matmul_2d: fp32 pitch %d", out->pitch);
        return matvec_raw(xr, x->dtype, x->pitch, rows, w, (float*)((uint8_t*)out->data + (size_t)start * out->pitch),
                          out->pitch / 4, st);
    }
    float* stage;
    int s = stage_buffer((size_t)rows * w->rows * 4, &stage);
    if (s) return s;
    if ((s = matvec_raw(xr, x->dtype, x->pitch, rows, w, stage, w->rows, st))) return s;
    return write_rows(stage, w->rows, (uint8_t*)out->data + (size_t)start * out->pitch, out->pitch, out->dtype, w->rows,
                      rows, st);
}
