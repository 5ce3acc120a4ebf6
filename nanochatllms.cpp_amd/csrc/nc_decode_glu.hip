// nc_decode_glu.hip -- the gate|up matvec of the single-row decode step with
// the SwiGLU epilogue (Q8 activations, Q4/Q8 weights): k_dmv_glu, and
// k_dmv_glu_spec, which computes the weight terms, fold and SwiGLU beside the
// exact norm sums from a predicted row (nc_dmv.h: spec_exact, spec_weights).  The
// arithmetic is the reference's block dot product, fold order and
// requantization points (tinyllama/tinyllama.cpp:88-97).
#include "nc_dmv.h"

namespace nc {

// Gate|up matvec with the SwiGLU epilogue: a workgroup owns output block b
// (values 32b .. 32b+31) and computes its 32 gate rows (32b + r) and 32 up
// rows (f + 32b + r) -- all of their weights requested up front -- in two
// halves through the fold, then m = Act(Act(silu(Act(g))) * Act(u)) for the
// block (tinyllama/tinyllama.cpp:88-97).  No workgroup waits for another.

template <int WT, int PRO, int NCH, int NB>
__global__ __launch_bounds__(kGluThreads) void k_dmv_glu(DmvArgs A)
{
    constexpr int WD = WT == Q4 ? 4 : 8;
    constexpr int WV = WD / 4;
    constexpr int TP = ((NB + 3) & ~3) + 4;
    constexpr int IT = NB * 64 / kGluThreads;  // weight blocks per thread (64 rows)
    static_assert(NB % 8 == 0 && IT <= kGluMaxItems, "gate|up block shape");
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ SsShared ssh;
    __shared__ SgShared sgh;
    __shared__ float s_out[64];
    uint32_t* xs = lds;
    float* T = reinterpret_cast<float*>(xs + NB * kStage);  // 64 rows (gate, then up) x 4 lanes x TP
    float* sq = T + 64 * 4 * TP;
    const int tid = threadIdx.x;
    const int f = A.N / 2, nblk = f / 32;

    uint4 w[IT][WV];
    uint16_t dw[IT];
    auto load_block = [&](int b) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int j = tid + it * kGluThreads;
            const int r = j / NB, i = j - r * NB;
            const int row = r < 32 ? 32 * b + r : f + 32 * b + (r - 32);
            const size_t bi = (size_t)row * NB + i;
            const uint4* src = reinterpret_cast<const uint4*>(A.wq + bi * WD);
#pragma unroll
            for (int v = 0; v < WV; v++) w[it][v] = load_stream(src + v);
            dw[it] = load_stream(A.wd + bi);
        }
    };
    int b = blockIdx.x;  // < nblk: the grid never exceeds the blocks
    DmvArgs P = A;
    P.nb = NB;
    dmv_prologue<PRO, NCH, false, kGluThreads>(P, xs, sq, ssh, sgh, [&] { load_block(b); });

    // the terms of all 64 rows, then the gate rows' folds (waves 0-1) and
    // the up rows' folds (waves 2-3) side by side
    auto pass = [&]() {
        // NB dividing the workgroup: every item of a thread is block
        // tid % NB, read from LDS once
        constexpr bool kOneBlock = kGluThreads % NB == 0;
        StagedX x0{};
        if (kOneBlock) x0 = load_staged(xs + (tid % NB) * kStage);
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int j = tid + it * kGluThreads;
            const int r = j / NB, i = j - r * NB;
            float tv[4];
            if (kOneBlock)
                q_block_terms<WT>(x0, w[it], dw[it], tv);
            else
                q_block_terms<WT>(xs + i * kStage, w[it], dw[it], tv);
            float* t = T + r * 4 * TP + i;
#pragma unroll
            for (int k = 0; k < 4; k++) t[k * TP] = tv[k];
        }
        lds_barrier();
        if (tid < 64 * 4) {
            // thread 4r + k folds lane k of row r in block order (waves 0-3)
            const float acc = seq_sum<16>(T + tid * TP, NB);
            const float res = (acc + dpp_f<kDppQuadXor1>(acc)) + (dpp_f<kDppQuadXor2>(acc) + dpp_f<0x1B>(acc));
            if ((tid & 3) == 0) {
                const int r = tid >> 2;  // 0..31 gate, 32..63 up
                s_out[r] = res;
                if (A.raw) A.raw[(r >= 32 ? f - 32 : 0) + 32 * b + r] = res;
            }
        }
        lds_barrier();
    };
    for (;;) {
        pass();
        if (tid < 64) {
            // lanes 0-31: the gate chain; lanes 32-63: the up value's round
            // trip beside it (each half-wavefront its own 32-value block)
            const float v = q8_roundtrip_lane(s_out[tid], true);
            const float uq = __shfl(v, (tid & 31) + 32);
            const float gs = q8_roundtrip_lane(v / (1.0f + expf_ref(-v)), true);
            act_store<Q8>(A.m_out, 32 * b + (tid & 31), f, gs * uq, tid < 32);
        }
        b += gridDim.x;
        if (b >= nblk) break;
        load_block(b);
    }
}

// Gate|up with the SwiGLU epilogue (as k_dmv_glu): 256 exact threads and
// 512 weight threads, 64 rows x NB blocks of terms.
template <int WT, int PRO, int NCH, int NB>
__global__ __launch_bounds__(kSpecExact + kGluThreads) void k_dmv_glu_spec(DmvArgs A)
{
    constexpr int NS = kGluThreads;
    constexpr int WD = WT == Q4 ? 4 : 8;
    constexpr int WV = WD / 4;
    constexpr int TP = ((NB + 3) & ~3) + 4;
    constexpr int IT = NB * 64 / NS;  // weight blocks per weight thread
    constexpr bool kOne = NS % NB == 0;
    static_assert(NB % 8 == 0 && NB * 64 % NS == 0 && IT <= kGluMaxItems, "gate|up block shape");
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ SsShared ssh;
    __shared__ SgShared sgh;
    __shared__ SpecSync sy;
    __shared__ float s_out[64];
    float* T = reinterpret_cast<float*>(lds);  // 64 rows (gate, then up) x 4 lanes x TP
    const SpecLds L = spec_lds(T + 64 * 4 * TP, NB, pro_ln(PRO));
    const int tid = threadIdx.x, s = tid - kSpecExact;
    const int f = A.N / 2, nblk = f / 32;

    uint4 w[IT][WV];
    uint16_t dw[IT];
    int b = blockIdx.x;  // < nblk: the grid never exceeds the blocks
    auto load_w = [&] {
        if (s < 0) return;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int j = s + it * NS;
            const int r = j / NB, i = j - r * NB;
            const int row = r < 32 ? 32 * b + r : f + 32 * b + (r - 32);
            const size_t bi = (size_t)row * NB + i;
            const uint4* src = reinterpret_cast<const uint4*>(A.wq + bi * WD);
#pragma unroll
            for (int v = 0; v < WV; v++) w[it][v] = load_stream(src + v);
            dw[it] = load_stream(A.wd + bi);
        }
    };
    // ph 1: every item from the speculative row; -1: the items of the
    // blocks that differ, from the exact row; -2: every item from the exact
    // row (a further gate|up block of this workgroup)
    auto terms = [&](int ph) {
        if (s < 0) return;
        if (kOne && ph == -1 && !L.bad[s % NB]) return;
        StagedX x0;
        if (kOne) x0 = make_staged(load_x_block(L.row, NB, s % NB));
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int j = s + it * NS;
            const int r = j / NB, i = j - r * NB;
            if (!kOne && ph == -1 && !L.bad[i]) continue;
            float tv[4];
            q_block_terms<WT>(kOne ? x0 : make_staged(load_x_block(L.row, NB, i)), w[it], dw[it], tv);
            float* t = T + r * 4 * TP + i;
#pragma unroll
            for (int k = 0; k < 4; k++) t[k * TP] = tv[k];
        }
    };
    // thread 4r + k folds lane k of row r in block order (rows 0..31 gate,
    // 32..63 up) into s_out
    auto fold = [&](int t) {
        const float acc = seq_sum<32>(T + t * TP, NB);
        const float res = (acc + dpp_f<kDppQuadXor1>(acc)) + (dpp_f<kDppQuadXor2>(acc) + dpp_f<0x1B>(acc));
        if ((t & 3) == 0) s_out[t >> 2] = res;
    };
    // SwiGLU of element 32 b + (l & 31) from s_out, on a whole wavefront
    // (l: its lane): m = Act(Act(silu(Act(g))) * Act(u)), its code and fp16
    // delta on lanes 0-31.  Lanes 32-63 round-trip the up value beside the
    // gate chain (each half-wavefront its own 32-value block); their other
    // results are not used.
    auto swiglu = [&](int l, uint16_t* d16) {
        const float v = q8_roundtrip_lane(s_out[l], true);
        const float uq = __shfl(v, (l & 31) + 32);
        const float gs = q8_roundtrip_lane(v / (1.0f + expf_ref(-v)), true);
        return q8_quant_lane(gs * uq, true, d16);
    };
    auto store = [&](int l, int8_t q, uint16_t d16) {
        reinterpret_cast<int8_t*>(A.m_out)[32 * b + l] = q;
        if (l == 0) reinterpret_cast<uint16_t*>(A.m_out + f)[b] = d16;
        if (A.raw) {
            A.raw[32 * b + l] = s_out[l];
            A.raw[f + 32 * b + l] = s_out[32 + l];
        }
    };
    int8_t sq8 = 0;
    uint16_t sd16 = 0;
    auto spec_tail = [&](auto& bar) {
        bar();
        if (s < 64 * 4) fold(s);
        bar();
        if (s < 64) sq8 = swiglu(s, &sd16);
    };
    // the exact role's fold and epilogue from the exact terms (every exact
    // thread folds one lane of one row)
    auto exact_tail = [&] {
        fold(tid);
        lds_barrier();
        if (tid < 64) {
            uint16_t d16;
            const int8_t q = swiglu(tid, &d16);
            if (tid < 32) store(tid, q, d16);
        }
    };
    DmvArgs P = A;
    P.nb = NB;
    // Further gate|up blocks of this workgroup (when the grid holds fewer
    // workgroups than blocks) take the exact row already in place: terms by
    // the weight role, then the exact role's tail.
    // Which role is on the critical path: with Q4 weights and rms_norm the
    // weight role (its terms, fold and SwiGLU take longer than the exact
    // sum; its wavefronts issue first: TinyLlama Q4 1,593 -> 1,620 tok/s,
    // MiniCPM Q4 566 -> 569), with layer_norm the exact role (the mean's
    // sum, then the variance's; weight-first Zephyr Q4 went 1,184 -> 1,150).
    // Q8 rms_norm launches measured the same either way (TinyLlama Q8 1,399
    // -> 1,397, OpenELM Q8 1,069 -> 1,070) and keep the exact role first.
    constexpr bool kWeightFirst = !pro_ln(PRO) && WT == Q4;
    if (__builtin_amdgcn_readfirstlane(tid) < kSpecExact) {
        Q8Chunk qx[NCH];
        spec_exact<PRO, NCH, NS, spec_issue<WT, PRO>(), kWeightFirst ? 0 : 3>(P, L, ssh, sgh, sy, qx);
        lds_barrier();  // B2
        if (sy.anybad) {
            spec_exact_fixup<NCH>(P, L, qx);
            exact_tail();
        }
        for (b += gridDim.x; b < nblk; b += gridDim.x) {
            lds_barrier();
            exact_tail();
        }
    } else {
        if (kWeightFirst) __builtin_amdgcn_s_setprio(2);
        spec_weights<PRO, NCH, NS, spec_issue<WT, PRO>()>(P, L, sy, load_w, terms, spec_tail);
        lds_barrier();  // B2
        if (!sy.anybad) {
            if (s < 32) store(s, sq8, sd16);
        } else {
            // the differing blocks' terms from the exact row, then the
            // exact role's tail
            lds_barrier();  // B3
            terms(-1);
            lds_barrier();  // B4
            lds_barrier();  // the exact tail's
        }
        for (b += gridDim.x; b < nblk; b += gridDim.x) {
            load_w();
            terms(-2);
            lds_barrier();
            lds_barrier();  // the exact tail's
        }
    }
}

// ------------------------------------------------------------ launches --

namespace {

template <int WT, int PRO, int NCH, int NB>
int glu_go(DmvArgs A, size_t lds, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    auto kern = k_dmv_glu<WT, PRO, NCH, NB>;
    static int max_grid = 0;
    if (!max_grid) {
        int per_cu = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kGluThreads, lds);
        if (e != hipSuccess) return hip_fail(e, "decode matvec: occupancy");
        max_grid = std::min(kDmvMaxGrid, std::max(1, per_cu) * device_cus());
    }
    const dim3 grid(std::min(A.N / 64, max_grid));
    if (ev0)
        hipExtLaunchKernelGGL(kern, grid, dim3(kGluThreads), lds, st, ev0, ev1, 0, A);
    else
        hipLaunchKernelGGL(kern, grid, dim3(kGluThreads), lds, st, A);
    return launch_status("k_dmv_glu");
}

template <int WT, int PRO, int NCH, int NB>
int glu_spec_go(DmvArgs A, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    constexpr int TP = ((NB + 3) & ~3) + 4;
    constexpr int NT = kSpecExact + kGluThreads;
    auto kern = k_dmv_glu_spec<WT, PRO, NCH, NB>;
    const size_t lds = (size_t)64 * 4 * TP * 4 + spec_lds_bytes(NB, pro_ln(PRO));
    static int max_grid = 0;
    if (!max_grid) {
        int per_cu = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NT, lds);
        if (e != hipSuccess) return hip_fail(e, "decode matvec: occupancy");
        max_grid = std::min(kDmvMaxGrid, std::max(1, per_cu) * device_cus());
    }
    const dim3 grid(std::min(A.N / 64, max_grid));
    if (ev0)
        hipExtLaunchKernelGGL(kern, grid, dim3(NT), lds, st, ev0, ev1, 0, A);
    else
        hipLaunchKernelGGL(kern, grid, dim3(NT), lds, st, A);
    return launch_status("k_dmv_glu_spec");
}

}  // namespace

// Speculative gate|up (k_dmv_glu_spec) in place of k_dmv_glu (false builds
// the plain kernel instead).
constexpr bool kSpecGlu = true;

int glu_dispatch(const DmvArgs& A, int wdtype, int pro, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    auto go = [&](auto wt) {
        constexpr int WT = decltype(wt)::value;
        // gate|up rows of 1280, 1536, 2048 or 2304 values (40, 48, 64, 72
        // blocks); layer_norm at 2048 only
        if constexpr (kSpecGlu) {
            if (A.nb == 64) {
                switch (pro) {
                case PRO_RMS: return glu_spec_go<WT, PRO_RMS, 1, 64>(A, st, ev0, ev1);
                case PRO_RES_RMS: return glu_spec_go<WT, PRO_RES_RMS, 1, 64>(A, st, ev0, ev1);
                case PRO_LN: return glu_spec_go<WT, PRO_LN, 1, 64>(A, st, ev0, ev1);
                default: return glu_spec_go<WT, PRO_RES_LN, 1, 64>(A, st, ev0, ev1);
                }
            }
            if (A.nb == 40)
                return pro == PRO_RMS ? glu_spec_go<WT, PRO_RMS, 1, 40>(A, st, ev0, ev1)
                                      : glu_spec_go<WT, PRO_RES_RMS, 1, 40>(A, st, ev0, ev1);
            if (A.nb == 48)
                return pro == PRO_RMS ? glu_spec_go<WT, PRO_RMS, 1, 48>(A, st, ev0, ev1)
                                      : glu_spec_go<WT, PRO_RES_RMS, 1, 48>(A, st, ev0, ev1);
            return pro == PRO_RMS ? glu_spec_go<WT, PRO_RMS, 2, 72>(A, st, ev0, ev1)
                                  : glu_spec_go<WT, PRO_RES_RMS, 2, 72>(A, st, ev0, ev1);
        } else {
            const int tp = ((A.nb + 3) & ~3) + 4;
            const size_t lds = (size_t)A.nb * kStage * 4 + (size_t)A.nb * 32 * 4 + (size_t)64 * 4 * tp * 4;
            if (A.nb == 64) {
                switch (pro) {
                case PRO_RMS: return glu_go<WT, PRO_RMS, 1, 64>(A, lds, st, ev0, ev1);
                case PRO_RES_RMS: return glu_go<WT, PRO_RES_RMS, 1, 64>(A, lds, st, ev0, ev1);
                case PRO_LN: return glu_go<WT, PRO_LN, 1, 64>(A, lds, st, ev0, ev1);
                default: return glu_go<WT, PRO_RES_LN, 1, 64>(A, lds, st, ev0, ev1);
                }
            }
            if (A.nb == 40) {
                if (pro == PRO_RMS) return glu_go<WT, PRO_RMS, 1, 40>(A, lds, st, ev0, ev1);
                return glu_go<WT, PRO_RES_RMS, 1, 40>(A, lds, st, ev0, ev1);
            }
            if (A.nb == 48) {
                if (pro == PRO_RMS) return glu_go<WT, PRO_RMS, 1, 48>(A, lds, st, ev0, ev1);
                return glu_go<WT, PRO_RES_RMS, 1, 48>(A, lds, st, ev0, ev1);
            }
            if (pro == PRO_RMS) return glu_go<WT, PRO_RMS, 1, 72>(A, lds, st, ev0, ev1);
            return glu_go<WT, PRO_RES_RMS, 1, 72>(A, lds, st, ev0, ev1);
        }
    };
    return wdtype == NC_Q4 ? go(std::integral_constant<int, Q4>{}) : go(std::integral_constant<int, Q8>{});
}

}  // namespace nc
