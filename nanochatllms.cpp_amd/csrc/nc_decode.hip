// nc_decode.hip -- fused matvec kernels of the single-row decode step (Q8
// activations, Q4/Q8 weights).
//
// Each Linear of a decode step is one launch that also produces its own
// input row: the residual add of the previous Linear's output, the
// rms_norm, or SwiGLU (prologues), so a layer takes four matvec launches
// plus qkv_post and attention, and no workgroup waits for another.  Every
// workgroup computes the prologue row itself (it is a few KB, read from L2)
// while its first weights are in flight; workgroup 0 stores the residual
// row the reference keeps.  The arithmetic is exactly that of the unfused
// path (nc_matvec.hip, nc_elementwise.hip): the reference's block dot
// product and fold order, and an Act write + read wherever the reference
// stores an intermediate row:
//   residual   h = Act(a + Act(y)) (MiniCPM: y = Act(Act(y) * scale)),
//              Residual::forward, gten/modules.cpp:66-76, minicpm/minicpm.cpp:57-66
//   rms_norm   y = h / (sqrt(sum h^2 / d) + 1e-6) * g, gten/ops.cpp:830-903,
//              the sum of squares in index order (nc_seqsum.h)
//   SwiGLU     Act(Act(silu(Act(g))) * Act(u)), tinyllama/tinyllama.cpp:88-97
//   lm head    greedy token: first index of the largest logit (sampler.cpp:33-41)
// Prologue rows are handled 8 values per thread, so a 32-value Q8 block is
// one lane quad and its absmax takes two DPP steps.
//
// Workgroups walk row groups g, g + grid, ... (the grid is capped at what
// the GPU holds at once) and request the next group's weights before they
// fold the current one.
#include "nc_dmv.h"

namespace nc {

// The next step's inputs from the greedy token `tok` at position pos + 1:
// token_embed (gten/ops.cpp:526-576: a Q8 row copied, a Q4 row dequantized
// and requantized; MiniCPM then scales it, minicpm.cpp:57-58) into the
// fixed row emb_cur (and row pos + 1 of emb_rows), and the RoPE row of
// position pos + 1.  Called by all threads of one workgroup; a lane quad
// holds one 32-value block, 8 values per lane.
template <int WT, int NCH>
__device__ __forceinline__ void next_step_inputs(const DmvArgs& A, int tok, int pos)
{
    constexpr int WD = WT == Q4 ? 4 : 8;
    const int tid = threadIdx.x;
    const int nb = A.nb, K = nb * 32, nch = K / 8;
    const bool row_ok = pos + 1 < A.max_ctx;
#pragma unroll
    for (int j = 0; j < NCH; j++) {
        if (j * kDmvThreads >= nch) break;  // uniform
        const int ch = tid + j * kDmvThreads;
        const int cc = ch < nch ? ch : 0;
        const size_t blk = (size_t)tok * nb + (cc >> 2);
        const uint32_t* bw = A.emb_codes + blk * WD;
        uint32_t w[WD];
#pragma unroll
        for (int v = 0; v < WD / 4; v++) {
            const uint4 t4 = reinterpret_cast<const uint4*>(bw)[v];
            w[4 * v] = t4.x;
            w[4 * v + 1] = t4.y;
            w[4 * v + 2] = t4.z;
            w[4 * v + 3] = t4.w;
        }
        const uint16_t d16 = A.emb_deltas[blk];
        const float dw = h2f(d16);
        // element e = 8 (cc & 3) + i of the lane-permuted block: dword
        // (i & 7) >> 1 (Q8: its upper half for e >= 16), byte (i & 1) +
        // 2 (cc & 1); Q4: high nibble for e < 16
        const int hi = (cc >> 1) & 1, sh8 = 16 * (cc & 1);
        int code[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int k = (i & 7) >> 1;
            const int shift = sh8 + 8 * (i & 1);
            if (WT == Q8) {
                const uint32_t dword = hi ? w[2 * k + 1] : w[2 * k];
                code[i] = (int)(int8_t)((dword >> shift) & 0xFFu);
            } else {
                const uint32_t byte = (w[k] >> shift) & 0xFFu;
                code[i] = (hi ? (int)(byte & 0x0Fu) : (int)(byte >> 4)) - 7;
            }
        }
        Q8Chunk q;
        if (WT == Q8 && A.emb_scale == 1.0f) {
#pragma unroll
            for (int i = 0; i < 8; i++) q.q[i] = (int8_t)code[i];
            q.d16 = d16;
        } else {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = (float)code[i] * dw;
            if (A.emb_scale != 1.0f) {
                quad_roundtrip(v);
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = v[i] * A.emb_scale;
            }
            q = quad_quantize(v);
        }
        if (ch < nch) {
            store_act_chunk(A.emb_cur, K, ch, q);
            if (row_ok) store_act_chunk(A.emb_rows + (size_t)(pos + 1) * A.emb_pitch, K, ch, q);
        }
    }
    if (row_ok && tid < A.rope_half)
        reinterpret_cast<float2*>(A.rope_cur)[tid] =
                reinterpret_cast<const float2*>(A.rope_table)[(size_t)(pos + 1) * A.rope_half + tid];
}

// The greedy-token epilogue: `best` holds this thread's largest argmax key
// (0 where it holds no row result; result lanes are multiples of 4 within
// the first fold_waves waves).  Two-level reduction over the workgroups;
// the workgroup that finds the token writes it (and the next step's inputs).
template <int WT, int NCH>
__device__ __forceinline__ void argmax_epilogue(const DmvArgs& A, unsigned long long best, int pos, int fold_waves,
                                                unsigned long long* s_key, int* s_tok_p)
{
    const int tid = threadIdx.x;
    const int G = gridDim.x;
    int& s_tok = *s_tok_p;

    // Two-level reduction over the workgroups: keys in slots, the last
    // of each 32 workgroups reduces its slots and stores the group's result,
    // then reads every group's (level 2 has no counter: one round trip
    // fewer after the last group).  Keys and level-1 results are written with agent-scope atomic
    // stores (through the XCD's L2) and read with agent-scope atomic loads,
    // so they are coherent across the XCDs' L2s without a cache flush.  A
    // writer waits for its store to complete (wait_stores_done) before it
    // bumps the counter (the release of that one location, without the L2
    // write-back of a release fence), so a reader that sees the count sees
    // every key counted; the last arriver takes an agent-scope acquire fence
    // before it reads them.
    // Scratch layout (64-bit words): [0] unused, [64, 192) level-1 results
    // (zero between launches), [192, 320) level-1 counters, [320, 320 +
    // grid) workgroup keys.
    unsigned long long* sub = A.amax + 64;
    unsigned long long* cnt = A.amax + 192;
    unsigned long long* slot = A.amax + 320;
    if (tid < fold_waves * kWave) {
#pragma unroll
        for (int o = 4; o < kWave; o <<= 1) {
            const unsigned long long other = __shfl_xor(best, o);
            best = other > best ? other : best;
        }
        if ((tid & (kWave - 1)) == 0) s_key[tid / kWave] = best;
    }
    if (tid == 0) s_tok = -1;
    lds_barrier();
    if (tid == 0)
        for (int w = 1; w < fold_waves; w++) best = s_key[w] > best ? s_key[w] : best;
    const int grp = blockIdx.x >> 5;
    const int ngrp = (G + 31) >> 5;
    if (tid < kWave) {
        unsigned long long done = 0;
        if (tid == 0) {
            __hip_atomic_store(slot + blockIdx.x, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wait_stores_done();
            done = __hip_atomic_fetch_add(cnt + grp, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const int members = min(32, G - grp * 32);
        done = __shfl(done, 0);
        if (done == (unsigned long long)members - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            unsigned long long k = tid < members
                    ? __hip_atomic_load(slot + grp * 32 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                    : 0ull;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                const unsigned long long other = __shfl_xor(k, o);
                k = other > k ? other : k;
            }
            // level 2 without a counter: this group's result stored (and
            // waited for), then every group's read at once; a level-1
            // finisher that sees them all (the last one does, and any other
            // that sees them agrees) takes the token and clears them for
            // the next launch (zero: not yet written; a result is nonzero)
            if (tid == 0) {
                __hip_atomic_store(cnt + grp, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(sub + grp, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wait_stores_done();
            }
            __builtin_amdgcn_wave_barrier();
            unsigned long long b2 = 0;
            bool all = true;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int q = tid + h * kWave;
                if (q < ngrp) {
                    const unsigned long long o = __hip_atomic_load(sub + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    all = all && o != 0;
                    b2 = o > b2 ? o : b2;
                }
            }
            if (__builtin_amdgcn_ballot_w64(!all) == 0) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) {
                    const unsigned long long other = __shfl_xor(b2, o);
                    b2 = other > b2 ? other : b2;
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int q = tid + h * kWave;
                    if (q < ngrp) __hip_atomic_store(sub + q, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                if (tid == 0) {
                    const int tok = (int32_t)(0xFFFFFFFFu - (uint32_t)(b2 & 0xFFFFFFFFull));
                    A.tokens[pos + 1] = tok;
                    if (A.dpos) A.pos_out[0] = pos + 1;
                    s_tok = tok;
                }
            }
        }
    }
    if (A.emb_codes) {
        // the workgroup that found the token prepares the next step
        lds_barrier();
        const int tok = s_tok;
        if (tok >= 0) next_step_inputs<WT, NCH>(A, tok, pos);
    }
}

template <int WT, int IT, int PRO, int EPI, int NCH, int NT = kDmvThreads>
__global__ __launch_bounds__(NT) void k_dmv(DmvArgs A)
{
    constexpr int WD = WT == Q4 ? 4 : 8;
    constexpr int WV = WD / 4;
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ SsShared ssh;
    __shared__ SgShared sgh;
    __shared__ unsigned long long s_key[4];
    __shared__ int s_tok;
    const int nb = A.nb, R = A.rows;
    const int tp = ((nb + 3) & ~3) + 4;
    uint32_t* xs = lds;                                     // staged row: nb * kStage dwords
    float* T = reinterpret_cast<float*>(xs + nb * kStage);  // fold terms: R * 4 * tp
    float* sq = T + R * 4 * tp;                         // prologue scratch
    const int tid = threadIdx.x;
    const int nitems = R * nb;

    // IT: weight blocks per thread (R rows x nb blocks <= IT x NT)
    uint4 wc[IT][WV];
    uint16_t dc[IT];
    auto load_group = [&](int g, uint4(&w)[IT][WV], uint16_t(&dw)[IT]) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            // every slot loads (items past the group and rows past N: block
            // 0), so the waits for these loads are exact counts
            const int j = tid + it * NT;
            const int r = j / nb, i = j - r * nb;
            const size_t b = j < nitems && g * R + r < A.N ? (size_t)(g * R + r) * nb + i : 0;
            const uint4* src = reinterpret_cast<const uint4*>(A.wq + b * WD);
#pragma unroll
            for (int v = 0; v < WV; v++) w[it][v] = load_stream(src + v);
            dw[it] = load_stream(A.wd + b);
        }
    };
    const int G = gridDim.x;
    int g = blockIdx.x;  // < ngroups: the grid never exceeds the groups
    const int pos = dmv_prologue<PRO, NCH, false, NT>(A, xs, sq, ssh, sgh, [&] { load_group(g, wc, dc); });

    // EPI_ARGMAX: each row's lane-0 thread keeps the best key of its rows
    unsigned long long best = 0;
    for (; g < A.ngroups; g += G) {
        const int gn = g + G;
        uint4 wn[IT][WV];
        uint16_t dn[IT];
        if (gn < A.ngroups) load_group(gn, wn, dn);
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int j = tid + it * NT;
            if (j >= nitems) continue;
            const int r = j / nb, i = j - r * nb;
            float tv[4];
            q_block_terms<WT>(xs + i * kStage, wc[it], dc[it], tv);
            float* t = T + r * 4 * tp + i;
#pragma unroll
            for (int k = 0; k < 4; k++) t[k * tp] = tv[k];
        }
        lds_barrier();
        if (tid < 4 * R) {
            // thread 4r + k folds lane k of row r in block order
            const float acc = seq_sum<16>(T + tid * tp, nb);
            // lanes 4r..4r+3 hold row r's four lane sums; lane 4r reads
            // the other three with quad_perm [1,0,3,2], [2,3,0,1], [3,2,1,0]
            const float a1 = dpp_f<kDppQuadXor1>(acc);
            const float a2 = dpp_f<kDppQuadXor2>(acc);
            const float a3 = dpp_f<0x1B>(acc);
            const float res = (acc + a1) + (a2 + a3);
            const int row = g * R + (tid >> 2);
            if ((tid & 3) == 0 && row < A.N) {
                A.raw[row] = res;
                if (EPI == EPI_ARGMAX) {
                    const unsigned long long key = greedy_key(res, row);
                    best = key > best ? key : best;
                }
            }
        }
        lds_barrier();
#pragma unroll
        for (int it = 0; it < IT; it++) {
#pragma unroll
            for (int v = 0; v < WV; v++) wc[it][v] = wn[it][v];
            dc[it] = dn[it];
        }
    }

    if (EPI == EPI_ARGMAX) {
        // row results sit on lanes 4r
        argmax_epilogue<WT, NCH>(A, best, pos, (4 * R + kWave - 1) / kWave, s_key, &s_tok);
    }
}

// The norm-prologue matvec of one group of R rows per workgroup (q|k|v)
// with the weight terms and the fold computed beside the exact norm sums
// from a predicted row (nc_dmv.h: spec_exact, spec_weights): kSpecExact
// threads of the exact role and NS of the weight role, which holds the
// group's weights (IT blocks per thread; where NB divides NS a thread's
// blocks are all the same block column).  Raw fp32 outputs.
template <int WT, int IT, int PRO, int NCH, int NB, int NS>
__global__ __launch_bounds__(kSpecExact + NS) void k_dmv_spec(DmvArgs A)
{
    constexpr int WD = WT == Q4 ? 4 : 8;
    constexpr int WV = WD / 4;
    constexpr int TP = ((NB + 3) & ~3) + 4;
    constexpr bool kOne = NS % NB == 0;
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ SsShared ssh;
    __shared__ SgShared sgh;
    __shared__ SpecSync sy;
    const int R = A.rows, nitems = R * NB;
    float* T = reinterpret_cast<float*>(lds);  // R rows x 4 lanes x TP
    const SpecLds L = spec_lds(T + R * 4 * TP, NB, pro_ln(PRO));
    const int tid = threadIdx.x, s = tid - kSpecExact;
    const int col = s % NB;  // the thread's block column (kOne)

    uint4 w[IT][WV];
    uint16_t dw[IT];
    int g = blockIdx.x;
    auto load_w = [&] {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            // every slot loads (items past the group and rows past N: block
            // 0), so the waits for these loads are exact counts
            const int j = s + it * NS;
            const int r = j / NB, i = j - r * NB;
            const size_t b = j < nitems && g * R + r < A.N ? (size_t)(g * R + r) * NB + i : 0;
            const uint4* src = reinterpret_cast<const uint4*>(A.wq + b * WD);
#pragma unroll
            for (int v = 0; v < WV; v++) w[it][v] = load_stream(src + v);
            dw[it] = load_stream(A.wd + b);
        }
    };
    // ph 1: every item from the speculative row; -1: the items of a block
    // column that differs, from the exact row; -2: every item from the exact
    // row (a further group of this workgroup)
    auto terms = [&](int ph) {
        if (kOne && ph == -1 && !L.bad[col]) return;
        StagedX x0;
        if (kOne) x0 = make_staged(load_x_block(L.row, NB, col));
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int j = s + it * NS;
            if (j >= nitems) continue;
            const int r = j / NB, i = j - r * NB;
            if (!kOne && ph == -1 && !L.bad[i]) continue;
            float tv[4];
            q_block_terms<WT>(kOne ? x0 : make_staged(load_x_block(L.row, NB, i)), w[it], dw[it], tv);
            float* t = T + r * 4 * TP + i;
#pragma unroll
            for (int k = 0; k < 4; k++) t[k * TP] = tv[k];
        }
    };
    // thread 4r + k folds lane k of row r in block order; lane 4r's result
    auto fold = [&](int t) {
        const float acc = seq_sum<16>(T + t * TP, NB);
        return (acc + dpp_f<kDppQuadXor1>(acc)) + (dpp_f<kDppQuadXor2>(acc) + dpp_f<0x1B>(acc));
    };
    auto store = [&](int t, float res) {
        const int row = g * R + (t >> 2);
        if ((t & 3) == 0 && row < A.N) A.raw[row] = res;
    };
    float sres = 0.0f;
    auto spec_tail = [&](auto& bar) {
        bar();
        if (s < 4 * R) sres = fold(s);
    };
    // the exact role folds R <= 64 rows: one lane of one row per thread
    auto exact_tail = [&] {
        if (tid < 4 * R) store(tid, fold(tid));
    };
    DmvArgs P = A;
    P.nb = NB;
    if (__builtin_amdgcn_readfirstlane(tid) < kSpecExact) {
        Q8Chunk qx[NCH];
        spec_exact<PRO, NCH, NS, spec_issue<WT, PRO>()>(P, L, ssh, sgh, sy, qx);
        lds_barrier();  // B2
        if (sy.anybad) {
            spec_exact_fixup<NCH>(P, L, qx);
            exact_tail();
            lds_barrier();  // B5: the folds done (the terms may be overwritten)
        }
        for (g += gridDim.x; g < A.ngroups; g += gridDim.x) {
            lds_barrier();  // the group's terms
            exact_tail();
            lds_barrier();  // its folds done
        }
    } else {
        spec_weights<PRO, NCH, NS, spec_issue<WT, PRO>()>(P, L, sy, load_w, terms, spec_tail);
        lds_barrier();  // B2
        if (!sy.anybad) {
            if (s < 4 * R) store(s, sres);
        } else {
            lds_barrier();  // B3
            terms(-1);
            lds_barrier();  // B4
            lds_barrier();  // B5
        }
        for (g += gridDim.x; g < A.ngroups; g += gridDim.x) {
            load_w();
            terms(-2);
            lds_barrier();
            lds_barrier();
        }
    }
}

// LM heads (32000 - 122753 rows of 1280 - 2304 values) read a second copy of
// the weight in the head layout (k_head_layout): rows in groups of 16, and
// per group and chunk of E blocks (Q4: 4, Q8: 2) the 16 rows x 4 lanes'
// 16 bytes in (row, lane) order -- lane k's code dwords of the chunk's
// blocks.  A wavefront is one row group, thread (row r, lane k) one chain
// of the reference's fold (acc_k += t_k(i) for blocks i in order), and one
// 16-byte load per thread is one contiguous 1 KB per wavefront that hands
// every thread its own next E blocks: no weights or terms through LDS, and
// the staged activation block is a broadcast read.  Deltas: per group and
// 8-block chunk the 16 rows' eight deltas (16 bytes).  Wavefronts walk
// groups w, w + waves, ...; each keeps DEPTH chunks in flight across group
// boundaries, the first DEPTH requested once the norm prologue's rows have
// arrived.  Lanes 4r .. 4r + 3 then combine as (a0 + a1) + (a2 + a3) (the
// two _mm_hadd_ps of gten/ops.cpp:358-360).  The kernel is instruction-
// bound as much as memory-bound (per block and lane: three LDS reads, two
// v_dot4 and the fold's fp32 operations), so every index is a constant.
constexpr int kHdGroup = 16;  // rows per group (a wavefront)

// Blocks per 16-byte head-layout load.
template <int WT>
__host__ __device__ constexpr int head_chunk_blocks()
{
    return WT == Q4 ? 4 : 2;
}

// Chunks a thread keeps in flight: a divisor of the chunks per row (so a
// chunk's register slot is the same in every group) of 16-18.
template <int WT, int NCK>
__host__ __device__ constexpr int head_depth()
{
    return WT == Q4 ? NCK : NCK / 2;
}

// NCK: 16-byte chunks per row (K / 32 / E).  All chunk and slot indices are
// compile-time after unrolling; a wavefront's group base is wave-uniform, so
// a load's address is one scalar base plus a constant offset.
template <int WT, int PRO, int EPI, int NCH, int NCK>
__global__ __launch_bounds__(kDmvThreads) void k_dmv_head(DmvArgs A)
{
    constexpr int E = head_chunk_blocks<WT>();
    constexpr int NB = NCK * E;                // blocks per row
    constexpr int DEPTH = head_depth<WT, NCK>();
    constexpr int DW = E / 2;                  // delta dwords per chunk
    static_assert(NCK % DEPTH == 0 && NB % 8 == 0, "head layout shape");
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ SsShared ssh;
    __shared__ SgShared sgh;
    __shared__ unsigned long long s_key[4];
    __shared__ int s_tok;
    uint32_t* xs = lds;                                      // staged row: NB * kStage dwords
    float* sq = reinterpret_cast<float*>(xs + NB * kStage);  // prologue scratch: K floats
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int rr = lane >> 2, k = lane & 3;                  // row in the group, lane
    // this wavefront, the wavefronts of the grid and its groups (>= 1: the
    // grid has at most one wavefront per group), all wave-uniform
    const int gw = (int)blockIdx.x * (kDmvThreads / kWave) + __builtin_amdgcn_readfirstlane(tid / kWave);
    const int GW = (int)gridDim.x * (kDmvThreads / kWave);
    const int ngr = (A.N + kHdGroup - 1) / kHdGroup;
    const int mine = (ngr - gw + GW - 1) / GW;

    uint4 wq[DEPTH];
    uint32_t wd[DEPTH][DW];  // the chunk's E deltas
    // Group g's codes and deltas as buffer resources (scalar registers):
    // chunk c's codes at byte 1024 c (this thread's 16 at + 16 lane), its E
    // deltas at half 128 (cE / 8) + 8 rr + cE % 8 ([8-block chunk][row][8]).
    // Every load is then one VGPR offset shared by all chunks plus a
    // constant.  A resource with no records (`live` false) turns its loads
    // into zeros that read no memory: the prefetch past a wavefront's last
    // group is issued unconditionally, so the loads per iteration are fixed
    // and every wait is exact.
    auto code_rsrc = [&](int g, bool live) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(A.wq) + (size_t)g * NCK * 256, (short)0,
                                                 live ? NCK * 1024 : 0, kBufferFlags);
    };
    auto delta_rsrc = [&](int g, bool live) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A.wd) + (size_t)g * NB * kHdGroup, (short)0,
                                                 live ? NB * kHdGroup * 2 : 0, kBufferFlags);
    };
    const int qoff = lane * 16, doff = rr * 16;
    auto issue = [&](__amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rd, int c, int b) {
        const auto q = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, c * 1024, kCacheStream);
        wq[b] = make_uint4(q[0], q[1], q[2], q[3]);
        const int dc = ((c * E / 8) * 128 + (c * E) % 8) * 2;
        if (E == 4) {
            const auto t2 = __builtin_amdgcn_raw_buffer_load_b64(rd, doff, dc, 0);
            wd[b][0] = t2[0];
            wd[b][DW - 1] = t2[1];
        } else {
            wd[b][0] = __builtin_amdgcn_raw_buffer_load_b32(rd, doff, dc, 0);
        }
    };
    const int pos = dmv_prologue<PRO, NCH, true>(A, xs, sq, ssh, sgh, [&] {
        const auto rq = code_rsrc(gw, true);
        const auto rd = delta_rsrc(gw, true);
#pragma unroll
        for (int c = 0; c < DEPTH; c++) issue(rq, rd, c, c);
    });

    float acc = 0.0f;
    unsigned long long best = 0;
    // xo: zero, opaque to the compiler per group, so the staged row's LDS
    // reads stay in the loop instead of being hoisted out of it into
    // registers (all NB blocks' worth, which would halve occupancy)
    int xo = 0;
    auto consume = [&](int c, int b) {
        const uint4 q = wq[b];
        const uint32_t qd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < E; e++) {
            // lane k of the staged block: xa, xb at dwords 2k, 2k + 1, the Q4
            // offset at 8 + k, the delta at 12
            const uint32_t* st = xs + xo + (c * E + e) * kStage;
            const uint2 xv = *reinterpret_cast<const uint2*>(st + 2 * k);
            const int cx = (int)st[8 + k];
            const float dx = __uint_as_float(st[12]);
            const float dd = dx * h2f((uint16_t)(wd[b][e >> 1] >> (16 * (e & 1))));
            int L;
            if (WT == Q4) {
                const uint32_t P = qd[e];
                L = __builtin_amdgcn_sdot4((int)((P >> 4) & 0x0F0F0F0Fu), (int)xv.x, cx, false);
                L = __builtin_amdgcn_sdot4((int)(P & 0x0F0F0F0Fu), (int)xv.y, L, false);
            } else {
                L = __builtin_amdgcn_sdot4((int)qd[2 * e], (int)xv.x, 0, false);
                L = __builtin_amdgcn_sdot4((int)qd[2 * e + 1], (int)xv.y, L, false);
            }
            acc = acc + (float)L * dd;
        }
    };
    for (int gi = 0; gi < mine; gi++) {
        const int g = gw + gi * GW;
        const bool more = gi + 1 < mine;  // wave-uniform
        asm volatile("" : "+v"(xo));
        const auto rq = code_rsrc(g, true);
        const auto rd = delta_rsrc(g, true);
        const auto rqn = code_rsrc(g + GW, more);
        const auto rdn = delta_rsrc(g + GW, more);
        // each consumed chunk's slot takes the chunk DEPTH on in the stream
#pragma unroll
        for (int c = 0; c < NCK; c++) {
            consume(c, c % DEPTH);
            if (c + DEPTH < NCK)
                issue(rq, rd, c + DEPTH, c % DEPTH);
            else
                issue(rqn, rdn, c + DEPTH - NCK, c % DEPTH);
            __builtin_amdgcn_sched_barrier(0);
        }
        // the row is done: lane 4r reads the other three lanes' sums
        const float a1 = dpp_f<kDppQuadXor1>(acc);
        const float a2 = dpp_f<kDppQuadXor2>(acc);
        const float a3 = dpp_f<0x1B>(acc);
        const int row = g * kHdGroup + rr;
        if (k == 0 && row < A.N) {
            const float res = (acc + a1) + (a2 + a3);
            A.raw[row] = res;
            if (EPI == EPI_ARGMAX) {
                const unsigned long long key = greedy_key(res, row);
                best = key > best ? key : best;
            }
        }
        acc = 0.0f;
    }

    if (EPI == EPI_ARGMAX) {
        // row results sit on lanes 4r
        argmax_epilogue<WT, NCH>(A, best, pos, kDmvThreads / kWave, s_key, &s_tok);
    }
}

// Copies a Q4 / Q8 weight [N, nb blocks] (codes and deltas) into the head
// layout of k_dmv_head; rows past N (up to the group of 16) are zeros.
// Thread = one (row, block).
template <int WT>
__global__ void k_head_layout(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ wd, int N, int nb,
                              uint32_t* __restrict__ hq, uint16_t* __restrict__ hd)
{
    constexpr int WD = WT == Q4 ? 4 : 8, E = head_chunk_blocks<WT>();
    const int npad = (N + kHdGroup - 1) / kHdGroup * kHdGroup;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)npad * nb) return;
    const int r = (int)(t / nb), i = (int)(t - (int64_t)r * nb);
    const size_t g = (size_t)(r / kHdGroup);
    const int rr = r % kHdGroup;
    const bool in = r < N;
    const int nck = nb / E;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        // lane k's dwords of block i: Q4 dword k, Q8 dwords 2k and 2k + 1
        const size_t dst = (((g * nck + i / E) * kHdGroup + rr) * 4 + k) * 4;
        if (WT == Q4) {
            hq[dst + i % E] = in ? wq[((size_t)r * nb + i) * WD + k] : 0u;
        } else {
            hq[dst + 2 * (i % E)] = in ? wq[((size_t)r * nb + i) * WD + 2 * k] : 0u;
            hq[dst + 2 * (i % E) + 1] = in ? wq[((size_t)r * nb + i) * WD + 2 * k + 1] : 0u;
        }
    }
    hd[((g * (nb / 8) + i / 8) * kHdGroup + rr) * 8 + i % 8] = in ? wd[(size_t)r * nb + i] : (uint16_t)0;
}

// ============================================================ launcher ==

int device_cus()
{
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    return cus;
}

namespace {


constexpr int kDmvDirectItems = 4;  // streaming launches: weight blocks per thread and group, at most

// Row groups of a launch.  Norm prologues, where every workgroup computes
// the row's sum of squares (chains of dependent steps that workgroups
// sharing a CU slow down for each other), spread N over the CUs in one pass
// when they can: one group per workgroup, one workgroup per CU, the fewest
// rows per group that do it within kDmvMaxItems blocks per thread.  Every
// other launch streams: the most rows that fit kDmvDirectItems blocks per
// thread while there are at least two groups per CU, as many workgroups as
// the GPU holds at once.
struct DmvShape {
    int rows;
    bool spread;
};

DmvShape dmv_shape(int nb, int N, bool norm)
{
    if (norm)
        for (int r : {4, 8, 16, 32})
            if (r * nb <= kDmvThreads * kDmvMaxItems && (N + r - 1) / r <= device_cus()) return {r, true};
    int best = 0;
    for (int r : {4, 8, 16}) {
        if (r * nb > kDmvThreads * kDmvDirectItems) break;
        if (best && (N + r - 1) / r < 2 * device_cus()) break;
        best = r;
    }
    return {best, false};
}

template <int WT, int IT, int PRO, int EPI, int NCH, int NT = kDmvThreads>
int dmv_go(DmvArgs A, size_t lds, bool spread, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    auto kern = k_dmv<WT, IT, PRO, EPI, NCH, NT>;
    static int max_grid = 0;  // per instantiation: workgroups resident at once
    if (!max_grid) {
        int per_cu = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, NT, lds);
        if (e != hipSuccess) return hip_fail(e, "decode matvec: occupancy");
        max_grid = std::min(kDmvMaxGrid, std::max(1, per_cu) * device_cus());
    }
    A.ngroups = (A.N + A.rows - 1) / A.rows;
    // spread: ngroups <= CUs, one workgroup each
    const dim3 grid(spread ? A.ngroups : std::min(A.ngroups, max_grid));
    if (ev0)
        hipExtLaunchKernelGGL(kern, grid, dim3(NT), lds, st, ev0, ev1, 0, A);
    else
        hipLaunchKernelGGL(kern, grid, dim3(NT), lds, st, A);
    return launch_status("k_dmv");
}

// LM heads in the head layout, rows of NCK chunks.
template <int WT, int PRO, int EPI, int NCH, int NCK>
int head_go(DmvArgs A, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    auto kern = k_dmv_head<WT, PRO, EPI, NCH, NCK>;
    const size_t lds = (size_t)A.nb * kStage * 4 + (size_t)A.nb * 32 * 4;
    static int max_grid = 0;  // workgroups resident at once
    if (!max_grid) {
        int per_cu = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kDmvThreads, lds);
        if (e != hipSuccess) return hip_fail(e, "decode matvec: occupancy");
        max_grid = std::min(kDmvMaxGrid, std::max(1, per_cu) * device_cus());
    }
    if (A.nb != NCK * head_chunk_blocks<WT>() || A.N < kHdGroup * (kDmvThreads / kWave))
        return fail(NC_ERR_ARG, "decode matvec: lm head of %d x %d blocks", A.N, A.nb);
    A.rows = kHdGroup;
    A.ngroups = (A.N + kHdGroup - 1) / kHdGroup;
    // every wavefront owns at least one group of 16 rows
    const dim3 grid(std::min(A.ngroups / (kDmvThreads / kWave), max_grid));
    if (ev0)
        hipExtLaunchKernelGGL(kern, grid, dim3(kDmvThreads), lds, st, ev0, ev1, 0, A);
    else
        hipLaunchKernelGGL(kern, grid, dim3(kDmvThreads), lds, st, A);
    return launch_status("k_dmv_head");
}

// The speculative q|k|v launch (k_dmv_spec): one group of R rows per
// workgroup, every workgroup resident at once.
template <int WT, int IT, int PRO, int NCH, int NB, int NS>
int dmv_spec_go(DmvArgs A, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    constexpr int TP = ((NB + 3) & ~3) + 4;
    auto kern = k_dmv_spec<WT, IT, PRO, NCH, NB, NS>;
    const size_t lds = (size_t)A.rows * 4 * TP * 4 + spec_lds_bytes(NB, pro_ln(PRO));
    A.ngroups = (A.N + A.rows - 1) / A.rows;
    const dim3 grid(A.ngroups);
    const dim3 block(kSpecExact + NS);
    if (ev0)
        hipExtLaunchKernelGGL(kern, grid, block, lds, st, ev0, ev1, 0, A);
    else
        hipLaunchKernelGGL(kern, grid, block, lds, st, A);
    return launch_status("k_dmv_spec");
}

// Speculative q|k|v (k_dmv_spec) for norm-prologue launches of rows of 2048
// values spread one group per CU with four blocks per weight thread
// (TinyLlama's 16-row groups: 1,489 -> 1,506 tok/s in an on-box A/B).  With
// fewer blocks per thread the weight terms are too short to hide much of
// the exact sum, and the wider workgroup costs more than it saves (OpenELM's
// 8-row groups: 1,059 -> 1,046 tok/s), so those keep k_dmv.
constexpr bool kSpecQkv = true;
// The same for 32-row groups of 2048-value rows (Zephyr's q|k|v) over 512
// weight threads: Zephyr-Q4 1,072 -> 1,086 tok/s, Zephyr-Q8 970 -> 1,009 in
// an on-box A/B.  MiniCPM's (rows of 2304 values, five blocks per weight
// thread) measured no gain (563 -> 562) and keeps k_dmv.
constexpr bool kSpecQkvWide = true;

// Launch with the items per thread the group needs (1, 2, 4, 8 or 12).
template <int WT, int PRO, int EPI, int NCH>
int dmv_r(DmvArgs A, size_t lds0, DmvShape sh, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    const int tp = ((A.nb + 3) & ~3) + 4;
    const size_t lds = lds0 + (size_t)sh.rows * 4 * tp * 4;
    A.rows = sh.rows;
    const int items = (sh.rows * A.nb + kDmvThreads - 1) / kDmvThreads;
    if (items <= 1) return dmv_go<WT, 1, PRO, EPI, NCH>(A, lds, sh.spread, st, ev0, ev1);
    if (items <= 2) return dmv_go<WT, 2, PRO, EPI, NCH>(A, lds, sh.spread, st, ev0, ev1);
    if (items <= 4) return dmv_go<WT, 4, PRO, EPI, NCH>(A, lds, sh.spread, st, ev0, ev1);
    if (items <= 8) return dmv_go<WT, 8, PRO, EPI, NCH>(A, lds, sh.spread, st, ev0, ev1);
    return dmv_go<WT, 12, PRO, EPI, NCH>(A, lds, sh.spread, st, ev0, ev1);
}

// Norm-prologue launches spread one group per CU whose groups hold more than
// four blocks per thread at 256 threads (MiniCPM's q|k|v: 32 rows x 72
// blocks) run 512 threads: the block terms and the prologue's elementwise
// work take half as long per thread, one 8-value chunk per thread up to 4096
// values.  At four blocks or fewer (TinyLlama's, OpenELM's q|k|v) the wider
// workgroup measured slower.
constexpr int kDmvWideThreads = 512;

template <int WT, int PRO>
int dmv_r_wide(DmvArgs A, size_t lds0, DmvShape sh, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    constexpr int NT = kDmvWideThreads;
    const int tp = ((A.nb + 3) & ~3) + 4;
    const size_t lds = lds0 + (size_t)sh.rows * 4 * tp * 4;
    A.rows = sh.rows;
    const int items = (sh.rows * A.nb + NT - 1) / NT;
    if (items <= 1) return dmv_go<WT, 1, PRO, EPI_RAW, 1, NT>(A, lds, sh.spread, st, ev0, ev1);
    if (items <= 2) return dmv_go<WT, 2, PRO, EPI_RAW, 1, NT>(A, lds, sh.spread, st, ev0, ev1);
    if (items <= 4) return dmv_go<WT, 4, PRO, EPI_RAW, 1, NT>(A, lds, sh.spread, st, ev0, ev1);
    return dmv_go<WT, 6, PRO, EPI_RAW, 1, NT>(A, lds, sh.spread, st, ev0, ev1);
}

// The launch for a prologue kind known at run time; layer_norm (PRO_LN,
// PRO_RES_LN) at one 8-value chunk per thread only.
template <int NCH, class Go>
int with_pro(int pro, Go&& go)
{
    switch (pro) {
    case PRO_RMS: return go(std::integral_constant<int, PRO_RMS>{});
    case PRO_RES_RMS: return go(std::integral_constant<int, PRO_RES_RMS>{});
    default:
        if constexpr (NCH == 1) {
            if (pro == PRO_LN) return go(std::integral_constant<int, PRO_LN>{});
            return go(std::integral_constant<int, PRO_RES_LN>{});
        } else {
            return fail(NC_ERR_ARG, "decode matvec: layer_norm prologue over more than 2048 values");
        }
    }
}

template <int WT>
int dmv_dispatch(const DmvArgs& A, int pro, int epi, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    const size_t K = (size_t)A.nb * 32;
    const bool norm = pro_norm(pro);
    const DmvShape R = dmv_shape(A.nb, A.N, norm);
    const bool two = K > (size_t)kDmvThreads * 8;  // norm prologue: two 8-value chunks per thread
    // staged row (kStage dwords per block), the fold terms, then the norm
    // prologue's squares / Act row
    const size_t lds0 = (size_t)A.nb * kStage * 4 + (norm ? K * 4 : 0);
    if (epi == EPI_SWIGLU) return glu_dispatch(A, WT == Q4 ? NC_Q4 : NC_Q8, pro, st, ev0, ev1);
    if (A.head) {
        // an lm head in the head layout: one fold chain per thread, the
        // weights streamed straight into registers
        if (!pro_res(pro) || epi == EPI_SWIGLU)
            return fail(NC_ERR_ARG, "decode matvec: head layout with prologue %d epilogue %d", pro, epi);
        // rows of 2048 (one 8-value chunk per thread in the prologue) or
        // 2304 values (two)
        constexpr int E = head_chunk_blocks<WT>();
        if (A.nb == 64)
            return with_pro<1>(pro, [&](auto p) {
                constexpr int P = decltype(p)::value;
                if (epi == EPI_ARGMAX) return head_go<WT, P, EPI_ARGMAX, 1, 64 / E>(A, st, ev0, ev1);
                return head_go<WT, P, EPI_RAW, 1, 64 / E>(A, st, ev0, ev1);
            });
        if (A.nb == 72 && pro == PRO_RES_RMS) {
            if (epi == EPI_ARGMAX) return head_go<WT, PRO_RES_RMS, EPI_ARGMAX, 2, 72 / E>(A, st, ev0, ev1);
            return head_go<WT, PRO_RES_RMS, EPI_RAW, 2, 72 / E>(A, st, ev0, ev1);
        }
        // OpenELM's narrower rows (1280, 1536 values)
        if (A.nb == 40 && pro == PRO_RES_RMS) {
            if (epi == EPI_ARGMAX) return head_go<WT, PRO_RES_RMS, EPI_ARGMAX, 1, 40 / E>(A, st, ev0, ev1);
            return head_go<WT, PRO_RES_RMS, EPI_RAW, 1, 40 / E>(A, st, ev0, ev1);
        }
        if (A.nb == 48 && pro == PRO_RES_RMS) {
            if (epi == EPI_ARGMAX) return head_go<WT, PRO_RES_RMS, EPI_ARGMAX, 1, 48 / E>(A, st, ev0, ev1);
            return head_go<WT, PRO_RES_RMS, EPI_RAW, 1, 48 / E>(A, st, ev0, ev1);
        }
        return fail(NC_ERR_ARG, "decode matvec: head layout rows of %d blocks, prologue %d", A.nb, pro);
    }
    if (pro == PRO_X) return dmv_r<WT, PRO_X, EPI_RAW, 1>(A, lds0, R, st, ev0, ev1);
    if (epi == EPI_ARGMAX) {
        if (two)
            return with_pro<2>(pro, [&](auto p) {
                return dmv_r<WT, decltype(p)::value, EPI_ARGMAX, 2>(A, lds0, R, st, ev0, ev1);
            });
        return with_pro<1>(
            pro, [&](auto p) { return dmv_r<WT, decltype(p)::value, EPI_ARGMAX, 1>(A, lds0, R, st, ev0, ev1); });
    }
    if (kSpecQkv && R.spread && A.nb == 64 && R.rows * A.nb == kDmvThreads * 4) {
        DmvArgs As = A;
        As.rows = R.rows;
        return with_pro<1>(
            pro, [&](auto p) { return dmv_spec_go<WT, 4, decltype(p)::value, 1, 64, kDmvThreads>(As, st, ev0, ev1); });
    }
    if (kSpecQkvWide && R.spread && R.rows == 32 && A.nb == 64) {
        DmvArgs As = A;
        As.rows = R.rows;
        return with_pro<1>(pro, [&](auto p) {
            return dmv_spec_go<WT, 4, decltype(p)::value, 1, 64, kDmvWideThreads>(As, st, ev0, ev1);
        });
    }
    if (R.spread && R.rows * A.nb > kDmvThreads * 4 && R.rows * A.nb <= kDmvWideThreads * 6) {
        if (K > (size_t)kDmvWideThreads * 8) {
            // more than one 8-value chunk per thread: rms_norm only
            if (pro == PRO_RMS) return dmv_r_wide<WT, PRO_RMS>(A, lds0, R, st, ev0, ev1);
            if (pro == PRO_RES_RMS) return dmv_r_wide<WT, PRO_RES_RMS>(A, lds0, R, st, ev0, ev1);
            return fail(NC_ERR_ARG, "decode matvec: layer_norm prologue over %zu values", K);
        }
        return with_pro<1>(
            pro, [&](auto p) { return dmv_r_wide<WT, decltype(p)::value>(A, lds0, R, st, ev0, ev1); });
    }
    if (two)
        return with_pro<2>(
            pro, [&](auto p) { return dmv_r<WT, decltype(p)::value, EPI_RAW, 2>(A, lds0, R, st, ev0, ev1); });
    return with_pro<1>(
        pro, [&](auto p) { return dmv_r<WT, decltype(p)::value, EPI_RAW, 1>(A, lds0, R, st, ev0, ev1); });
}

}  // namespace

bool decode_matvec_supported(int wdtype, int K, int N, int pro, int epi)
{
    if (wdtype != NC_Q4 && wdtype != NC_Q8) return false;
    if (pro < PRO_X || pro > PRO_RES_LN || epi < EPI_RAW || epi > EPI_SWIGLU) return false;
    const bool norm = pro_norm(pro);
    // layer_norm: rows of 2048 values (its mean is the workgroup's exact
    // sum over one 8-value chunk per thread)
    if (pro_ln(pro) && K != 2048) return false;
    if (K <= 0 || K % 32 || N <= 0 || !dmv_shape(K / 32, N, norm).rows) return false;
    if (norm && (K % kSsThreads || K > kDmvThreads * 8 * kDmvNormChunks)) return false;
    if (epi == EPI_ARGMAX && !norm) return false;
    if (epi == EPI_SWIGLU && (N % 64 || (K != 1280 && K != 1536 && K != 2048 && K != 2304) || !norm)) return false;
    return true;
}

bool head_layout_supported(int wdtype, int N, int K)
{
    if (wdtype != NC_Q4 && wdtype != NC_Q8) return false;
    return (K == 1280 || K == 1536 || K == 2048 || K == 2304) && N >= kHdGroup * (kDmvThreads / kWave);
}

int head_layout_bytes(int wdtype, int N, int K, size_t* code_bytes, size_t* delta_bytes)
{
    const size_t npad = (size_t)(N + kHdGroup - 1) / kHdGroup * kHdGroup, nb = (size_t)K / 32;
    *code_bytes = npad * nb * (wdtype == NC_Q4 ? 16 : 32);
    *delta_bytes = npad * nb * 2;
    return NC_OK;
}

int head_layout_launch(const nc_tensor* w, void* codes, void* deltas, hipStream_t st)
{
    if (!head_layout_supported(w->dtype, w->rows, w->cols))
        return fail(NC_ERR_ARG, "head layout: [%d x %d] dtype %d", w->rows, w->cols, w->dtype);
    const int nb = w->cols / 32;
    const int64_t n = (int64_t)(w->rows + kHdGroup - 1) / kHdGroup * kHdGroup * nb;
    const dim3 grid((unsigned)((n + 255) / 256));
    if (w->dtype == NC_Q4)
        hipLaunchKernelGGL(k_head_layout<Q4>, grid, dim3(256), 0, st, (const uint32_t*)w->data,
                           (const uint16_t*)w->deltas, w->rows, nb, (uint32_t*)codes, (uint16_t*)deltas);
    else
        hipLaunchKernelGGL(k_head_layout<Q8>, grid, dim3(256), 0, st, (const uint32_t*)w->data,
                           (const uint16_t*)w->deltas, w->rows, nb, (uint32_t*)codes, (uint16_t*)deltas);
    return launch_status("k_head_layout");
}

namespace {
float g_spec_skew = 1.0f;
int* g_spec_fixups = nullptr;
}  // namespace

int decode_matvec(const DmvArgs& A0, int wdtype, int pro, int epi, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1)
{
    if (!decode_matvec_supported(wdtype, A0.nb * 32, A0.N, pro, epi))
        return fail(NC_ERR_ARG, "decode matvec: unsupported [%d x %d] dtype %d prologue %d epilogue %d", A0.N,
                    A0.nb * 32, wdtype, pro, epi);
    DmvArgs A = A0;
    A.spec_skew = g_spec_skew;
    A.spec_fixups = g_spec_fixups;
    return wdtype == NC_Q4 ? dmv_dispatch<Q4>(A, pro, epi, st, ev0, ev1) : dmv_dispatch<Q8>(A, pro, epi, st, ev0, ev1);
}

// The next step's inputs for a token another kernel chose: the position is
// read from A.pos_out (already advanced to the token's position p), the
// token from A.tokens[p]; the embedding and RoPE rows are those the argmax
// epilogue prepares for position p.
template <int WT, int NCH>
__global__ __launch_bounds__(kDmvThreads) void k_next_inputs(DmvArgs A)
{
    const int p = load_pos(A.pos_out);
    next_step_inputs<WT, NCH>(A, A.tokens[p], p - 1);
}

int next_inputs_launch(const DmvArgs& A, int wdtype, hipStream_t st)
{
    const int K = A.nb * 32;
    if ((wdtype != NC_Q4 && wdtype != NC_Q8) || K % 32 || K > 2 * kDmvThreads * 8 || !A.pos_out || !A.tokens ||
        !A.emb_codes)
        return fail(NC_ERR_ARG, "next inputs: unsupported (dtype %d, %d values)", wdtype, K);
    const bool two = K > kDmvThreads * 8;
    auto kern = wdtype == NC_Q4 ? (two ? k_next_inputs<Q4, 2> : k_next_inputs<Q4, 1>)
                                : (two ? k_next_inputs<Q8, 2> : k_next_inputs<Q8, 1>);
    hipLaunchKernelGGL(kern, dim3(1), dim3(kDmvThreads), 0, st, A);
    return launch_status("k_next_inputs");
}

}  // namespace nc

extern "C" int nc_debug_spec(float skew, void* fixups)
{
    NC_CHECK_ARG(skew > 0.0f && skew < 1e30f, "debug_spec: skew %g", (double)skew);
    nc::g_spec_skew = skew;
    nc::g_spec_fixups = static_cast<int*>(fixups);
    return NC_OK;
}
