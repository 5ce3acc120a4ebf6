// nc_seqsum.h -- the reference's left-to-right fp32 sum of non-negative
// terms (sum of squares of rms_norm, gten/ops.cpp:833-835), computed by a
// whole workgroup with the result of the sequential loop, bit for bit.
//
// Why it can be parallel: while the running sum s stays inside one binade
// [2^E, 2^(E+1)) every step rounds to the same grid of spacing
// u = ulp(2^E), so s + t rounds to s + u * D with D an integer that depends
// on t and on one bit of state, the parity of s / u (the tie case of round-
// to-nearest-even).  A run of such steps is therefore a map
//     parity p  ->  C_p units added          (p = 0, 1)
// and runs compose associatively:  (A then B)_p = A_p + B_{(p + A_p) & 1}.
// A run's map is read off two representatives, an even and an odd value of
// the binade: each takes the run's fp32 adds, and C_p is how far its bit
// pattern moved (consecutive grid values have consecutive bit patterns).
// The representatives start at the predicted running sum, so they stay in
// the binade whenever the prediction is right; one that leaves it voids
// the map.
// Steps that leave the binade ("crossings") are few -- the sum of
// non-negative terms only grows, so at most one per binade passed -- and
// are replayed exactly, one fp32 add each, by a single lane.
//
// Which steps cross is predicted from an approximate prefix sum; every
// segment between crossings is then checked to start and end inside the
// binade it was computed for, which makes every one of its steps exact.  A
// failed check (a prefix sum within rounding distance of a power of two,
// infinities, too many crossings) falls back to the plain sequential loop.
#pragma once

#include "nc_device.h"

namespace nc {

// Binade index used for the rounding grid: the biased exponent, with zero
// and subnormals sharing binade 1's grid (spacing 2^-149).
NC_HD int ss_binade(float x)
{
    const int e = (int)(__builtin_bit_cast(uint32_t, x) >> 23);
    return e < 1 ? 1 : e;
}

// Parity map of a run of in-binade steps: c[p] grid units added when the
// run starts on a value of parity p.  nz: the run holds a nonzero term (a
// run of zeros is the identity on any grid and needs no binade check).
struct SsMap {
    int c0, c1;
    bool nz;
};

NC_HD SsMap ss_identity() { return SsMap{0, 0, false}; }

NC_HD SsMap ss_compose(const SsMap& a, const SsMap& b)
{
    SsMap r;
    r.c0 = a.c0 + ((a.c0 & 1) ? b.c1 : b.c0);
    r.c1 = a.c1 + ((a.c1 & 1) ? b.c0 : b.c1);
    r.nz = a.nz || b.nz;
    return r;
}

// First value above binade E (1 <= E <= 254): 2^(E-126); binade 254's is
// +inf, and E = 255 (inf, NaN) gets -0, below everything.  A representative
// r of E stays inside it while r < ss_top(E) (it only grows).
NC_HD float ss_top(int E) { return __builtin_bit_cast(float, (uint32_t)(E + 1) << 23); }

// Representatives of a run that starts near p: the even bit pattern at or
// below p's (same binade: binade boundaries are even patterns) and the next.
NC_HD int ss_rep_base(float p) { return __builtin_bit_cast(int, p) & ~1; }

// Applies a segment map computed for binade E to the exact value s.
// Within binade E consecutive grid values have consecutive bit patterns
// (E = 1 spans the subnormals too), so s + u C is bits(s) + C and the
// parity of s / u is the last bit.  Returns false when s does not lie in E
// or the result leaves it.
NC_HD bool ss_apply(float& s, const SsMap& m, int E)
{
    if (!m.nz) return true;
    if (E >= 255 || ss_binade(s) != E) return false;  // infinities and NaNs take the plain loop
    const int sb = __builtin_bit_cast(int, s);
    const float r = __builtin_bit_cast(float, sb + ((sb & 1) ? m.c1 : m.c0));
    if (ss_binade(r) != E) return false;
    s = r;
    return true;
}

#if defined(__HIPCC__)

constexpr int kSsThreads = 256;   // workgroup size the block sum is written for
constexpr int kSsMaxPer = 16;     // terms per thread: n <= 4096
constexpr int kSsMaxCross = 63;   // crossings handled before the fallback
constexpr int kSsMaxRec = 4;      // crossings one thread's chunk may hold before the fallback
constexpr int kSsWaveRec = 16;    // crossings one wavefront's chunks may hold before the fallback (16 x 4 = 64 lanes)
constexpr int kSsHead = 8;        // chunks in the head

static_assert(kSsWaveRec * (kSsThreads / kWave) == kWave, "one lane per record slot in the replay");

// Crossing record flags (next to the binade in a record's third word).
constexpr int kSsRecNz = 0x100;    // the record's map holds a nonzero term
constexpr int kSsRecBack = 0x200;  // its segment opened in an earlier wavefront

struct SsShared {
    // the wave arrays are read as one 16-byte vector each: keep them first
    float wf[kSsThreads / kWave];
    int wc0[kSsThreads / kWave], wc1[kSsThreads / kWave], wfl[kSsThreads / kWave], wcnt[kSsThreads / kWave];
    // per wavefront, its crossing records in order: the map (c0, c1) of the
    // segment that ends at the crossing, binade | flags, the crossing term's bits
    int4 rec[kSsThreads / kWave][kSsWaveRec];
    int ok;
    float result;
    float head;  // the exact sum of the head chunks
    int tail_e;  // the binade of the segment after the last crossing
};

// Segmented scan element: a parity map and flags (bit 0: nz, bit 1: the
// element holds a crossing, i.e. its map restarts the open segment).
struct SsSeg {
    int c0, c1, f, n;  // n: crossings so far (a plain sum, not segmented)
};

// (a then b): b alone when b restarts, else the composition.
// Written with bit selects (no branches): p0, p1 are all ones where a's
// count is odd (b then starts on the other parity), rb where b restarts.
__device__ __forceinline__ SsSeg ss_seg(const SsSeg& a, const SsSeg& b)
{
    const int p0 = -(a.c0 & 1), p1 = -(a.c1 & 1);
    const int c0 = a.c0 + ((p0 & b.c1) | (~p0 & b.c0));
    const int c1 = a.c1 + ((p1 & b.c0) | (~p1 & b.c1));
    const int rb = -((b.f >> 1) & 1);
    return SsSeg{(rb & b.c0) | (~rb & c0), (rb & b.c1) | (~rb & c1), b.f | (~rb & a.f), a.n + b.n};
}

template <int CTRL, int ROW_MASK = 0xf, bool BZ = true>
__device__ __forceinline__ SsSeg ss_dpp(const SsSeg& x)
{
    // lanes without a source get 0s: the identity element
    return SsSeg{dpp_i<CTRL, ROW_MASK, BZ>(x.c0), dpp_i<CTRL, ROW_MASK, BZ>(x.c1), dpp_i<CTRL, ROW_MASK, BZ>(x.f),
                 dpp_i<CTRL, ROW_MASK, BZ>(x.n)};
}

// Inclusive wave scans (row_shr steps within rows of 16, then the row
// broadcasts), with DPP moves instead of LDS permutes.
__device__ __forceinline__ float wave_scan_add(float v)
{
    v = v + dpp_f<0x111>(v);
    v = v + dpp_f<0x112>(v);
    v = v + dpp_f<0x114>(v);
    v = v + dpp_f<0x118>(v);
    v = v + dpp_f<kDppBcast15, 0xa, false>(v);
    v = v + dpp_f<kDppBcast31, 0xc, false>(v);
    return v;
}
__device__ __forceinline__ SsSeg wave_scan_seg(SsSeg x)
{
    x = ss_seg(ss_dpp<0x111>(x), x);
    x = ss_seg(ss_dpp<0x112>(x), x);
    x = ss_seg(ss_dpp<0x114>(x), x);
    x = ss_seg(ss_dpp<0x118>(x), x);
    x = ss_seg(ss_dpp<kDppBcast15, 0xa, false>(x), x);
    x = ss_seg(ss_dpp<kDppBcast31, 0xc, false>(x), x);
    return x;
}

// Sum of t[0..n) in index order, as the sequential fp32 loop computes it,
// for t >= 0 in LDS; n a multiple of 256, n <= 4096.  Called by every
// thread of a workgroup of 256 or more threads (the first 256 compute, the
// others only join the barriers); every thread returns the sum.  *fast (thread
// 0's view) tells whether the parallel path was taken.  Synchronizes the
// workgroup through LDS barriers only (global loads may stay in flight).
//
// Thread j owns the j-th chunk of c terms.  The first kSsHead chunks (the
// region where the running sum crosses binades most often) form the head:
// their threads only feed the prediction, and the last thread adds the head
// exactly (the start of everything after it).  Every later thread walks its
// chunk once: binade predicted from an approximate prefix, step maps
// composed, and up to four crossings recorded (more fall back).  A segmented
// scan joins the chunks of a wavefront, which stores its records at once;
// after one barrier every computing wavefront composes the four wavefronts'
// open segments and replays the few records in order.
//
// The barrier among the 256 threads is a functor: the workgroup's LDS
// barrier, or SsWaveBarrier when the first four wavefronts compute the sum
// while the others do work of their own.
struct SsLdsBarrier {
    __device__ void operator()() { lds_barrier(); }
};

// Barrier among the first NW wavefronts through an LDS counter (zeroed by
// a workgroup barrier before each sum that uses it): each wavefront adds one
// and waits until the count reaches NW times the number of barriers passed.
// LDS traffic only (global loads stay in flight across it).
template <int NW>
struct SsWaveBarrier {
    int* cnt;
    int gen;
    __device__ void operator()()
    {
        gen += NW;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if ((threadIdx.x & (kWave - 1)) == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < gen) {
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
};

// Phase one of the sum, threads 0..255 with their chunk of c terms in v:
// the chunks' approximate inclusive prefix within the wavefront (returned)
// and the wavefront totals in sh.wf.  A barrier must follow before
// block_seq_sum_after.
template <int C>
__device__ __forceinline__ float ss_prefix(const float (&v)[kSsMaxPer], int c, SsShared& sh)
{
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    // chunk sum in order (a prediction only)
    float cs = 0.0f;
#pragma unroll
    for (int k = 0; k < kSsMaxPer; k++)
        if (k < c) cs = cs + v[k];
    // ---- approximate inclusive prefix I of the chunk sums.  Neighbouring
    // threads must agree bit for bit on the value at their shared boundary
    // (thread j's last step ends where thread j + 1's first starts): within
    // a wave the exclusive value is the previous lane's I, and across waves
    // I = local + WP with WP_w = ((0 + wf_0) + wf_1) + ... + wf_{w-1}, so the
    // last lane's wf_{w-1} + WP_{w-1} equals the next wave's WP_w.
    const float I = wave_scan_add(cs);
    if (lane == kWave - 1) sh.wf[w] = I;
    return I;
}

// The rest of the sum after ss_prefix and a barrier (threads 0..255): the
// terms t[0..n) also in LDS (the head and the fallback read them there).
// Every computing thread returns the sum.  BCAST: a barrier after the
// replay publishes the result and sh.ok, for threads past the first 256 that
// take the barriers without computing.  FINAL: end with a barrier after which
// sh may be reused (without it, sh must not be written again by this
// workgroup).
template <int C, bool FINAL, bool BCAST, class Bar>
__device__ __forceinline__ float block_seq_sum_after(const float (&v)[kSsMaxPer], float I, const float* t, int n,
                                                     SsShared& sh, bool* fast, Bar& bar)
{
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const int c = C ? C : n / kSsThreads;
    const int nh = kSsHead * c;  // head terms
    float WP = 0.0f;
    {
        const float4 F = *reinterpret_cast<const float4*>(sh.wf);  // every wave's total at once
        const float f[4] = {F.x, F.y, F.z, F.w};
        static_assert(kSsThreads / kWave == 4, "four wave totals");
#pragma unroll
        for (int q = 0; q < 3; q++)
            if (q < w) WP = WP + f[q];
    }
    I = I + WP;
    float A = dpp_f<kDppWaveShr1>(I);  // the previous lane's I
    if (lane == 0) A = WP;
    // ---- walk (threads >= 1): binade of each step predicted from the
    // approximate prefix; in-binade steps taken by the two representatives
    // (r0 even, r1 odd, from bit pattern b0), crossing steps recorded with
    // the map before them.  Steps before the last only grow the prefix, so
    // one compare finds their crossings; the last step's prefix is I, which
    // may round below the walked one.
    int c0 = 0, c1 = 0, nz = 0, ncross = 0, bad = 0;
    int4 rec[kSsMaxRec];  // (c0, c1, binade or 0, term bits) of this chunk's crossings
#pragma unroll
    for (int q = 0; q < kSsMaxRec; q++) rec[q] = make_int4(0, 0, 0, 0);
    if (tid >= kSsHead) {
        float P = A;
        int Eb = ss_binade(A);
        float top = ss_top(Eb);
        int b0 = ss_rep_base(A);
        float r0 = __builtin_bit_cast(float, b0), r1 = __builtin_bit_cast(float, b0 | 1);
        uint32_t nzb = 0;  // OR of the open run's term bits
#pragma unroll
        for (int k = 0; k < kSsMaxPer; k++) {
            if (k < c) {
                const float x = v[k];
                const bool last = k + 1 == c;
                const float Pa = last ? I : P + x;
                const bool cross = last ? ss_binade(Pa) != Eb : !(Pa < top);
                const float n0 = r0 + x, n1 = r1 + x;
                const uint32_t nn = nzb | __builtin_bit_cast(uint32_t, x);
                if (__builtin_amdgcn_ballot_w64(cross)) {
                    if (cross) {
                        bad |= !(r1 < top) ? 1 : 0;
                        const int4 r = make_int4(__builtin_bit_cast(int, r0) - b0,
                                                 __builtin_bit_cast(int, r1) - (b0 | 1), nzb ? Eb : 0,
                                                 __builtin_bit_cast(int, x));
#pragma unroll
                        for (int q = 0; q < kSsMaxRec; q++)
                            if (ncross == q) rec[q] = r;
                        ncross++;
                        Eb = ss_binade(Pa);
                        top = ss_top(Eb);
                        b0 = ss_rep_base(Pa);
                        r0 = __builtin_bit_cast(float, b0);
                        r1 = __builtin_bit_cast(float, b0 | 1);
                        nzb = 0;
                    } else {
                        r0 = n0;
                        r1 = n1;
                        nzb = nn;
                    }
                } else {
                    r0 = n0;
                    r1 = n1;
                    nzb = nn;
                }
                P = Pa;
            }
        }
        bad |= !(r1 < top) ? 1 : 0;
        c0 = __builtin_bit_cast(int, r0) - b0;
        c1 = __builtin_bit_cast(int, r1) - (b0 | 1);
        nz = nzb ? 1 : 0;
    }
    // the head's exact sum, by the last thread (after its own chunk), and the
    // binade of the segment after the last crossing (the prefix at the end)
    if (tid == kSsThreads - 1) {
        sh.head = seq_sum(t, nh);
        sh.tail_e = ss_binade(I);
    }
    // ---- segmented scan of (open map, has-crossing) and scan of the counts,
    // within the wavefront
    SsSeg x{c0, c1, nz | (ncross > 0 ? 2 : 0), ncross};
    x = wave_scan_seg(x);
    // a chunk with too many crossings or a representative that left its
    // binade takes the plain loop
    const int over = __builtin_amdgcn_ballot_w64(ncross > kSsMaxRec || bad) != 0;
    // the open segment entering this chunk (from the wavefront's start), and
    // the wavefront's crossings before it
    SsSeg in = ss_dpp<kDppWaveShr1>(x);
    if (lane == 0) in = SsSeg{0, 0, 0, 0};
    const int base = in.n;
    if (ncross > 0) {
        // the first crossing closes the segment open at the chunk start (its
        // binade: no crossing before it in this chunk); when that segment
        // opened before this wavefront, the replay composes the earlier
        // wavefronts' part in front of it (kSsRecBack)
        const SsMap m0 = ss_compose(SsMap{in.c0, in.c1, (in.f & 1) != 0}, SsMap{rec[0].x, rec[0].y, rec[0].z != 0});
        rec[0] = make_int4(m0.c0, m0.c1, ss_binade(A) | (m0.nz ? kSsRecNz : 0) | ((in.f & 2) ? 0 : kSsRecBack),
                           rec[0].w);
#pragma unroll
        for (int q = 1; q < kSsMaxRec; q++) rec[q].z = rec[q].z ? (rec[q].z | kSsRecNz) : 0;
#pragma unroll
        for (int q = 0; q < kSsMaxRec; q++)
            if (q < ncross && base + q < kSsWaveRec) sh.rec[w][base + q] = rec[q];
    }
    if (lane == kWave - 1) {
        sh.wc0[w] = x.c0;
        sh.wc1[w] = x.c1;
        sh.wfl[w] = x.f;
        sh.wcnt[w] = x.n | (over << 30);
    }
    bar();
    // ---- replay, on every computing wavefront (no barrier needed after
    // it).  Lane l reads record l & 15 of wavefront l >> 4 together with the
    // wavefronts' totals (one LDS round trip; lanes past a wavefront's count
    // hold stale words and take no part).  The open segment entering each
    // wavefront is composed from the totals and put in front of that
    // wavefront's first record where its segment opened earlier; the chain
    // then takes the records lane by lane in order, and the segment after
    // the last crossing last.  Per record s = s + u C(parity) when its
    // segment holds a nonzero term, then the crossing add; the binade checks
    // ride beside the chain.
    const int4 W0 = *reinterpret_cast<const int4*>(sh.wc0), W1 = *reinterpret_cast<const int4*>(sh.wc1);
    const int4 WF = *reinterpret_cast<const int4*>(sh.wfl), WN = *reinterpret_cast<const int4*>(sh.wcnt);
    int4 R = sh.rec[lane >> 4][lane & (kSsWaveRec - 1)];
    const int n0 = WN.x & 0xFFFF, n1 = WN.y & 0xFFFF, n2 = WN.z & 0xFFFF, n3 = WN.w & 0xFFFF;
    const int most = max(max(n0, n1), max(n2, n3));
    int ok = n0 + n1 + n2 + n3 < kSsMaxCross && most <= kSsWaveRec && ((WN.x | WN.y | WN.z | WN.w) >> 30) == 0;
    // the open segment entering wavefront q (P1..P3) and after the last (P4)
    const SsSeg P1 = ss_seg(SsSeg{0, 0, 0, 0}, SsSeg{W0.x, W1.x, WF.x, 0});
    const SsSeg P2 = ss_seg(P1, SsSeg{W0.y, W1.y, WF.y, 0});
    const SsSeg P3 = ss_seg(P2, SsSeg{W0.z, W1.z, WF.z, 0});
    const SsSeg P4 = ss_seg(P3, SsSeg{W0.w, W1.w, WF.w, 0});
    int sb = __builtin_bit_cast(int, sh.head);
    if (ok) {
        const int wr = lane >> 4, k = lane & (kSsWaveRec - 1);
        const bool valid = k < (wr == 0 ? n0 : wr == 1 ? n1 : wr == 2 ? n2 : n3);
        if (valid && (R.z & kSsRecBack)) {
            const int pc0 = wr == 1 ? P1.c0 : wr == 2 ? P2.c0 : wr == 3 ? P3.c0 : 0;
            const int pc1 = wr == 1 ? P1.c1 : wr == 2 ? P2.c1 : wr == 3 ? P3.c1 : 0;
            const int pf = wr == 1 ? P1.f : wr == 2 ? P2.f : wr == 3 ? P3.f : 0;
            const SsMap m = ss_compose(SsMap{pc0, pc1, (pf & 1) != 0}, SsMap{R.x, R.y, (R.z & kSsRecNz) != 0});
            R = make_int4(m.c0, m.c1, (R.z & 0xFF) | (m.nz ? kSsRecNz : 0), R.w);
        }
        // within binade E consecutive grid values have consecutive bit
        // patterns (E = 1 spans the subnormals too), so s + u C is bits + C
        // and the parity of s / u is the last bit: C = C0, or C0 + (C1 - C0)
        // when the bits are odd.  The chain reads the records with readlane,
        // in vector registers (the empty asm marks the state lane-varying, so
        // it does not bounce through scalar registers).
        const int dc = R.y - R.x;
        asm volatile("" : "+v"(sb));
        int sbl = 0, nbl = 0;  // the chain's value entering / leaving this lane's record (for the checks)
        uint64_t mask = __builtin_amdgcn_ballot_w64(valid);
        while (mask) {
            const int src = __builtin_ctzll(mask);
            mask &= mask - 1;
            const int C0 = __builtin_amdgcn_readlane(R.x, src), DC = __builtin_amdgcn_readlane(dc, src);
            const float tr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(R.w, src));
            const int nb = sb + C0 + (-(sb & 1) & DC);
            sbl = lane == src ? sb : sbl;
            nbl = lane == src ? nb : nbl;
            sb = __builtin_bit_cast(int, __builtin_bit_cast(float, nb) + tr);
        }
        // the segment after the last crossing
        const int nt = sb + P4.c0 + (-(sb & 1) & (P4.c1 - P4.c0));
        const bool tail_ok = !(P4.f & 1) || (sh.tail_e < 255 && ss_binade(__builtin_bit_cast(float, sb)) == sh.tail_e &&
                                             ss_binade(__builtin_bit_cast(float, nt)) == sh.tail_e);
        sb = nt;
        // every record's segment must start and end inside its binade
        int okl = !valid || !(R.z & kSsRecNz) ||
                  ((R.z & 0xFF) < 255 && ss_binade(__builtin_bit_cast(float, sbl)) == (R.z & 0xFF) &&
                   ss_binade(__builtin_bit_cast(float, nbl)) == (R.z & 0xFF));
        ok = tail_ok && __builtin_amdgcn_ballot_w64(!okl) == 0;
    }
    float res = __builtin_bit_cast(float, sb);
    if (BCAST) {
        // for threads past the computing ones (they take the barriers too)
        if (tid == 0) {
            sh.result = res;
            sh.ok = ok;
        }
        bar();
    }
    if (!ok) {
        // fallback (the same on every computing wavefront): the plain loop
        // on one wavefront
        if (tid < kWave) {
            const float s = seq_sum(t, n);
            if (tid == 0) sh.result = s;
        }
        bar();
        res = sh.result;
    }
    if (fast && tid == 0) *fast = ok != 0;
    if (FINAL) bar();  // sh reusable after return
    return res;
}

// Threads 0..255 only (BCAST: see block_seq_sum_after).
template <int C, bool BCAST = false, class Bar>
__device__ __forceinline__ float block_seq_sum_core(const float* t, int n, SsShared& sh, bool* fast, Bar& bar)
{
    const int tid = threadIdx.x;
    const int c = C ? C : n / kSsThreads;
    const int i0 = tid * c;
    float v[kSsMaxPer];
    if (c % 4 == 0) {
#pragma unroll
        for (int k = 0; k < kSsMaxPer; k += 4) {
            if (k < c) {
                const float4 q = *reinterpret_cast<const float4*>(t + i0 + k);
                v[k] = q.x;
                v[k + 1] = q.y;
                v[k + 2] = q.z;
                v[k + 3] = q.w;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < kSsMaxPer; k++)
            if (k < c) v[k] = t[i0 + k];
    }
    const float I = ss_prefix<C>(v, c, sh);
    bar();
    return block_seq_sum_after<C, true, BCAST>(v, I, t, n, sh, fast, bar);
}


// Every thread of a workgroup of 256 or more threads calls it; threads past
// the first 256 only keep the barrier count of the computing ones.
template <int C>
__device__ __forceinline__ float block_seq_sum_impl(const float* t, int n, SsShared& sh, bool* fast)
{
    if (threadIdx.x >= kSsThreads) {
        // the three phase barriers, the fallback's barrier when it is
        // taken, and the final one
        lds_barrier();
        lds_barrier();
        lds_barrier();
        if (!sh.ok) lds_barrier();
        const float res = sh.result;
        lds_barrier();
        return res;
    }
    SsLdsBarrier bar;
    return block_seq_sum_core<C, true>(t, n, sh, fast, bar);
}

// The sum of 2048 terms where thread j < 256 holds terms [8 j, 8 j + 8) in
// registers (t8) as well as in LDS (t), called by every thread of a
// workgroup of 256 or more threads after the terms are stored: the sum's
// first phase runs from the registers before the barrier that publishes
// them (this call's first), and no barrier follows the result (sh must not
// be written again; t may be, by any thread, once the call returns).
__device__ __forceinline__ float block_seq_sum_regs8(const float (&t8)[8], const float* t, SsShared& sh)
{
    float v[kSsMaxPer];
    float I = 0.0f;
    if (threadIdx.x < kSsThreads) {
#pragma unroll
        for (int k = 0; k < kSsMaxPer; k++) v[k] = k < 8 ? t8[k] : 0.0f;
        I = ss_prefix<8>(v, 8, sh);
    }
    lds_barrier();
    if (threadIdx.x >= kSsThreads) {
        // the phase barriers of the computing threads, and the fallback's
        lds_barrier();
        lds_barrier();
        if (!sh.ok) lds_barrier();
        return sh.result;
    }
    SsLdsBarrier bar;
    return block_seq_sum_after<8, false, true>(v, I, t, 8 * kSsThreads, sh, nullptr, bar);
}

// Dispatch on the terms per thread (compile-time chunk lengths for the
// model widths: 2048 -> 8, 2304 -> 9).
__device__ __forceinline__ float block_seq_sum_nonneg(const float* t, int n, SsShared& sh, bool* fast = nullptr)
{
    if (n == 8 * kSsThreads) return block_seq_sum_impl<8>(t, n, sh, fast);
    if (n == 9 * kSsThreads) return block_seq_sum_impl<9>(t, n, sh, fast);
    return block_seq_sum_impl<0>(t, n, sh, fast);
}

// The same on threads 0..255 with a barrier object of the caller's (an
// SsWaveBarrier already used for other sums keeps its count).
template <class Bar>
__device__ __forceinline__ float block_seq_sum_nonneg_bar(const float* t, int n, SsShared& sh, Bar& bar)
{
    if (n == 8 * kSsThreads) return block_seq_sum_core<8>(t, n, sh, nullptr, bar);
    if (n == 9 * kSsThreads) return block_seq_sum_core<9>(t, n, sh, nullptr, bar);
    return block_seq_sum_core<0>(t, n, sh, nullptr, bar);
}

// The same computed by threads 0..255 alone (only they call it), which
// synchronize through the LDS counter *cnt (zeroed before each call, then a
// workgroup barrier): the workgroup's other wavefronts run work of their
// own meanwhile.  Returns the sum on threads 0..255.
__device__ __forceinline__ float block_seq_sum_nonneg_waves(const float* t, int n, SsShared& sh, int* cnt)
{
    SsWaveBarrier<kSsThreads / kWave> bar{cnt, 0};
    return block_seq_sum_nonneg_bar(t, n, sh, bar);
}

// ---------------------------------------------------------------------------
// The left-to-right fp32 sum of signed values on the fp16 grid (layer_norm's
// mean, gten/ops.cpp:673-676, over an fp16 or Q8 activation row), computed
// by a whole workgroup with the sequential loop's result, bit for bit.
//
// Why it can be parallel: every value is a multiple of 2^-24 below 2^17 in
// magnitude (an fp16 value, or a Q8 code times an fp16 delta), so every
// prefix sum P_i = x_0 + ... + x_{i-1} is exact in fp64 (at most 51
// significant bits), in any order.  The sequential fp32 sum is s_i = P_i +
// e_i, where e_i is the rounding error so far; it changes only at the steps
// whose exact result s_i + x_i is not an fp32 value.  From a step r with
// known e, every step up to the first i >= r at which P_{i+1} + e is not an
// fp32 value is exact, and that step is one fp32 add:
// s_{i+1} = fl(s_i + x_i), e = s_{i+1} - P_{i+1} (exact in fp64).  Sums of
// 2048 fp16 activations round at 3-10 steps (measured on normal and
// heavy-tailed rows), so a few parallel passes over the row replace the
// 2048-step chain.  Values off the grid, or more passes than kSgMaxPass,
// fall back to the plain loop; the result is exact either way.
constexpr int kSgMaxPass = 48;
constexpr int kSgMaxWaves = 16;

struct SgShared {
    double tot[kSgMaxWaves];            // wavefront totals
    double err[2][kSgMaxWaves];         // per pass and wavefront: the error after its first rounding step
    int idx[2][kSgMaxWaves];            // ... and that step (n: none)
    int bad;
    float result;
};

// Lane moves of a double (its halves moved alike).
template <int CTRL, int ROW_MASK = 0xf, bool BZ = true>
__device__ __forceinline__ double dpp_d(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)dpp_i<CTRL, ROW_MASK, BZ>((int)(uint32_t)u);
    const uint32_t hi = (uint32_t)dpp_i<CTRL, ROW_MASK, BZ>((int)(uint32_t)(u >> 32));
    return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}

// Inclusive wave scan of exact doubles (any order is exact here).
__device__ __forceinline__ double wave_scan_add_d(double v)
{
    v = v + dpp_d<0x111>(v);
    v = v + dpp_d<0x112>(v);
    v = v + dpp_d<0x114>(v);
    v = v + dpp_d<0x118>(v);
    v = v + dpp_d<kDppBcast15, 0xa, false>(v);
    v = v + dpp_d<kDppBcast31, 0xc, false>(v);
    return v;
}

// A value the parallel path takes: finite, |x| < 2^17, a multiple of 2^-24.
NC_HD bool sg_on_grid(float x)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, x) & 0x7FFFFFFFu;
    if (u == 0) return true;
    const int e = (int)(u >> 23);
    if (e == 0 || e >= 127 + 17) return false;  // subnormal (below 2^-126), too large, inf, NaN
    // the lowest set bit of the significand, as a power of two
    const uint32_t m = (u & 0x7FFFFFu) | 0x800000u;
    return e - 150 + __builtin_ctz(m) >= -24;
}

// Sum of x[0..n) in index order, n = C * NT, called by threads 0 .. NT-1
// (NT a multiple of 64, at most 1024), which synchronize through bar; thread
// t owns x[t C .. t C + C).  Every calling thread returns the sum; *passes
// (thread 0's view) gets the passes made (0: the plain loop ran).
template <int C, int NT, class Bar>
__device__ __forceinline__ float block_seq_sum_grid(const float* x, SgShared& sh, int* passes, Bar& bar)
{
    static_assert(NT % kWave == 0 && NT / kWave <= kSgMaxWaves, "workgroup");
    constexpr int NW = NT / kWave;
    const int n = C * NT;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    float v[C];
    double p[C];  // P at the end of each of this thread's steps
    bool ok = true;
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < C; k++) {
        v[k] = x[tid * C + k];
        ok = ok && sg_on_grid(v[k]);
        acc = acc + (double)v[k];
        p[k] = acc;
    }
    const double incl = wave_scan_add_d(acc);
    if (lane == kWave - 1) sh.tot[w] = incl;
    if (tid == 0) sh.bad = 0;
    bar();
    if (__builtin_amdgcn_ballot_w64(!ok) && lane == 0) sh.bad = 1;
    double base = incl - acc;  // this thread's first P: the earlier waves' totals, then the lanes'
#pragma unroll
    for (int q = 0; q < NW - 1; q++)
        if (q < w) base = base + sh.tot[q];
    const double pn = [&] {
        double t = 0.0;
#pragma unroll
        for (int q = 0; q < NW; q++) t = t + sh.tot[q];
        return t;
    }();
#pragma unroll
    for (int k = 0; k < C; k++) p[k] = p[k] + base;
    bar();
    int np = 0;
    float res = 0.0f;
    bool done = false;
    double e = 0.0;
    int r = 0;
    // values off the grid go straight to the plain loop
    while (!done && sh.bad == 0 && np < kSgMaxPass) {
        // this thread's first step i >= r whose exact result is not an fp32 value
        int f = n;
        double en = 0.0;
#pragma unroll
        for (int k = C - 1; k >= 0; k--) {
            const int i = tid * C + k;
            const double val = p[k] + e;
            if (i >= r && (double)(float)val != val) {
                f = i;
                const float si = (float)((k ? p[k - 1] : base) + e);  // s_i, an fp32 value
                const float sn = si + v[k];
                en = (double)sn - p[k];
            }
        }
        // the wavefront's first such step: its lowest lane's (chunks are in
        // lane order)
        const uint64_t m = __builtin_amdgcn_ballot_w64(f < n);
        const int slot = np & 1;
        int wf = n;
        double we = 0.0;
        if (m) {
            const int fl = __builtin_ctzll(m);
            wf = __builtin_amdgcn_readlane(f, fl);
            const uint64_t eb = __builtin_bit_cast(uint64_t, en);
            const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)eb, fl);
            const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(eb >> 32), fl);
            we = __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
        }
        if (lane == 0) {
            sh.idx[slot][w] = wf;
            sh.err[slot][w] = we;
        }
        bar();
        np++;
        int fi = n;
        double ei = 0.0;
#pragma unroll
        for (int q = NW - 1; q >= 0; q--)
            if (sh.idx[slot][q] < n) {
                fi = sh.idx[slot][q];
                ei = sh.err[slot][q];
            }
        if (fi == n) {
            res = (float)(pn + e);
            done = true;
        } else {
            e = ei;
            r = fi + 1;
        }
    }
    if (!done) {
        // off the grid or too many rounding steps: the plain loop
        if (tid < kWave) {
            float s = 0.0f;
            for (int i = 0; i < n; i++) s = s + x[i];
            if (tid == 0) sh.result = s;
        }
        bar();
        res = sh.result;
        np = 0;
    }
    if (passes && tid == 0) *passes = np;
    bar();  // sh reusable after return
    return res;
}

// The same with the workgroup's LDS barrier (all NT threads of the
// workgroup call it).
template <int C, int NT>
__device__ __forceinline__ float block_seq_sum_grid(const float* x, SgShared& sh, int* passes = nullptr)
{
    SsLdsBarrier bar;
    return block_seq_sum_grid<C, NT>(x, sh, passes, bar);
}

#endif  // __HIPCC__

}  // namespace nc
