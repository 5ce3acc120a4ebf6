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

// One step s -> RN(s + t) with s and the result in binade E: the units
// added from parity 0 and from parity 1.  t / u is exact (a power-of-two
// scale of a value below 2^(E+1), so below 2^24 units); a tie rounds to the
// even result.
NC_HD SsMap ss_step(float t, int E)
{
    const float q = __builtin_ldexpf(t, 150 - E);
    const float fl = __builtin_floorf(q);
    const float fr = q - fl;
    const int f = (int)fl;
    const int up = fr > 0.5f ? 1 : 0;
    const bool tie = fr == 0.5f;
    SsMap m;
    m.c0 = f + up + ((tie && (f & 1)) ? 1 : 0);   // parity 0: s/u + f odd when f odd
    m.c1 = f + up + ((tie && !(f & 1)) ? 1 : 0);  // parity 1: odd when f even
    m.nz = t != 0.0f;
    return m;
}

// Applies a segment map computed for binade E to the exact value s.
// Returns false when s does not lie in E or the result leaves it.
NC_HD bool ss_apply(float& s, const SsMap& m, int E)
{
    if (!m.nz) return true;
    if (E >= 255 || ss_binade(s) != E) return false;  // infinities and NaNs take the plain loop
    const int units = (int)__builtin_ldexpf(s, 150 - E);  // exact: s is on the grid, < 2^24 units
    const int after = units + ((units & 1) ? m.c1 : m.c0);
    if (after >= (1 << 24)) return false;
    s = __builtin_ldexpf((float)after, E - 150);
    return true;
}

#if defined(__HIPCC__)

constexpr int kSsThreads = 256;   // workgroup size the block sum is written for
constexpr int kSsMaxPer = 16;     // terms per thread: n <= 4096
constexpr int kSsMaxCross = 63;   // crossings handled before the fallback (one per lane of a wave)

struct SsShared {
    float wf[kSsThreads / kWave];
    int wc0[kSsThreads / kWave], wc1[kSsThreads / kWave], wfl[kSsThreads / kWave], wcnt[kSsThreads / kWave];
    int rc0[kSsMaxCross + 1], rc1[kSsMaxCross + 1], rE[kSsMaxCross + 1];
    float rt[kSsMaxCross + 1];
    int m;
    int ok;
    float result;
};

// Segmented scan element: a parity map and flags (bit 0: nz, bit 1: the
// element holds a crossing, i.e. its map restarts the open segment).
struct SsSeg {
    int c0, c1, f;
};

// (a then b): b alone when b restarts, else the composition.
__device__ __forceinline__ SsSeg ss_seg(const SsSeg& a, const SsSeg& b)
{
    if (b.f & 2) return b;
    const SsMap m = ss_compose(SsMap{a.c0, a.c1, (a.f & 1) != 0}, SsMap{b.c0, b.c1, (b.f & 1) != 0});
    return SsSeg{m.c0, m.c1, (m.nz ? 1 : 0) | (a.f & 2)};
}

template <int CTRL, int ROW_MASK = 0xf, bool BZ = true>
__device__ __forceinline__ SsSeg ss_dpp(const SsSeg& x)
{
    // lanes without a source get 0s: the identity element
    return SsSeg{dpp_i<CTRL, ROW_MASK, BZ>(x.c0), dpp_i<CTRL, ROW_MASK, BZ>(x.c1), dpp_i<CTRL, ROW_MASK, BZ>(x.f)};
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
__device__ __forceinline__ int wave_scan_add_i(int v)
{
    v = v + dpp_i<0x111>(v);
    v = v + dpp_i<0x112>(v);
    v = v + dpp_i<0x114>(v);
    v = v + dpp_i<0x118>(v);
    v = v + dpp_i<kDppBcast15, 0xa, false>(v);
    v = v + dpp_i<kDppBcast31, 0xc, false>(v);
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
// for t >= 0 in LDS; n a multiple of 256, n <= 4096.  Called by all 256
// threads of the workgroup; every thread returns the sum.  *fast (thread
// 0's view) tells whether the parallel path was taken.  Synchronizes the
// workgroup through LDS barriers only (global loads may stay in flight).
__device__ float block_seq_sum_nonneg(const float* t, int n, SsShared& sh, bool* fast = nullptr)
{
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const int c = n / kSsThreads;
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
    float I = wave_scan_add(cs);
    if (lane == kWave - 1) sh.wf[w] = I;
    lds_barrier();
    float WP = 0.0f;
    for (int q = 0; q < w; q++) WP = WP + sh.wf[q];
    I = I + WP;
    float A = dpp_f<kDppWaveShr1>(I);  // the previous lane's I
    if (lane == 0) A = WP;
    // ---- walk 1: crossings of this chunk and the map after the last one
    int ncross = 0;
    SsMap tail = ss_identity();
    {
        float P = A;
        int Eb = ss_binade(A);
#pragma unroll
        for (int k = 0; k < kSsMaxPer; k++) {
            if (k < c) {
                const float Pa = k + 1 < c ? P + v[k] : I;
                const int Ea = ss_binade(Pa);
                if (Ea == Eb) {
                    tail = ss_compose(tail, ss_step(v[k], Eb));
                } else {
                    ncross++;
                    tail = ss_identity();
                }
                P = Pa;
                Eb = Ea;
            }
        }
    }
    // ---- segmented scan of (tail, has-crossing) and scan of the counts
    SsSeg x{tail.c0, tail.c1, (tail.nz ? 1 : 0) | (ncross > 0 ? 2 : 0)};
    x = wave_scan_seg(x);
    int cnt = wave_scan_add_i(ncross);
    if (lane == kWave - 1) {
        sh.wc0[w] = x.c0;
        sh.wc1[w] = x.c1;
        sh.wfl[w] = x.f;
        sh.wcnt[w] = cnt;
    }
    lds_barrier();
    SsSeg pre{0, 0, 0};
    int pre_cnt = 0;
    for (int q = 0; q < w; q++) {
        pre = ss_seg(pre, SsSeg{sh.wc0[q], sh.wc1[q], sh.wfl[q]});
        pre_cnt += sh.wcnt[q];
    }
    x = ss_seg(pre, x);
    cnt += pre_cnt;
    // exclusive values: the open segment entering this chunk, crossings before it
    SsSeg in = ss_dpp<kDppWaveShr1>(x);
    int base = dpp_i<kDppWaveShr1>(cnt);
    if (lane == 0) {
        in = pre;
        base = pre_cnt;
    }
    // the final segment (after the last crossing) and the crossing count
    if (tid == kSsThreads - 1) {
        sh.m = cnt;
        if (cnt <= kSsMaxCross) {
            sh.rc0[cnt] = x.c0;
            sh.rc1[cnt] = x.c1;
            sh.rE[cnt] = (x.f & 1) ? ss_binade(I) : 0;
        }
    }
    // ---- walk 2: records of the crossings, in index order
    if (ncross > 0 && base + ncross <= kSsMaxCross) {
        SsMap cur{in.c0, in.c1, (in.f & 1) != 0};
        float P = A;
        int Eb = ss_binade(A);
        int r = base;
#pragma unroll
        for (int k = 0; k < kSsMaxPer; k++) {
            if (k < c) {
                const float Pa = k + 1 < c ? P + v[k] : I;
                const int Ea = ss_binade(Pa);
                if (Ea == Eb) {
                    cur = ss_compose(cur, ss_step(v[k], Eb));
                } else {
                    sh.rc0[r] = cur.c0;
                    sh.rc1[r] = cur.c1;
                    sh.rE[r] = cur.nz ? Eb : 0;
                    sh.rt[r] = v[k];
                    r++;
                    cur = ss_identity();
                }
                P = Pa;
                Eb = Ea;
            }
        }
    }
    lds_barrier();
    // ---- replay on wave 0: record r in lane r, segment maps and crossing
    // adds applied in order (a uniform loop over readlanes)
    if (w == 0) {
        const int mm = sh.m;
        bool ok = mm <= kSsMaxCross;
        if (ok) {
            const int rl = lane <= mm ? lane : 0;
            const int lc0 = sh.rc0[rl], lc1 = sh.rc1[rl], lE = sh.rE[rl];
            const float lt = sh.rt[rl];
            float s = 0.0f;
            for (int r = 0; r <= mm; r++) {
                const int E = __builtin_amdgcn_readlane(lE, r);
                const SsMap sm{__builtin_amdgcn_readlane(lc0, r), __builtin_amdgcn_readlane(lc1, r), E != 0};
                ok = ss_apply(s, sm, E) && ok;
                if (r < mm) s = s + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lt), r));
            }
            if (lane == 0) sh.result = s;
        }
        if (lane == 0) sh.ok = ok;
    }
    lds_barrier();
    if (!sh.ok) {
        // fallback: the plain loop on one wavefront
        if (tid < kWave) {
            const float s = seq_sum(t, n);
            if (tid == 0) sh.result = s;
        }
        lds_barrier();
    }
    if (fast && tid == 0) *fast = sh.ok != 0;
    const float res = sh.result;
    lds_barrier();  // sh reusable after return
    return res;
}

#endif  // __HIPCC__

}  // namespace nc
