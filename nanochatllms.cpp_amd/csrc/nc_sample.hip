// nc_sample.hip -- top-k / temperature sampling of a logits row on the
// device, with the reference's results (gten/sampler.cpp:63-143) and its
// random source made reproducible: std::mt19937 seeded with a given value
// instead of std::random_device (sampler.cpp:70-71).
//
// One sampling step of the reference, as libstdc++ runs its calls:
//   1. pairs (logit / temp in double, index); std::partial_sort of the first
//      k = min(top_k, 1000) by value, descending -- a heap select;
//   2. e_j = std::exp(v_j) (glibc's double exp) and sum_exp = e_0 + e_1 + ...
//      in that descending order; p_j = e_j / sum_exp;
//   3. std::discrete_distribution over the n-entry weight vector (p_j at
//      index i_j, zeros elsewhere): s = 0.0 + w_0 + ... + w_{n-1} in index
//      order, q_i = w_i / s, cumulative c_i = q_0 + ... + q_i with c_{n-1}
//      set to 1;
//   4. u = generate_canonical<double, 53>: two mt19937 outputs,
//      (u1 + u2 * 2^32) rounded to double, times 2^-64 (a result of 1 becomes
//      the double below 1); the token is lower_bound(c, u).
//
// On the device, workgroups of 1024 threads:
//   * candidates: a systematic sample of 1024 logits sets a threshold (each
//     wavefront sorts its 64 in registers and offers the quantile that would
//     keep about 1.5 k + 256 logits; the median offer is taken; every
//     workgroup computes the same one), and every logit at or above it is
//     gathered (up to 4096): each workgroup gathers a slice of at least 4096
//     logits, and the last one to finish takes the candidates into LDS and
//     runs the rest of the step alone.  For k < 64 an
//     8-bit radix select finds the (k+1)-th largest candidate and the k above
//     it are sorted in one wavefront's registers; larger k bitonic-sort the
//     candidates.  The top k are the heap select's k when the k-th value is
//     not tied with the next; the ordering of the logits equals that of
//     logit / temp (distinct floats stay distinct doubles), with -0 == +0.
//   * exact fallback: when the k-th value is tied with the (k+1)-th (the heap
//     order then decides which tied indices stay), a logit is NaN, or the
//     threshold gathers fewer than k or more than 4096, thread 0 replays the
//     heap select (make_heap, pop_heap, the sift order of libstdc++) over
//     every logit, staged through LDS; rare and slower (~1 ms).
//   * the three sums are the reference's sequential chains, run by thread 0
//     over LDS; exp, the divisions and the sorts are parallel.  Weights are
//     nonzero only at the k indices, so the n-term sums and the cumulative
//     table reduce to the k entries in index order (adding +0.0 changes
//     nothing); lower_bound runs libstdc++'s binary search over the implied
//     n-entry table.  A NaN weight (from NaN logits, or an exp overflow
//     giving inf / inf) makes the sum NaN and every entry NaN: the table is
//     then NaN up to the final 1.  Where the implied table is non-decreasing
//     (no NaN weight, the entry before the final 1 at most 1) lower_bound is
//     the first entry >= u, found by one wavefront's ballot over the k kept
//     entries; otherwise thread 0 runs libstdc++'s binary search.
#include <hip/hip_runtime.h>

#include "nc_device.h"
#include "nc_exp64.h"
#include "nc_kernels.h"

namespace nc {

constexpr int kSmThreads = 1024;
constexpr int kSmCap = 4096;      // candidates sorted in LDS
constexpr int kSmSample = 1024;   // threshold sample size
constexpr int kSmStage = 8192;    // logits per LDS stage of the fallback

// ---- std::mt19937 (state: 624 words, then the index of the next word) ----

void mt_seed_host(uint32_t seed, uint32_t* st)
{
    st[0] = seed;
    for (uint32_t i = 1; i < 624; i++) st[i] = 1812433253u * (st[i - 1] ^ (st[i - 1] >> 30)) + i;
    st[624] = 624;
}

__device__ uint32_t mt_next(uint32_t* mt)
{
    if (mt[624] >= 624) {
        for (int i = 0; i < 624; i++) {
            const uint32_t y = (mt[i] & 0x80000000u) | (mt[i + 1 < 624 ? i + 1 : 0] & 0x7fffffffu);
            mt[i] = mt[i + 397 < 624 ? i + 397 : i - 227] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        mt[624] = 0;
    }
    uint32_t z = mt[mt[624]++];
    z ^= z >> 11;
    z ^= (z << 7) & 0x9d2c5680u;
    z ^= (z << 15) & 0xefc60000u;
    z ^= z >> 18;
    return z;
}

// ---- ordering keys -------------------------------------------------------

// Unsigned key with the float order; -0 and +0 share a key.  Finite and
// infinite values map above 0x007fffff, so 0 pads below all of them.
__device__ __forceinline__ uint32_t fkey(float x)
{
    uint32_t b = __float_as_uint(x);
    if (b == 0x80000000u) b = 0;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float fkey_value(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? k ^ 0x80000000u : ~k); }

// Bitonic sort of P (a power of two) entries in LDS, descending or ascending.
template <bool DESC, typename T>
__device__ void bitonic(T* a, int P)
{
    for (int size = 2; size <= P; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < P / 2; t += kSmThreads) {
                const int i = 2 * t - (t & (stride - 1)), j = i + stride;
                const bool up = (i & size) == 0;
                const T x = a[i], y = a[j];
                if (DESC ? (up ? x < y : x > y) : (up ? x > y : x < y)) {
                    a[i] = y;
                    a[j] = x;
                }
            }
            lds_barrier();
        }
}

__device__ __forceinline__ int pow2_at_least(int n)
{
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

// ---- libstdc++'s heap over (value, index), ordered by value descending ----
// (std::partial_sort's comparator a.first > b.first: the heap top is the
// smallest kept value).

__device__ void heap_push(float* hv, int* hi, int hole, int top, float v, int ix)
{
    int parent = (hole - 1) / 2;
    while (hole > top && hv[parent] > v) {
        hv[hole] = hv[parent];
        hi[hole] = hi[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    hv[hole] = v;
    hi[hole] = ix;
}

__device__ void heap_adjust(float* hv, int* hi, int hole, int len, float v, int ix)
{
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (hv[child] > hv[child - 1]) child--;
        hv[hole] = hv[child];
        hi[hole] = hi[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        hv[hole] = hv[child - 1];
        hi[hole] = hi[child - 1];
        hole = child - 1;
    }
    heap_push(hv, hi, hole, top, v, ix);
}

struct SampleArgs {
    const float* logits;
    int n;
    int k;          // min(top_k, 1000), 1 <= k <= n
    double temp;    // min(temp, 2.0f), > 0
    uint32_t* rng;  // 625 words, read and written back
    int32_t* tokens;  // the token goes to tokens[pos + 1]
    int* dpos;        // device position, advanced by one (or null: pos)
    int pos;
    double* probs;    // optional: the n normalized weights
    // optional: {k, temp} read on the device instead of the two fields
    // above (a captured step then serves every setting)
    const double* dset;
};

// ---- wavefront sorts in registers (no barriers) ----------------------------

// Bitonic sort of one value per lane: lane i ends with the i-th largest
// (DESC) or the i-th smallest.
template <bool DESC, typename T>
__device__ __forceinline__ T wave_sort(T v)
{
    static_assert(sizeof(T) == 4, "32-bit values");
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const T o = (T)__shfl_xor((int)v, stride);
            const bool lower = (lane & stride) == 0;
            const bool first = (lane & size) == 0;  // this block's order is the final one
            const bool keep_big = (lower == first) == DESC;
            v = keep_big ? (o > v ? o : v) : (o < v ? o : v);
        }
    }
    return v;
}

// Settings handled by one wavefront after the gather: the k kept entries
// and the next one fit its 64 lanes.
constexpr int kSmFastK = kWave - 1;

// The gather runs on up to kSmMaxWg workgroups, at least kSmSlice logits
// each (one pass of kSmGu loads per thread).  They append their candidates
// to g_cand (device memory of the library, one copy per GPU), and the last
// one to finish takes them over and runs the rest of the step, then clears
// the counters for the next launch.  Launches that overlap on one GPU race
// on this state.
constexpr int kSmMaxWg = 64;
constexpr int kSmSlice = 4096;
constexpr int kSmGu = 32;
constexpr int kSmMaxN = kSmMaxWg * kSmGu * kSmThreads;
static __device__ uint64_t g_cand[kSmCap];
static __device__ unsigned g_cnt, g_done, g_nan;

static int sample_grid(int n)
{
    const int g = (n + kSmSlice - 1) / kSmSlice;
    return g < 1 ? 1 : (g > kSmMaxWg ? kSmMaxWg : g);
}

__global__ __launch_bounds__(kSmThreads) void k_sample_topk(SampleArgs A)
{
    // cand: candidate (key << 32 | index); later the fallback's logit stage,
    // then the index-ordered weights and cumulative table
    __shared__ union {
        uint64_t cand[kSmCap];
        float stage[kSmStage];
        struct {
            double c[1024];
            int idx[1024];
        } t;
    } U;
    __shared__ union {
        struct {
            float hv[1024];
            int hi[1024];
        } h;
        uint64_t byidx[1024];  // (index << 32 | rank in descending order)
    } V;
    __shared__ double ev[1024];  // e_j, then p_j, in descending order
    __shared__ uint32_t mt[625];
    __shared__ uint32_t s_wq[kSmThreads / kWave];
    __shared__ int hist[4][256];  // radix-select counts, one array per pass
    __shared__ uint64_t top[kSmFastK + 1];
    __shared__ int s_nan, s_last, s_top, s_need;
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_thr;
    __shared__ double s_sum;

    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const int n = A.n;
    const int k = A.dset ? (int)A.dset[0] : A.k;
    const double temp = A.dset ? A.dset[1] : A.temp;
    const int pos = A.dpos ? load_pos(A.dpos) : A.pos;
    // this workgroup's slice of the logits (a multiple of 1024, at most
    // kSmGu per thread)
    const int G = gridDim.x;
    const int slice = ((n + G - 1) / G + kSmThreads - 1) / kSmThreads * kSmThreads;
    const int lo = (int)blockIdx.x * slice, hi = min(n, lo + slice);
    // the threshold sample and the slice requested together
    const bool sampled = n > kSmCap;
    const float sx = sampled ? A.logits[(long long)tid * n / kSmSample] : 0.0f;
    float x[kSmGu];
#pragma unroll
    for (int u = 0; u < kSmGu; u++) {
        const int i = lo + u * kSmThreads + tid;
        x[u] = i < hi ? A.logits[i] : -INFINITY;
    }
    for (int i = tid; i < 625; i += kSmThreads) mt[i] = A.rng[i];
    for (int i = tid; i < 4 * 256; i += kSmThreads) (&hist[0][0])[i] = 0;
    if (tid == 0) s_top = 0;

    // threshold: about the (1.5 k + 256) n / 1024-th largest logit, from a
    // systematic sample of 1024 (only a candidate bound: any threshold gives
    // the same result, the fallback covers the rest): each wavefront sorts
    // its 64 sampled keys in registers and offers its r/16-th largest; the
    // threshold is the median of the 16 offers (every workgroup finds the
    // same one)
    uint32_t thr = 0;
    if (sampled) {
        const long long r = ((long long)(3 * k / 2 + 256) * kSmSample) / n;
        const int rw = (int)(r / (kSmThreads / kWave)) < kWave - 1 ? (int)(r / (kSmThreads / kWave)) : kWave - 1;
        if (rw == 0) {
            // the wavefront's largest (the large vocabularies)
            uint32_t v = fkey(sx);
#pragma unroll
            for (int o = kWave / 2; o > 0; o >>= 1) {
                const uint32_t y = (uint32_t)__shfl_xor((int)v, o);
                v = y > v ? y : v;
            }
            if (lane == 0) s_wq[w] = v;
        } else {
            const uint32_t v = wave_sort<true>(fkey(sx));
            if (lane == rw) s_wq[w] = v;
        }
        lds_barrier();
        // the 8th largest of the 16 offers (ties: any of the equal ones), by
        // wavefront 0's first 16 lanes
        if (w == 0 && lane < kSmThreads / kWave) {
            const uint32_t mine = s_wq[lane];
            int gt = 0, eq = 0;
#pragma unroll
            for (int j = 0; j < kSmThreads / kWave; j++) {
                const uint32_t o = s_wq[j];
                gt += o > mine;
                eq += o == mine;
            }
            if (gt <= 7 && gt + eq > 7) s_thr = mine;
        }
        lds_barrier();
        thr = s_thr;
    }

    // gather this slice's logits with key >= thr: one compare per logit
    // (!(x < t) also holds for NaN, told apart below; thr = 0, no sample,
    // takes every logit), one slot reservation per wavefront
    {
        const float thr_x = thr ? fkey_value(thr) : -INFINITY;
        unsigned long long hm[kSmGu];
        int tot = 0;
#pragma unroll
        for (int u = 0; u < kSmGu; u++) {
            const int i = lo + u * kSmThreads + tid;
            hm[u] = __ballot(i < hi && !(x[u] < thr_x));
            tot += __popcll(hm[u]);
        }
        if (tot) {  // uniform
            int wbase = 0;
            if (lane == 0)
                wbase = (int)__hip_atomic_fetch_add(&g_cnt, (unsigned)tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wbase = __shfl(wbase, 0);
#pragma unroll
            for (int u = 0; u < kSmGu; u++) {
                const unsigned long long m = hm[u];
                if (m == 0) continue;  // uniform
                const int i = lo + u * kSmThreads + tid;
                const int at = wbase + __popcll(m & ((1ull << lane) - 1ull));
                wbase += __popcll(m);
                if ((m >> lane) & 1ull) {
                    // a NaN passes the compare: flagged (the fallback then
                    // runs) and stored like the others, never read
                    if (x[u] != x[u]) __hip_atomic_store(&g_nan, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (at < kSmCap)
                        __hip_atomic_store(&g_cand[at], ((uint64_t)fkey(x[u]) << 32) | (uint32_t)i,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
    // the last workgroup to finish its gather runs the rest: each counts
    // itself after its stores have completed; the last takes an acquire
    // fence before it reads what the others stored
    wait_stores_done();
    lds_barrier();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(&g_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)G - 1;
    lds_barrier();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // the count and every candidate slot at once (slots past the count are
    // not used)
    int C = (int)__hip_atomic_load(&g_cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint64_t cv[kSmCap / kSmThreads];
#pragma unroll
    for (int j = 0; j < kSmCap / kSmThreads; j++)
        cv[j] = __hip_atomic_load(&g_cand[tid + j * kSmThreads], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) s_nan = (int)__hip_atomic_load(&g_nan, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int j = 0; j < kSmCap / kSmThreads; j++) U.cand[tid + j * kSmThreads] = cv[j];
    if (A.probs)
        for (int i = tid; i < n; i += kSmThreads) A.probs[i] = 0.0;
    lds_barrier();
    if (tid == 0) {
        // every workgroup has counted itself: the counters are free
        __hip_atomic_store(&g_cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&g_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&g_nan, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    bool fallback = s_nan || C < k || C > kSmCap;
    const bool fast = k <= kSmFastK;
    if (!fallback && fast) {
        // the (k+1)-th largest key of the candidates by an 8-bit radix
        // select, then the keys above it: exactly k of them unless the k-th
        // value ties with the (k+1)-th (the heap order then decides)
        if (C > k) {
            uint32_t prefix = 0, mask = 0;
            int need = k + 1;  // rank (from 1) within the keys matching prefix
#pragma unroll
            for (int pass = 0; pass < 4; pass++) {
                const int shift = 24 - 8 * pass;
                for (int j = tid; j < C; j += kSmThreads) {
                    const uint32_t key = (uint32_t)(U.cand[j] >> 32);
                    if ((key & mask) == prefix) atomicAdd(&hist[pass][(key >> shift) & 255], 1);
                }
                lds_barrier();
                if (w == 0) {
                    // bins from the top: lane l holds bins 255 - 4l .. 252 - 4l
                    int c4[4], tot = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        c4[i] = hist[pass][255 - 4 * lane - i];
                        tot += c4[i];
                    }
                    int incl = tot;
#pragma unroll
                    for (int o = 1; o < kWave; o <<= 1) {
                        const int y = __shfl_up(incl, o);
                        if (lane >= o) incl += y;
                    }
                    int before = incl - tot;  // keys in higher bins
                    int bin = -1, above = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if (bin < 0 && before + c4[i] >= need) {
                            bin = 255 - 4 * lane - i;
                            above = before;
                        }
                        before += c4[i];
                    }
                    const unsigned long long fm = __ballot(bin >= 0);
                    const int fl = __ffsll((long long)fm) - 1;  // highest bins first
                    if (lane == fl) {
                        s_prefix = prefix | ((uint32_t)bin << shift);
                        s_need = need - above;
                    }
                }
                lds_barrier();
                prefix = s_prefix;
                need = s_need;
                mask |= 255u << shift;
            }
            // prefix = the (k+1)-th largest key; need > 1: keys equal to it
            // rank above the (k+1)-th, so the k-th equals it
            if (need > 1) fallback = true;
            if (!fallback) {
                for (int j = tid; j < C; j += kSmThreads) {
                    const uint64_t c = U.cand[j];
                    if ((uint32_t)(c >> 32) > prefix) top[atomicAdd(&s_top, 1)] = c;
                }
            }
        } else {
            for (int j = tid; j < C; j += kSmThreads) top[j] = U.cand[j];
        }
        lds_barrier();
        if (!fallback && tid < k) {
            // the k kept entries in descending order: each one's rank among
            // them (entries are distinct: their indices differ)
            const uint64_t e = top[tid];
            int r = 0;
            for (int j = 0; j < k; j++) r += top[j] > e;
            U.cand[r] = e;
        }
    } else if (!fallback) {
        const int P = pow2_at_least(C);
        for (int i = C + tid; i < P; i += kSmThreads) U.cand[i] = 0;
        lds_barrier();
        bitonic<true>(U.cand, P);
        // a tie between the k-th and (k+1)-th value: the heap order decides
        if (C > k && (uint32_t)(U.cand[k - 1] >> 32) == (uint32_t)(U.cand[k] >> 32)) fallback = true;
    }
    lds_barrier();
    if (fallback) {
        // std::partial_sort's heap select, replayed by thread 0
        for (int j = tid; j < k; j += kSmThreads) {
            V.h.hv[j] = A.logits[j];
            V.h.hi[j] = j;
        }
        lds_barrier();
        if (tid == 0 && k >= 2)
            for (int parent = (k - 2) / 2;; parent--) {
                heap_adjust(V.h.hv, V.h.hi, parent, k, V.h.hv[parent], V.h.hi[parent]);
                if (parent == 0) break;
            }
        for (int base = k; base < n; base += kSmStage) {
            const int m = min(kSmStage, n - base);
            lds_barrier();
            for (int j = tid; j < m; j += kSmThreads) U.stage[j] = A.logits[base + j];
            lds_barrier();
            if (tid == 0)
                for (int j = 0; j < m; j++) {
                    const float v = U.stage[j];
                    if (v > V.h.hv[0]) heap_adjust(V.h.hv, V.h.hi, 0, k, v, base + j);
                }
        }
        lds_barrier();
        // the kept k, sorted by value (their order among equal values does
        // not change any sum)
        const int P = pow2_at_least(k);
        for (int j = tid; j < P; j += kSmThreads)
            U.cand[j] = j < k ? ((uint64_t)fkey(V.h.hv[j]) << 32) | (uint32_t)V.h.hi[j] : 0ull;
        lds_barrier();
        bitonic<true>(U.cand, P);
        C = k;
    }

    if (fast) {
        // the rest on wavefront 0, lane j holding the j-th kept entry, the
        // sequential chains on lane 0 over LDS: no workgroup barrier
        if (w != 0) return;
        auto wsync = [] {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        };
        const bool in = lane < k;
        const uint64_t c = in ? U.cand[lane] : 0ull;
        const int idx = (int)(uint32_t)c;
        const float xv = s_nan ? (in ? A.logits[idx] : 0.0f) : fkey_value((uint32_t)(c >> 32));
        // e_j = exp(v_j / temp); sum_exp in descending order
        if (in) ev[lane] = exp_ref((double)xv / temp);
        // each kept index's place in index order (indices are distinct)
        int r = 0;
        if (in)
            for (int j = 0; j < k; j++) r += (int)(uint32_t)U.cand[j] < idx;
        wsync();
        if (lane == 0) {
            double s1 = 0;
            for (int j = 0; j < k; j++) s1 += ev[j];
            s_sum = s1;
        }
        wsync();
        if (in) {
            // weights in index order
            U.t.idx[r] = idx;
            U.t.c[r] = ev[lane] / s_sum;
        }
        wsync();
        if (lane == 0) {
            double s2 = 0.0;
            for (int j = 0; j < k; j++) s2 += U.t.c[j];
            s_sum = s2;
        }
        wsync();
        const double s2 = s_sum;
        const bool nan_sum = s2 != s2;
        if (in) U.t.c[lane] = U.t.c[lane] / s2;
        if (A.probs) {
            if (!nan_sum) {
                if (in) A.probs[U.t.idx[lane]] = U.t.c[lane];
            } else {
                for (int i = lane; i < n; i += kWave) A.probs[i] = s2;
            }
        }
        wsync();
        if (lane == 0) {
            // the cumulative table, c_{k-1} = 1 when the last kept index is
            // n - 1
            double cq = U.t.c[0];
            for (int j = 1; j < k; j++) {
                cq = cq + U.t.c[j];
                U.t.c[j] = cq;
            }
            if (U.t.idx[k - 1] == n - 1) U.t.c[k - 1] = 1.0;
            // generate_canonical<double, 53>
            double sum = 0.0, tmp = 1.0;
            for (int rr = 0; rr < 2; rr++) {
                sum += (double)mt_next(mt) * tmp;
                tmp *= 4294967296.0;
            }
            double u = sum / tmp;
            if (u >= 1.0) u = 0x1.fffffffffffffp-1;
            s_sum = u;
        }
        wsync();
        const double u = s_sum;
        // lower_bound over the n-entry table (0 before the first kept index,
        // c_j from index idx_j on, 1 at n - 1).  Where it is non-decreasing
        // (no NaN weight, the entry before the final 1 at most 1) that is the
        // first entry >= u, found by a ballot; otherwise libstdc++'s binary
        // search runs as it is, on lane 0.
        const bool last_is_end = U.t.idx[k - 1] == n - 1;
        const int lastc = last_is_end ? k - 2 : k - 1;
        const bool mono = !nan_sum && (lastc < 0 || U.t.c[lastc] <= 1.0);
        int tok = n - 1;
        if (mono) {
            const unsigned long long m = __ballot(in && U.t.c[lane] >= u);
            if (u == 0.0) tok = 0;
            else if (m) tok = U.t.idx[__ffsll((long long)m) - 1];
        } else if (lane == 0) {
            int first = 0, len = n;
            while (len > 0) {
                const int half = len >> 1, mid = first + half;
                double cm;
                if (mid == n - 1) {
                    cm = 1.0;
                } else if (nan_sum) {
                    cm = s2;
                } else {
                    int lo2 = 0, hi2 = k;  // number of kept indices <= mid
                    while (lo2 < hi2) {
                        const int h = (lo2 + hi2) >> 1;
                        if (U.t.idx[h] <= mid) lo2 = h + 1;
                        else hi2 = h;
                    }
                    cm = lo2 ? U.t.c[lo2 - 1] : 0.0;
                }
                if (cm < u) {
                    first = mid + 1;
                    len = len - half - 1;
                } else {
                    len = half;
                }
            }
            tok = first;
        }
        if (lane == 0) {
            A.tokens[pos + 1] = tok;
            if (A.dpos) A.dpos[0] = pos + 1;
        }
        wsync();
        for (int i = lane; i < 625; i += kWave) A.rng[i] = mt[i];
        return;
    }

    // e_j = exp(v_j / temp) in descending order; sum_exp in that order
    int my_idx = 0;
    if (tid < k) {
        const uint64_t c = U.cand[tid];
        my_idx = (int)(uint32_t)c;
        const float xv = s_nan ? A.logits[my_idx] : fkey_value((uint32_t)(c >> 32));
        ev[tid] = exp_ref((double)xv / temp);
    }
    lds_barrier();
    if (tid == 0) {
        double s = 0;
        for (int j = 0; j < k; j++) s += ev[j];
        s_sum = s;
    }
    lds_barrier();
    if (tid < k) ev[tid] = ev[tid] / s_sum;
    const int P2 = pow2_at_least(k);
    if (tid < P2) V.byidx[tid] = tid < k ? ((uint64_t)(uint32_t)my_idx << 32) | (uint32_t)tid : ~0ull;
    lds_barrier();
    bitonic<false>(V.byidx, P2);
    // index order: weights p, their sum, q = p / sum, the cumulative table
    if (tid < k) {
        const uint64_t b = V.byidx[tid];
        U.t.idx[tid] = (int)(b >> 32);
        U.t.c[tid] = ev[(uint32_t)b];
    }
    lds_barrier();
    if (tid == 0) {
        double s = 0.0;
        for (int j = 0; j < k; j++) s += U.t.c[j];
        s_sum = s;
    }
    lds_barrier();
    // a NaN weight makes the sum NaN, and then every weight, the zeros
    // included (0 / NaN), and every cumulative entry but the last
    const bool nan_sum = s_sum != s_sum;
    if (tid < k) {
        const double q = U.t.c[tid] / s_sum;
        U.t.c[tid] = q;
        if (A.probs && !nan_sum) A.probs[U.t.idx[tid]] = q;
    }
    if (A.probs && nan_sum)
        for (int i = tid; i < n; i += kSmThreads) A.probs[i] = s_sum;
    lds_barrier();
    if (tid == 0) {
        double c = U.t.c[0];
        for (int j = 1; j < k; j++) {
            c = c + U.t.c[j];
            U.t.c[j] = c;
        }
        if (U.t.idx[k - 1] == n - 1) U.t.c[k - 1] = 1.0;
        // generate_canonical<double, 53>
        double sum = 0.0, tmp = 1.0;
        for (int r = 0; r < 2; r++) {
            sum += (double)mt_next(mt) * tmp;
            tmp *= 4294967296.0;
        }
        double u = sum / tmp;
        if (u >= 1.0) u = 0x1.fffffffffffffp-1;
        // lower_bound over the n-entry cumulative table
        int first = 0, len = n;
        while (len > 0) {
            const int half = len >> 1, mid = first + half;
            double cm;
            if (mid == n - 1) {
                cm = 1.0;
            } else if (nan_sum) {
                cm = s_sum;
            } else {
                int lo2 = 0, hi2 = k;  // number of kept indices <= mid
                while (lo2 < hi2) {
                    const int h = (lo2 + hi2) >> 1;
                    if (U.t.idx[h] <= mid) lo2 = h + 1;
                    else hi2 = h;
                }
                cm = lo2 ? U.t.c[lo2 - 1] : 0.0;
            }
            if (cm < u) {
                first = mid + 1;
                len = len - half - 1;
            } else {
                len = half;
            }
        }
        A.tokens[pos + 1] = first;
        if (A.dpos) A.dpos[0] = pos + 1;
    }
    lds_barrier();
    for (int i = tid; i < 625; i += kSmThreads) A.rng[i] = mt[i];
}

int sample_topk_launch(const float* logits, int n, float temp, int top_k, uint32_t* rng, int32_t* tokens, int* dpos,
                       int pos, double* probs, hipStream_t st, const double* dset)
{
    // sampler.cpp:66-67: std::min(top_k, 1000), std::min(temp, 2.0f)
    const int k = 1000 < top_k ? 1000 : top_k;
    const float t = 2.0f < temp ? 2.0f : temp;
    NC_CHECK_ARG(logits && rng && tokens && n >= 2 && n <= kSmMaxN, "sample_topk: bad arguments (n = %d)", n);
    NC_CHECK_ARG(dset || (k >= 1 && k <= n), "sample_topk: top_k %d for %d logits", top_k, n);
    NC_CHECK_ARG(dset || t > 0.0f, "sample_topk: temperature %g", (double)temp);
    SampleArgs a{logits, n, k, (double)t, rng, tokens, dpos, pos, probs, dset};
    hipLaunchKernelGGL(k_sample_topk, dim3(sample_grid(n)), dim3(kSmThreads), 0, st, a);
    return launch_status("k_sample_topk");
}

__global__ void k_exp(const double* __restrict__ x, double* __restrict__ y, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = exp_ref(x[i]);
}

}  // namespace nc

using namespace nc;

extern "C" {

int nc_rng_seed(uint32_t seed, uint32_t* state)
{
    NC_CHECK_ARG(state, "rng_seed: null state");
    mt_seed_host(seed, state);
    return NC_OK;
}

int nc_sample_topk(const float* logits, int n_vocab, float temp, int top_k, uint32_t* rng_state, int32_t* token,
                   double* probs, void* stream)
{
    return sample_topk_launch(logits, n_vocab, temp, top_k, rng_state, token, nullptr, -1, probs, stream_of(stream));
}

double nc_exp_host(double x) { return exp_ref(x); }

int nc_exp(const double* x, double* y, int64_t n, void* stream)
{
    NC_CHECK_ARG(x && y && n >= 0, "exp: bad arguments");
    if (!n) return NC_OK;
    hipLaunchKernelGGL(k_exp, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream_of(stream), x, y, n);
    return launch_status("k_exp");
}

}  // extern "C"
