// nc_device.h -- device-side numerics shared by the gfx950 kernels.
//
// Every helper reproduces one rounding step of the reference CPU path
// exactly; the kernels are compiled with -ffp-contract=off and IEEE fp32
// division / sqrt so that no step is fused or approximated.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nc_layout.h"

namespace nc {

constexpr int kWave = 64;

// Streaming loads (the nt bit) for data a launch reads once, the weights of
// a decode matvec: with the default policy the hundreds of MB of weights a
// decode step streams through L2 push out the small rows every launch
// re-reads (activations, norm gains, cache rows); streamed lines do not.
typedef unsigned int NcU32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint4* p)
{
    const NcU32x4 v = __builtin_nontemporal_load(reinterpret_cast<const NcU32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint16_t load_stream(const uint16_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint32_t load_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }
typedef unsigned int NcU32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 load_stream(const uint2* p)
{
    const NcU32x2 v = __builtin_nontemporal_load(reinterpret_cast<const NcU32x2*>(p));
    return make_uint2(v.x, v.y);
}

// Raw buffer loads (__builtin_amdgcn_raw_buffer_load_*): the resource's
// third dword for gfx9 untyped buffers, and the cache-policy operand of a
// streaming (nontemporal) load, as load_stream issues it.
constexpr int kBufferFlags = 0x00020000;
constexpr int kCacheStream = 2;

// fp16 -> fp32, exact (gten/gten_types.h:129-133).
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// fp32 -> fp16, round to nearest even (gten/gten_types.h:136-139; F16C
// _mm256_cvtps_ph(x, 0) in gten/ops.cpp:97-107).
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// std::exp(float) as the reference calls it (gten/ops.cpp:752,1072): the
// reference runs glibc's expf, which on x86-64 hosts with FMA is the
// table-driven algorithm of ARM's optimized-routines (math/expf.c,
// math/exp2f_data.c; MIT / Apache-2.0) compiled with fused multiply-adds.
// Restated here step by step so the device result equals the host's bit for
// bit:  x*N/ln2 = k + r (N = 32, round-to-nearest via the 1.5*2^52 shift),
// 2^(k/N) from a 32-entry table, 2^(r/N) by a cubic, all in double, one
// rounding to fp32 at the end.  kExp2Tab[i] = bits(2^(i/32)) - (i << 47).
constexpr uint64_t kExp2Tab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

NC_HD float expf_ref(float x)
{
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {                            // |x| >= 88 or NaN
        if (ux == 0xff800000u) return 0.0f;            // -inf
        if (abstop >= 0x7f8u) return x + x;            // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff(); // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;           // underflow
    }
    constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
    constexpr double kShift = 0x1.8p+52;
    constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    const uint64_t t = kExp2Tab[ki & 31u] + (ki << 47);
    const double s = __builtin_bit_cast(double, t);
    const double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// The device-held decode position, read with a vector load.  A scalar load
// would be waited for together with the kernel-argument loads (scalar loads
// complete out of order, so every wait on them is a wait for all), holding
// back every later load; a vector load is waited for only where the
// position is used.
__device__ __forceinline__ int load_pos(const int* dpos)
{
    return __hip_atomic_load(dpos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Greedy-token key of logit v at index idx: the largest key over a row is
// the index greedy_sample (gten/sampler.cpp:30-38) picks.  That scan starts
// from max = -inf, index 0, and takes a value only when `val > max`: NaN and
// -inf are never taken (rank 0 here, so with nothing else the smallest index,
// 0, wins), -0 ties with +0, and of equal values the first wins.  Key =
// order-preserving bits << 32 | ~index.  Every key is nonzero, so 0 can pad.
__device__ __forceinline__ unsigned long long greedy_key(float v, int idx)
{
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0;
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    if (v != v || u == 0xFF800000u) ord = 0;
    return ((unsigned long long)ord << 32) | (0xFFFFFFFFu - (uint32_t)idx);
}

// Orders this thread's earlier global stores and atomics before its later
// ones at agent scope, for data written with agent-scope atomic stores: those
// write through the XCD's L2, and the wait for their completion is the whole
// ordering they need (no L2 write-back, which a release fence adds for plain
// stores).
__device__ __forceinline__ void wait_stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Waits until this thread's global loads so far have returned, so the loads
// issued next do not queue ahead of their data.
__device__ __forceinline__ void wait_loads_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// accesses, not for its global loads (which may stay in flight across it).
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// DPP lane moves (gfx9 encodings): quad_perm, row_shr:n (0x110 + n),
// wave_shr:1 (0x138), row_bcast:15 (0x142), row_bcast:31 (0x143).  Lanes
// without a source read 0 (bound_ctrl) or keep `old` (masked rows).
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = true>
__device__ __forceinline__ int dpp_i(int v, int old = 0)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, BOUND_ZERO);
}
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_ZERO = true>
__device__ __forceinline__ float dpp_f(float v, float old = 0.0f)
{
    return __builtin_bit_cast(float, dpp_i<CTRL, ROW_MASK, BOUND_ZERO>(__builtin_bit_cast(int, v),
                                                                      __builtin_bit_cast(int, old)));
}
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppWaveShr1 = 0x138;
constexpr int kDppBcast15 = 0x142;
constexpr int kDppBcast31 = 0x143;

// Maximum over the 4 lanes of a quad (all four lanes active).
__device__ __forceinline__ float quad_max(float v)
{
    v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
    return fmaxf(v, dpp_f<kDppQuadXor2>(v));
}

// Maximum of a non-negative value across the 32 lanes of a half-wave:
// quad_perm (xor 1, xor 2), row_half_mirror and row_mirror DPP moves pair
// ever larger groups inside a 16-lane row, then a ds_swizzle exchanges the
// two rows (xor 16).  Lanes of the half-wave that are inactive read as 0.
__device__ __forceinline__ float half_wave_max(float v)
{
    v = quad_max(v);
    v = fmaxf(v, dpp_f<0x141>(v));  // row_half_mirror: lane i <-> 7 - i
    v = fmaxf(v, dpp_f<0x140>(v));  // row_mirror: lane i <-> 15 - i
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
}

// q8_quantize_block (gten/quants.cpp:16-30) for one 32-value block held one
// value per lane of a 32-lane group: absmax (order-free), delta =
// absmax/127 (IEEE division), fp16 delta stored, scale = 1/delta from the
// fp32 delta, q = (int8)roundf(x * scale).  `valid` lanes beyond a partial
// block's end contribute nothing.  Returns the int8 code; *d16 gets the
// stored delta.
__device__ __forceinline__ int8_t q8_quant_lane(float x, bool valid, uint16_t* d16)
{
    const float a = valid ? fabsf(x) : 0.0f;
    const float amax = half_wave_max(a);
    const float delta = amax / 127.0f;
    *d16 = f2h(delta);
    const float scale = delta != 0.0f ? 1.0f / delta : 0.0f;
    return (int8_t)roundf(x * scale);
}

// Q8 round trip of one value of a lane-resident block: what
// write_row_from_float followed by read_row_to_float leaves.
__device__ __forceinline__ float q8_roundtrip_lane(float x, bool valid)
{
    uint16_t d16;
    const int8_t q = q8_quant_lane(x, valid, &d16);
    return (float)q * h2f(d16);
}

__device__ __forceinline__ float f16_roundtrip(float x) { return h2f(f2h(x)); }

// Sequential fp32 sum of buf[0..n) in index order, every calling lane
// reading the same addresses (an LDS broadcast), so every lane ends with the
// sum.  This is the scalar accumulation loop of the reference's norms and
// softmax (gten/ops.cpp:673-683,833-835,1069-1075).  The adds form one
// dependent chain (about 6 cycles per add on gfx950); each CH-value chunk is
// read from LDS with all its loads in flight at once before its adds run
// (CH trades registers for fewer LDS round trips).
template <int CH = 64>
__device__ __forceinline__ float seq_sum(const float* buf, int n)
{
    float s = 0.0f;
    int c = 0;
    for (; c + CH <= n; c += CH) {
        float4 v[CH / 4];
#pragma unroll
        for (int j = 0; j < CH / 4; j++) v[j] = reinterpret_cast<const float4*>(buf + c)[j];
#pragma unroll
        for (int j = 0; j < CH / 4; j++) {
            s = s + v[j].x;
            s = s + v[j].y;
            s = s + v[j].z;
            s = s + v[j].w;
        }
    }
    for (; c + 4 <= n; c += 4) {
        const float4 v = *reinterpret_cast<const float4*>(buf + c);
        s = s + v.x;
        s = s + v.y;
        s = s + v.z;
        s = s + v.w;
    }
    for (; c < n; c++) s = s + buf[c];
    return s;
}

}  // namespace nc
