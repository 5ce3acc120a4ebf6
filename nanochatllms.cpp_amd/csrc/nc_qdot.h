// nc_qdot.h -- the reference's Q8 x Q8 / Q8 x Q4 block dot product
// (vec_dot_product_q8 / _q8_q4, gten/ops.cpp:292-490) as used by the matvec
// kernels: the activation block is staged once in LDS with its codes
// regrouped by AVX lane, and each weight block then gives its four exact
// integer lane sums with v_dot4 and the four fp32 terms
// t_k = float(L_k) * (d_x * d_w) that the kernels fold in block order.
#pragma once

#include "nc_device.h"

namespace nc {

// Dwords between staged blocks in LDS: 16 used, padded to 20 so that the
// 16-byte reads of consecutive blocks by consecutive lanes fall in distinct
// banks (a 64-byte stride would put every fourth lane on the same banks).
constexpr int kStage = 20;

__device__ __forceinline__ uint32_t pick_pair(uint32_t lo, uint32_t hi, int odd)
{
    // bytes (2*odd, 2*odd+1) of lo followed by the same bytes of hi
    return odd ? ((lo >> 16) | (hi & 0xFFFF0000u)) : ((lo & 0xFFFFu) | (hi << 16));
}

// Stage block i of a Q8 activation row: 16 dwords
// [xa0 xb0 xa1 xb1 xa2 xb2 xa3 xb3 | c0 c1 c2 c3 | dx 0 0 0]
// xa_k = codes {2k,2k+1,2k+8,2k+9}, xb_k = codes {2k+16,2k+17,2k+24,2k+25},
// c_k = -7 * (sum of those eight codes).
struct XRaw {
    uint4 a, b;
    uint16_t d16;
};

__device__ __forceinline__ XRaw load_x_block(const uint8_t* xrow, int nb, int i)
{
    const uint4* q = reinterpret_cast<const uint4*>(xrow + (size_t)i * 32);
    return XRaw{q[0], q[1], reinterpret_cast<const uint16_t*>(xrow + (size_t)nb * 32)[i]};
}

// A staged activation block: the lane codes, the lane offsets c_k and the
// delta.
struct StagedX {
    uint32_t xa[4], xb[4];
    int c[4];
    float dx;
};

// The staged form of a raw block, in registers.
__device__ __forceinline__ StagedX make_staged(const XRaw& x)
{
    const uint4 a = x.a, b = x.b;
    const uint32_t X[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    StagedX r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t xa = pick_pair(X[k >> 1], X[2 + (k >> 1)], k & 1);
        const uint32_t xb = pick_pair(X[4 + (k >> 1)], X[6 + (k >> 1)], k & 1);
        r.xa[k] = xa;
        r.xb[k] = xb;
        const int s = __builtin_amdgcn_sdot4((int)xa, 0x01010101, __builtin_amdgcn_sdot4((int)xb, 0x01010101, 0, false),
                                             false);
        r.c[k] = -7 * s;
    }
    r.dx = h2f(x.d16);
    return r;
}

__device__ __forceinline__ void stage_x_block(const XRaw& x, uint32_t* dst)
{
    const StagedX t = make_staged(x);
    uint4* d = reinterpret_cast<uint4*>(dst);
    d[0] = make_uint4(t.xa[0], t.xb[0], t.xa[1], t.xb[1]);
    d[1] = make_uint4(t.xa[2], t.xb[2], t.xa[3], t.xb[3]);
    d[2] = make_uint4((uint32_t)t.c[0], (uint32_t)t.c[1], (uint32_t)t.c[2], (uint32_t)t.c[3]);
    d[3] = make_uint4(__float_as_uint(t.dx), 0u, 0u, 0u);
}

__device__ __forceinline__ StagedX load_staged(const uint32_t* staged)
{
    const uint4* s = reinterpret_cast<const uint4*>(staged);
    const uint4 s0 = s[0], s1 = s[1], s2 = s[2], s3 = s[3];
    return StagedX{{s0.x, s0.z, s1.x, s1.z}, {s0.y, s0.w, s1.y, s1.w}, {(int)s2.x, (int)s2.y, (int)s2.z, (int)s2.w},
                   __uint_as_float(s3.x)};
}

// The four lane terms of one weight block against a staged activation
// block.  W holds the block's lane-permuted codes (4 dwords Q4, 8 Q8).
template <int WT>
__device__ __forceinline__ void q_block_terms(const StagedX& x, const uint4 (&w)[WT == Q4 ? 1 : 2], uint16_t dw16,
                                              float (&t)[4])
{
    constexpr int WD = WT == Q4 ? 4 : 8;
    const float dd = x.dx * h2f(dw16);
    uint32_t W[WD];
#pragma unroll
    for (int v = 0; v < WD / 4; v++) {
        W[4 * v] = w[v].x;
        W[4 * v + 1] = w[v].y;
        W[4 * v + 2] = w[v].z;
        W[4 * v + 3] = w[v].w;
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        int L;
        if (WT == Q4) {
            // value = code - 7: sum (code - 7) x = sum code x - 7 sum x, the
            // -7 sum x of the lane pre-computed at staging
            const uint32_t P = W[k];
            L = __builtin_amdgcn_sdot4((int)((P >> 4) & 0x0F0F0F0Fu), (int)x.xa[k], x.c[k], false);
            L = __builtin_amdgcn_sdot4((int)(P & 0x0F0F0F0Fu), (int)x.xb[k], L, false);
        } else {
            L = __builtin_amdgcn_sdot4((int)W[2 * k], (int)x.xa[k], 0, false);
            L = __builtin_amdgcn_sdot4((int)W[2 * k + 1], (int)x.xb[k], L, false);
        }
        t[k] = (float)L * dd;
    }
}

template <int WT>
__device__ __forceinline__ void q_block_terms(const uint32_t* staged, const uint4 (&w)[WT == Q4 ? 1 : 2], uint16_t dw16,
                                              float (&t)[4])
{
    q_block_terms<WT>(load_staged(staged), w, dw16, t);
}

}  // namespace nc
