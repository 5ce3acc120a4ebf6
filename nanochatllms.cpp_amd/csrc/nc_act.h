// nc_act.h -- activation-row access for the elementwise / norm / attention
// kernels.  The thread that handles element e of a row sits on lane e % 64
// of some wavefront, so each 32-value Q8 block lives on one 32-lane half of
// a wavefront and can be (re)quantized with half-wave shuffles.
#pragma once

#include "nc_device.h"

namespace nc {

// Value of element e of an activation row (read_row_to_float,
// gten/ops.cpp:41-84): Q8 code * fp16 delta (one exact product), F16
// widened, F32 as is.
template <int ADT>
__device__ __forceinline__ float act_load(const uint8_t* row, int e, int dofs)
{
    if (ADT == Q8) {
        const int8_t q = reinterpret_cast<const int8_t*>(row)[e];
        return (float)q * h2f(reinterpret_cast<const uint16_t*>(row + dofs)[e >> 5]);
    } else if (ADT == F16) {
        return h2f(reinterpret_cast<const uint16_t*>(row)[e]);
    } else {
        return reinterpret_cast<const float*>(row)[e];
    }
}

// write_row_from_float for one element held by this lane (all 32 lanes of
// the block call together; lanes with valid = false skip the store).
template <int ADT>
__device__ __forceinline__ void act_store(uint8_t* row, int e, int dofs, float v, bool valid)
{
    if (ADT == Q8) {
        uint16_t d16;
        const int8_t q = q8_quant_lane(v, valid, &d16);
        if (valid) {
            reinterpret_cast<int8_t*>(row)[e] = q;
            if ((e & 31) == 0) reinterpret_cast<uint16_t*>(row + dofs)[e >> 5] = d16;
        }
    } else if (ADT == F16) {
        if (valid) reinterpret_cast<uint16_t*>(row)[e] = f2h(v);
    } else {
        if (valid) reinterpret_cast<float*>(row)[e] = v;
    }
}

// The value an activation of dtype ADT holds after write + read back.
template <int ADT>
__device__ __forceinline__ float act_roundtrip(float v, bool valid)
{
    if (ADT == Q8) return q8_roundtrip_lane(v, valid);
    if (ADT == F16) return f16_roundtrip(v);
    return v;
}

// (x_j, x_{j+d/2}) -> (x_j cos - x_{j+d/2} sin, x_j sin + x_{j+d/2} cos) on
// the first d_r dims of a 64-wide head held one value per lane.
__device__ __forceinline__ float rope_lane(float x, int lane, int d_half, const float2* cs)
{
    const int d_r = 2 * d_half;
    const int partner = lane < d_half ? lane + d_half : (lane < d_r ? lane - d_half : lane);
    const float xp = __shfl(x, partner);
    if (lane < d_half) {
        const float2 t = cs[lane];
        return x * t.x - xp * t.y;
    }
    if (lane < d_r) {
        const float2 t = cs[lane - d_half];
        return xp * t.y + x * t.x;
    }
    return x;
}

// The same with the lane's (cos, sin) pair already loaded (cs[lane] for
// lane < d_half, cs[lane - d_half] for d_half <= lane < 2 d_half).
__device__ __forceinline__ float rope_lane_pair(float x, int lane, int d_half, float2 t)
{
    const int d_r = 2 * d_half;
    const int partner = lane < d_half ? lane + d_half : (lane < d_r ? lane - d_half : lane);
    const float xp = __shfl(x, partner);
    if (lane < d_half) return x * t.x - xp * t.y;
    if (lane < d_r) return xp * t.y + x * t.x;
    return x;
}

// Code of element e (0..31) in a lane-permuted weight block (see
// nc_layout.h): dword index and byte position of the element.
__device__ __forceinline__ int wblock_byte_pos(int e) { return (e & 1) + (((e & 15) >> 3) << 1); }

__device__ __forceinline__ int q4_weight_code(const uint32_t* blk, int e)
{
    const int k = (e & 7) >> 1;
    const uint32_t byte = (blk[k] >> (8 * wblock_byte_pos(e))) & 0xFFu;
    return e < 16 ? (int)(byte >> 4) : (int)(byte & 0x0Fu);
}

__device__ __forceinline__ int q8_weight_code(const uint32_t* blk, int e)
{
    const int k = (e & 7) >> 1;
    const uint32_t dw = blk[2 * k + (e >> 4)];
    return (int)(int8_t)((dw >> (8 * wblock_byte_pos(e))) & 0xFFu);
}

// Index (in uint16 units) of (row, col) in the F16 weight layout.
__device__ __forceinline__ size_t f16_weight_index(int row, int col, int npad)
{
    const int g = col >> 6, m = (col >> 3) & 7, j = col & 7;
    return ((((size_t)g * npad + row) * 8 + j) * 8) + m;
}

}  // namespace nc
