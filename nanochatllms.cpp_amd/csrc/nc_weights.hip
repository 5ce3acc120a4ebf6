// nc_weights.hip -- weight generation, quantization and repacking.
//
// Stored weight semantics are the reference's: Q8/Q4 blocks of 32 values
// with an fp16 delta, quantized as the converters do (tinyllama/
// tinyllama_to_gten.py:24-91: fp32 delta = absmax/127 (or /7), fp32
// 1/delta, torch.round = round half to even, fp16 delta by RNE; Q4 codes
// +7, element j in the high nibble of byte j, element j+16 in the low).
// Only the placement in HBM differs (nc_layout.h): codes are lane-permuted
// within each block and the deltas live in a separate array, so a matvec
// thread reads a block's codes as aligned 16-byte vectors.
#include <cstring>
#include <vector>

#include "nc_act.h"
#include "nc_runtime.h"

namespace nc {

__host__ __device__ inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Irwin-Hall N(0, stddev): 12 24-bit uniforms from six counter-based
// splitmix64 hashes, exact integer sum, one double scaling, one fp32 rounding.
__global__ void k_gen_normal(uint64_t seed, uint32_t tensor_id, double k, int64_t n, float* __restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t s = 0;
    const uint64_t base = seed * 0x9E3779B97F4A7C15ull + (uint64_t)tensor_id * 0xD1B54A32D192ED03ull;
#pragma unroll
    for (int j = 0; j < 6; j++) {
        const uint64_t h = mix64(base + (uint64_t)i * 6u + (uint64_t)j);
        s += (int64_t)((h >> 40) & 0xFFFFFFu) + (int64_t)((h >> 8) & 0xFFFFFFu);
    }
    out[i] = (float)((double)(s - 6 * 16777216LL) * k);
}

// One half-wave per 32-value block (lane = element).
template <int WT>
__global__ __launch_bounds__(256) void k_quantize_weights(const float* __restrict__ w, int64_t n_blocks,
                                                          uint8_t* __restrict__ codes, uint16_t* __restrict__ deltas)
{
    const int64_t blk = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 5;
    const int e = threadIdx.x & 31;
    const bool valid = blk < n_blocks;
    const float x = valid ? w[blk * 32 + e] : 0.0f;
    const float amax = half_wave_max(fabsf(x));
    const float delta = amax / (WT == Q4 ? 7.0f : 127.0f);
    const float s = delta != 0.0f ? 1.0f / delta : 0.0f;
    const float r = rintf(x * s);  // round half to even, as torch.round
    const int k = (e & 7) >> 1, pos = wblock_byte_pos(e);
    if (WT == Q8) {
        if (valid) {
            codes[blk * 32 + (2 * k + (e >> 4)) * 4 + pos] = (uint8_t)(int8_t)r;
            if (e == 0) deltas[blk] = f2h(delta);
        }
    } else {
        const uint32_t code = (uint32_t)(uint8_t)(r + 7.0f);
        const uint32_t lo = (uint32_t)__shfl_down((int)code, 16, 32);
        if (valid && e < 16) {
            codes[blk * 16 + k * 4 + pos] = (uint8_t)((code << 4) | (lo & 0x0Fu));
            if (e == 0) deltas[blk] = f2h(delta);
        }
    }
}

__global__ void k_f16_weights(const float* __restrict__ w, int rows, int cols, int npad, uint16_t* __restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i - (int64_t)r * cols);
    out[f16_weight_index(r, c, npad)] = f2h(w[i]);
}

}  // namespace nc

using namespace nc;

static inline uint16_t ld16(const uint8_t* p) { uint16_t v; std::memcpy(&v, p, 2); return v; }

extern "C" {

int nc_act_pitch(int dtype, int cols) { return act_pitch(dtype, cols); }

int nc_act_from_reference(const void* ref, void* dev_layout, int dtype, int rows, int cols)
{
    NC_CHECK_ARG(ref && dev_layout && rows >= 0 && cols > 0, "act_from_reference: bad arguments");
    const int pitch = act_pitch(dtype, cols);
    const uint8_t* src = static_cast<const uint8_t*>(ref);
    uint8_t* dst = static_cast<uint8_t*>(dev_layout);
    std::memset(dst, 0, (size_t)rows * pitch);
    if (dtype == NC_Q8) {
        const int nb = qblocks(cols);
        for (int r = 0; r < rows; r++) {
            const uint8_t* s = src + (size_t)r * nb * 34;
            uint8_t* d = dst + (size_t)r * pitch;
            for (int b = 0; b < nb; b++) {
                const int n = b == nb - 1 && cols % 32 ? cols % 32 : 32;
                std::memcpy(d + b * 32, s + b * 34 + 2, n);
                std::memcpy(d + nb * 32 + b * 2, s + b * 34, 2);
            }
        }
    } else {
        const int eb = dtype == NC_F16 ? 2 : 4;
        for (int r = 0; r < rows; r++) std::memcpy(dst + (size_t)r * pitch, src + (size_t)r * cols * eb, (size_t)cols * eb);
    }
    return NC_OK;
}

int nc_act_to_reference(const void* dev_layout, void* ref, int dtype, int rows, int cols)
{
    NC_CHECK_ARG(ref && dev_layout && rows >= 0 && cols > 0, "act_to_reference: bad arguments");
    const int pitch = act_pitch(dtype, cols);
    const uint8_t* src = static_cast<const uint8_t*>(dev_layout);
    uint8_t* dst = static_cast<uint8_t*>(ref);
    if (dtype == NC_Q8) {
        const int nb = qblocks(cols);
        for (int r = 0; r < rows; r++) {
            const uint8_t* s = src + (size_t)r * pitch;
            uint8_t* d = dst + (size_t)r * nb * 34;
            for (int b = 0; b < nb; b++) {
                std::memcpy(d + b * 34, s + nb * 32 + b * 2, 2);
                std::memcpy(d + b * 34 + 2, s + b * 32, 32);
            }
        }
    } else {
        const int eb = dtype == NC_F16 ? 2 : 4;
        for (int r = 0; r < rows; r++) std::memcpy(dst + (size_t)r * cols * eb, src + (size_t)r * pitch, (size_t)cols * eb);
    }
    return NC_OK;
}

int nc_weight_bytes(int dtype, int rows, int cols, size_t* code_bytes, size_t* delta_bytes)
{
    NC_CHECK_ARG(code_bytes && delta_bytes && rows > 0 && cols > 0, "weight_bytes: bad arguments");
    if (dtype == NC_Q8 || dtype == NC_Q4) {
        NC_CHECK_ARG(cols % 32 == 0, "weight_bytes: %d columns is not a multiple of 32", cols);
        const size_t nblk = (size_t)rows * (cols / 32);
        *code_bytes = nblk * (dtype == NC_Q8 ? 32 : 16);
        *delta_bytes = nblk * 2;
    } else if (dtype == NC_F16) {
        NC_CHECK_ARG(cols % 64 == 0, "weight_bytes: fp16 weights need a multiple of 64 columns, got %d", cols);
        *code_bytes = (size_t)((rows + 7) & ~7) * cols * 2;
        *delta_bytes = 0;
    } else {
        return fail(NC_ERR_ARG, "weight_bytes: dtype %d", dtype);
    }
    return NC_OK;
}

int nc_weight_from_reference(const void* ref, int dtype, int rows, int cols, void* codes, void* deltas)
{
    size_t cb, db;
    int st = nc_weight_bytes(dtype, rows, cols, &cb, &db);
    if (st) return st;
    NC_CHECK_ARG(ref && codes && (deltas || dtype == NC_F16), "weight_from_reference: null buffer");
    const uint8_t* src = static_cast<const uint8_t*>(ref);
    if (dtype == NC_F16) {
        const int npad = (rows + 7) & ~7;
        uint16_t* out = static_cast<uint16_t*>(codes);
        std::memset(out, 0, cb);
        const uint16_t* s = reinterpret_cast<const uint16_t*>(src);
        for (int r = 0; r < rows; r++)
            for (int c = 0; c < cols; c++) {
                const int g = c >> 6, m = (c >> 3) & 7, j = c & 7;
                out[(((size_t)g * npad + r) * 8 + j) * 8 + m] = s[(size_t)r * cols + c];
            }
        return NC_OK;
    }
    const size_t nblk = (size_t)rows * (cols / 32);
    uint8_t* cd = static_cast<uint8_t*>(codes);
    uint16_t* dl = static_cast<uint16_t*>(deltas);
    for (size_t b = 0; b < nblk; b++) {
        if (dtype == NC_Q8) {
            const uint8_t* s = src + b * 34;
            dl[b] = ld16(s);
            for (int e = 0; e < 32; e++) {
                const int k = (e & 7) >> 1;
                const int pos = (e & 1) + (((e & 15) >> 3) << 1);
                cd[b * 32 + (2 * k + (e >> 4)) * 4 + pos] = s[2 + e];
            }
        } else {
            const uint8_t* s = src + b * 18;
            dl[b] = ld16(s);
            for (int j = 0; j < 16; j++) {
                const int k = (j & 7) >> 1;
                const int pos = (j & 1) + ((j >> 3) << 1);
                cd[b * 16 + k * 4 + pos] = s[2 + j];
            }
        }
    }
    return NC_OK;
}

int nc_gen_normal(uint64_t seed, uint32_t tensor_id, float stddev, int64_t n, float* out, void* stream)
{
    NC_CHECK_ARG(out && n >= 0, "gen_normal: bad arguments");
    if (!n) return NC_OK;
    const double k = (double)stddev * (1.0 / 16777216.0);
    const int64_t nblk = (n + 255) / 256;
    hipLaunchKernelGGL(k_gen_normal, dim3((unsigned)nblk), dim3(256), 0, stream_of(stream), seed, tensor_id, k, n, out);
    return launch_status("k_gen_normal");
}

int nc_weight_quantize(const float* w, nc_tensor* out, void* stream)
{
    NC_CHECK_ARG(w && out && out->data, "weight_quantize: null buffer");
    size_t cb, db;
    int st = nc_weight_bytes(out->dtype, out->rows, out->cols, &cb, &db);
    if (st) return st;
    hipStream_t s = stream_of(stream);
    if (out->dtype == NC_F16) {
        const int64_t n = (int64_t)out->rows * out->cols;
        hipLaunchKernelGGL(k_f16_weights, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w, out->rows, out->cols,
                           (out->rows + 7) & ~7, (uint16_t*)out->data);
        return launch_status("k_f16_weights");
    }
    NC_CHECK_ARG(out->deltas, "weight_quantize: null delta buffer");
    const int64_t nblk = (int64_t)out->rows * (out->cols / 32);
    const unsigned grid = (unsigned)((nblk + 7) / 8);
    if (out->dtype == NC_Q8)
        hipLaunchKernelGGL((k_quantize_weights<Q8>), dim3(grid), dim3(256), 0, s, w, nblk, (uint8_t*)out->data,
                           (uint16_t*)out->deltas);
    else
        hipLaunchKernelGGL((k_quantize_weights<Q4>), dim3(grid), dim3(256), 0, s, w, nblk, (uint8_t*)out->data,
                           (uint16_t*)out->deltas);
    return launch_status("k_quantize_weights");
}

}  // extern "C"

// ============================================================ copy ==

namespace nc {
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}
}  // namespace nc

extern "C" int nc_copy_d2d(void* dst, const void* src, size_t bytes, void* stream)
{
    NC_CHECK_ARG(dst && src && bytes % 16 == 0 && ((uintptr_t)dst | (uintptr_t)src) % 16 == 0,
                 "copy_d2d: %zu bytes (16-byte multiples and alignment)", bytes);
    if (!bytes) return NC_OK;
    const size_t n = bytes / 16;
    const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(nc::k_copy16, dim3(grid), dim3(256), 0, nc::stream_of(stream), (const uint4*)src, (uint4*)dst, n);
    return nc::launch_status("k_copy16");
}
