/*
 * oracle.c -- CPU restatement of the gten op numerics (test infrastructure).
 *
 * The checker for the HIP path.  It restates, in scalar C, the arithmetic of
 * the reference's AVX build (the configuration its CMakeLists.txt:22-125
 * selects): the same lane structure for every dot product, the same
 * sequential sums, the same rounding of every intermediate.  Compile with
 * -ffp-contract=off: the reference is built with -mavx -mf16c and no FMA, so
 * no a*b+c in it is ever contracted.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t ld16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline void st16(uint8_t* p, uint16_t v) { memcpy(p, &v, 2); }

/* fp16 -> fp32, exact (gten/gten_types.h:69-89 table of fpcvt::fp16_to_fp32). */
float or_fp16_to_fp32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero / subnormal: m * 2^-24, exact in fp32 */
        const float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* fp32 -> fp16, round to nearest even, NaN -> 0x7E00
 * (gten/gten_types.h:91-110; also what F16C's _mm256_cvtps_ph(x, 0) and
 * torch's .to(float16) produce for non-NaN input). */
uint16_t or_fp32_to_fp16(float f)
{
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    const uint32_t e = ax >> 23;
    if (e < 113) {
        /* result is an fp16 subnormal (or rounds up to the smallest normal):
         * value / 2^-24 = mant * 2^(e - 126), rounded to nearest even */
        if (e < 101) return sign; /* < 2^-26: rounds to zero */
        const uint32_t mant = (ax & 0x7fffffu) | (e ? 0x800000u : 0u);
        const uint32_t s = 126 - e; /* 14..25 */
        uint32_t q = mant >> s;
        const uint32_t rem = mant & ((1u << s) - 1u);
        const uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t q = ((e - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

void or_fp16_to_fp32_array(const uint16_t* in, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = or_fp16_to_fp32(in[i]);
}

void or_fp32_to_fp16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; i++) out[i] = or_fp32_to_fp16(in[i]);
}

size_t or_row_bytes(int dtype, int cols)
{
    switch (dtype) {
    case OR_Q8: return (size_t)((cols + OR_QBLOCK - 1) / OR_QBLOCK) * OR_Q8_BLOCK_BYTES;
    case OR_Q4: return (size_t)(cols / OR_QBLOCK) * OR_Q4_BLOCK_BYTES;
    case OR_F16: return (size_t)cols * 2;
    default: return (size_t)cols * 4;
    }
}

/* q8_quantize_block (gten/quants.cpp:16-30): absmax, delta = absmax/127,
 * stored as fp16, scale = 1/delta from the fp32 delta, roundf (half away). */
static void q8_quantize_block(const float* x, uint8_t* blk, int bs)
{
    float amax = 0.0f;
    for (int j = 0; j < bs; j++) {
        const float a = fabsf(x[j]);
        if (amax < a) amax = a; /* std::max(absmax, fabsf(x)) */
    }
    const float delta = amax / 127.0f;
    st16(blk, or_fp32_to_fp16(delta));
    const float scale = delta != 0.0f ? 1.0f / delta : 0.0f;
    int8_t* q = (int8_t*)(blk + 2);
    for (int j = 0; j < bs; j++) q[j] = (int8_t)roundf(x[j] * scale);
}

/* q8_quantize_row (gten/quants.cpp:140-158): a partial last block is
 * quantized on its own. */
void or_q8_quantize_row(const float* in, uint8_t* blocks, int n)
{
    const int nb = n / OR_QBLOCK;
    for (int i = 0; i < nb; i++) q8_quantize_block(in + i * OR_QBLOCK, blocks + i * OR_Q8_BLOCK_BYTES, OR_QBLOCK);
    const int rem = n % OR_QBLOCK;
    if (rem) q8_quantize_block(in + nb * OR_QBLOCK, blocks + nb * OR_Q8_BLOCK_BYTES, rem);
}

/* q8_dequantize_row / q4_dequantize_row (gten/quants.cpp:33-63,81-138,160-185):
 * x = float(q) * fp16_to_fp32(delta), one (exact) product. */
static void q8_dequantize_row(const uint8_t* blocks, float* out, int n)
{
    for (int i = 0; i < n; i++) {
        const uint8_t* b = blocks + (i / OR_QBLOCK) * OR_Q8_BLOCK_BYTES;
        const float d = or_fp16_to_fp32(ld16(b));
        out[i] = (float)((const int8_t*)(b + 2))[i % OR_QBLOCK] * d;
    }
}

static inline int q4_code(const uint8_t* p, int e)
{
    return e < 16 ? (p[e] >> 4) : (p[e - 16] & 0x0f);
}

static void q4_dequantize_row(const uint8_t* blocks, float* out, int n)
{
    for (int i = 0; i < n; i++) {
        const uint8_t* b = blocks + (i / OR_QBLOCK) * OR_Q4_BLOCK_BYTES;
        const float d = or_fp16_to_fp32(ld16(b));
        out[i] = (float)(q4_code(b + 2, i % OR_QBLOCK) - 7) * d;
    }
}

void or_read_row(const void* row, int dtype, float* out, int n)
{
    switch (dtype) {
    case OR_Q4: q4_dequantize_row((const uint8_t*)row, out, n); break;
    case OR_Q8: q8_dequantize_row((const uint8_t*)row, out, n); break;
    case OR_F16:
        for (int i = 0; i < n; i++) out[i] = or_fp16_to_fp32(((const uint16_t*)row)[i]);
        break;
    default: memcpy(out, row, (size_t)n * 4); break;
    }
}

void or_write_row(const float* in, void* row, int dtype, int n)
{
    switch (dtype) {
    case OR_Q8: or_q8_quantize_row(in, (uint8_t*)row, n); break;
    case OR_F16:
        for (int i = 0; i < n; i++) ((uint16_t*)row)[i] = or_fp32_to_fp16(in[i]);
        break;
    default: memcpy(row, in, (size_t)n * 4); break;
    }
}

/* Weight quantizers of the converters (tinyllama/tinyllama_to_gten.py:24-91).
 * torch semantics: delta = absmax / 127 (or 7) in fp32; scalars = 1/delta for
 * non-zero deltas; q = torch.round(x * scalar) (round half to even);
 * stored delta = delta.to(float16) (RNE). */
static void quantize_weights(const float* w, int64_t n_blocks, uint8_t* out, int q4)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_blocks; i++) {
        const float* x = w + i * OR_QBLOCK;
        float amax = 0.0f;
        for (int j = 0; j < OR_QBLOCK; j++) {
            const float a = fabsf(x[j]);
            if (a > amax) amax = a;
        }
        const float delta = amax / (q4 ? 7.0f : 127.0f);
        const float s = delta != 0.0f ? 1.0f / delta : 0.0f;
        float r[OR_QBLOCK];
        for (int j = 0; j < OR_QBLOCK; j++) r[j] = nearbyintf(x[j] * s); /* RNE */
        if (!q4) {
            uint8_t* b = out + i * OR_Q8_BLOCK_BYTES;
            st16(b, or_fp32_to_fp16(delta));
            for (int j = 0; j < OR_QBLOCK; j++) ((int8_t*)(b + 2))[j] = (int8_t)r[j];
        } else {
            uint8_t* b = out + i * OR_Q4_BLOCK_BYTES;
            st16(b, or_fp32_to_fp16(delta));
            for (int j = 0; j < 16; j++) {
                const uint8_t hi = (uint8_t)(r[j] + 7.0f);
                const uint8_t lo = (uint8_t)(r[j + 16] + 7.0f);
                b[2 + j] = (uint8_t)((hi << 4) | (lo & 0x0f));
            }
        }
    }
}

void or_q8_quantize_weights(const float* w, int64_t n_blocks, uint8_t* out) { quantize_weights(w, n_blocks, out, 0); }
void or_q4_quantize_weights(const float* w, int64_t n_blocks, uint8_t* out) { quantize_weights(w, n_blocks, out, 1); }

/* vec_dot_product_q8 (gten/ops.cpp:292-360, AVX path).  Per block i:
 * four int32 lane sums L_k over elements j with (j mod 8) in {2k, 2k+1}
 * (_mm_madd_epi16 pairs), t_k = float(L_k) * (d_a * d_b), acc_k += t_k in
 * block order, result (acc0 + acc1) + (acc2 + acc3) (two _mm_hadd_ps). */
float or_dot_q8(const uint8_t* a, const uint8_t* b, int n)
{
    const int nb = n / OR_QBLOCK;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < nb; i++) {
        const uint8_t* A = a + i * OR_Q8_BLOCK_BYTES;
        const uint8_t* B = b + i * OR_Q8_BLOCK_BYTES;
        const int8_t* qa = (const int8_t*)(A + 2);
        const int8_t* qb = (const int8_t*)(B + 2);
        int32_t L[4] = {0, 0, 0, 0};
        for (int j = 0; j < OR_QBLOCK; j++) L[(j & 7) >> 1] += (int32_t)qa[j] * (int32_t)qb[j];
        const float dd = or_fp16_to_fp32(ld16(A)) * or_fp16_to_fp32(ld16(B));
        for (int k = 0; k < 4; k++) acc[k] = acc[k] + (float)L[k] * dd;
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

/* vec_dot_product_q8_q4 (gten/ops.cpp:387-459): same lane/block structure;
 * weight element j decodes to code(j) - 7. */
float or_dot_q8_q4(const uint8_t* a, const uint8_t* b, int n)
{
    const int nb = n / OR_QBLOCK;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < nb; i++) {
        const uint8_t* A = a + i * OR_Q8_BLOCK_BYTES;
        const uint8_t* B = b + i * OR_Q4_BLOCK_BYTES;
        const int8_t* qa = (const int8_t*)(A + 2);
        int32_t L[4] = {0, 0, 0, 0};
        for (int j = 0; j < OR_QBLOCK; j++) L[(j & 7) >> 1] += (int32_t)qa[j] * (q4_code(B + 2, j) - 7);
        const float dd = or_fp16_to_fp32(ld16(A)) * or_fp16_to_fp32(ld16(B));
        for (int k = 0; k < 4; k++) acc[k] = acc[k] + (float)L[k] * dd;
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

/* vec_dot_product_f16 (gten/ops.cpp:208-228; gten/simd_ops.h:71-78): eight
 * fp32 lanes (lane = index mod 8), acc = (a*b) + acc without FMA, lanes
 * summed left to right, then the scalar tail. */
float or_dot_f16(const uint16_t* a, const uint16_t* b, int n)
{
    const int simd = (n / 8) * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < simd; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = or_fp16_to_fp32(a[i + j]) * or_fp16_to_fp32(b[i + j]) + acc[j];
    float s = acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
    for (int i = simd; i < n; i++) s += or_fp16_to_fp32(a[i]) * or_fp16_to_fp32(b[i]);
    return s;
}

/* vec_dot_product_f32 (gten/ops.cpp:245-265): as or_dot_f16 on fp32 rows. */
float or_dot_f32(const float* a, const float* b, int n)
{
    const int simd = (n / 8) * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < simd; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = a[i + j] * b[i + j] + acc[j];
    float s = acc[0] + acc[1] + acc[2] + acc[3] + acc[4] + acc[5] + acc[6] + acc[7];
    for (int i = simd; i < n; i++) s += a[i] * b[i];
    return s;
}

/* vec_dot_product dispatch (gten/ops.cpp:493-523). */
float or_dot(const void* a, int adt, const void* b, int bdt, int n)
{
    switch (adt) {
    case OR_Q8:
        return bdt == OR_Q4 ? or_dot_q8_q4((const uint8_t*)a, (const uint8_t*)b, n)
                            : or_dot_q8((const uint8_t*)a, (const uint8_t*)b, n);
    case OR_F16: return or_dot_f16((const uint16_t*)a, (const uint16_t*)b, n);
    default: return or_dot_f32((const float*)a, (const float*)b, n);
    }
}

float or_seq_sum(const float* y, int n)
{
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += y[i];
    return s;
}

float or_expf(float x) { return expf(x); }

/* Number of inputs among the bit patterns [start, start + count) where
 * fn(x) differs from expf(x) in its bits (NaN equal to NaN). */
int64_t or_check_expf_fn(float (*fn)(float), uint64_t start, uint64_t count, int64_t* first)
{
    int64_t cnt = 0, f = -1;
#pragma omp parallel for reduction(+ : cnt) schedule(static)
    for (int64_t i = 0; i < (int64_t)count; i++) {
        const float x = u2f((uint32_t)(start + (uint64_t)i));
        const float e = expf(x), y = fn(x);
        if (!((isnan(e) && isnan(y)) || f2u(e) == f2u(y))) {
            cnt++;
#pragma omp critical
            if (f < 0 || (int64_t)(start + (uint64_t)i) < f) f = (int64_t)(start + (uint64_t)i);
        }
    }
    *first = f;
    return cnt;
}

/* Number of i with bits(y[i]) != bits(expf(x[i])) (NaN results compare
 * equal to NaN); the first such index goes to *first (-1 if none). */
int64_t or_expf_mismatches(const float* x, const float* y, int64_t n, int64_t* first)
{
    int64_t cnt = 0, f = -1;
#pragma omp parallel for reduction(+ : cnt) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float e = expf(x[i]);
        const int same = (isnan(e) && isnan(y[i])) || f2u(e) == f2u(y[i]);
        if (!same) {
            cnt++;
#pragma omp critical
            if (f < 0 || i < f) f = i;
        }
    }
    *first = f;
    return cnt;
}

/* matmul_2d_impl (gten/ops.cpp:579-614): every output element of a row is
 * one full dot product (OpenMP over output columns), the row is then
 * written in the output dtype. */
void or_matmul(const void* x, int xdt, const void* w, int wdt, void* out, int odt, int K, int N,
               int start, int n_ctx, float* raw_out)
{
    const size_t xrb = or_row_bytes(xdt, K), wrb = or_row_bytes(wdt, K), orb = or_row_bytes(odt, N);
    float* buf = (float*)malloc((size_t)N * 4);
    for (int r = start; r < n_ctx; r++) {
        const uint8_t* xr = (const uint8_t*)x + (size_t)r * xrb;
#pragma omp parallel for schedule(static)
        for (int c = 0; c < N; c++) buf[c] = or_dot(xr, xdt, (const uint8_t*)w + (size_t)c * wrb, wdt, K);
        or_write_row(buf, (uint8_t*)out + (size_t)r * orb, odt, N);
        if (raw_out && r == n_ctx - 1) memcpy(raw_out, buf, (size_t)N * 4);
    }
    free(buf);
}

/* rms_norm_vec_f32 (gten/ops.cpp:830-846): sequential sum of squares
 * (std::pow(x, 2.0f) is x*x), rms = sqrtf(ss / n), y = x / (rms + 1e-6f) * w. */
static void rms_norm_vec(const float* x, const uint16_t* w, float* y, int n)
{
    float ss = 0.0f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float rms = sqrtf(ss / (float)n);
    for (int i = 0; i < n; i++) y[i] = x[i] / (rms + 1e-6f) * or_fp16_to_fp32(w[i]);
}

void or_rms_norm(const void* x, int dt, const uint16_t* w, void* out, int d, int start, int n_ctx)
{
    const size_t rb = or_row_bytes(dt, d);
    float* a = (float*)malloc((size_t)d * 8);
    float* y = a + d;
    for (int r = start; r < n_ctx; r++) {
        or_read_row((const uint8_t*)x + r * rb, dt, a, d);
        rms_norm_vec(a, w, y, d);
        or_write_row(y, (uint8_t*)out + r * rb, dt, d);
    }
    free(a);
}

/* 3-D rms_norm: one norm per head of d_head values (gten/ops.cpp:856-882). */
void or_rms_norm_heads(const void* x, int dt, const uint16_t* w, void* out, int n_heads, int d_head,
                       int start, int n_ctx)
{
    const size_t rb = or_row_bytes(dt, n_heads * d_head);
    const size_t hb = or_row_bytes(dt, d_head);
    float a[256], y[256];
    for (int r = start; r < n_ctx; r++)
        for (int h = 0; h < n_heads; h++) {
            or_read_row((const uint8_t*)x + r * rb + h * hb, dt, a, d_head);
            rms_norm_vec(a, w, y, d_head);
            or_write_row(y, (uint8_t*)out + r * rb + h * hb, dt, d_head);
        }
}

/* vec_layer_norm_f32 (gten/ops.cpp:669-698): sequential mean and variance,
 * eps added to the standard deviation. */
void or_layer_norm(const void* x, int dt, const uint16_t* w, const uint16_t* b, void* out, int d,
                   int start, int n_ctx)
{
    const size_t rb = or_row_bytes(dt, d);
    float* a = (float*)malloc((size_t)d * 8);
    float* y = a + d;
    for (int r = start; r < n_ctx; r++) {
        or_read_row((const uint8_t*)x + r * rb, dt, a, d);
        float sum = 0.0f;
        for (int i = 0; i < d; i++) sum += a[i];
        const float mean = sum / d;
        float ssq = 0.0f;
        for (int i = 0; i < d; i++) ssq += (a[i] - mean) * (a[i] - mean);
        const float sd = sqrtf(ssq / (float)d);
        for (int i = 0; i < d; i++)
            y[i] = ((a[i] - mean) / (sd + 1e-05f)) * or_fp16_to_fp32(w[i]) + or_fp16_to_fp32(b[i]);
        or_write_row(y, (uint8_t*)out + r * rb, dt, d);
    }
    free(a);
}

/* rotary_emb_impl (gten/ops.cpp:775-821): NEOX pairs (j, j + d_r/2) over the
 * first d_r = int(d_head * pct) dims of every head, angle
 * m * powf(10000, -(2j/d_r)); written back in the input dtype. */
void or_rotary_emb(const void* x, void* out, int dt, int d, int d_head, float rope_pct, int start,
                   int n_ctx)
{
    const size_t rb = or_row_bytes(dt, d);
    const int n_head = d / d_head;
    const int rope_d = (int)((float)d_head * rope_pct);
    const int d_half = rope_d / 2;
    const float df = (float)rope_d;
    float* a = (float*)malloc((size_t)d * 4);
    for (int r = start; r < n_ctx; r++) {
        or_read_row((const uint8_t*)x + r * rb, dt, a, d);
        const float m = (float)r;
        for (int h = 0; h < n_head; h++) {
            float* v = a + h * d_head;
            for (int j = 0; j < d_half; j++) {
                const float x0 = v[j], x1 = v[j + d_half];
                const float th = m * powf(10000.0f, -(2.0f * j / df));
                const float c = cosf(th), s = sinf(th);
                v[j] = x0 * c - x1 * s;
                v[j + d_half] = x0 * s + x1 * c;
            }
        }
        or_write_row(a, (uint8_t*)out + r * rb, dt, d);
    }
    free(a);
}

/* silu_impl (gten/ops.cpp:733-757): x / (1 + expf(-x)). */
void or_silu(const void* x, void* out, int dt, int d, int start, int n_ctx)
{
    const size_t rb = or_row_bytes(dt, d);
    float* a = (float*)malloc((size_t)d * 4);
    for (int r = start; r < n_ctx; r++) {
        or_read_row((const uint8_t*)x + r * rb, dt, a, d);
        for (int i = 0; i < d; i++) a[i] = a[i] / (1.0f + expf(-a[i]));
        or_write_row(a, (uint8_t*)out + r * rb, dt, d);
    }
    free(a);
}

static void binary_op(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx, int mul)
{
    const size_t rb = or_row_bytes(dt, d);
    float* x0 = (float*)malloc((size_t)d * 12);
    float* x1 = x0 + d;
    float* y = x1 + d;
    for (int r = start; r < n_ctx; r++) {
        or_read_row((const uint8_t*)a + r * rb, dt, x0, d);
        or_read_row((const uint8_t*)b + r * rb, dt, x1, d);
        for (int i = 0; i < d; i++) y[i] = mul ? x0[i] * x1[i] : x0[i] + x1[i];
        or_write_row(y, (uint8_t*)out + r * rb, dt, d);
    }
    free(x0);
}

/* mul_impl (gten/ops.cpp:925-953) and add_impl (gten/ops.cpp:973-1001). */
void or_multiply(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx)
{
    binary_op(a, b, out, dt, d, start, n_ctx, 1);
}

void or_add(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx)
{
    binary_op(a, b, out, dt, d, start, n_ctx, 0);
}

/* scale (gten/ops.cpp:146-164): in place, x * s. */
void or_scale(void* x, int dt, float s, int d, int start, int n_ctx)
{
    const size_t rb = or_row_bytes(dt, d);
    float* a = (float*)malloc((size_t)d * 4);
    for (int r = start; r < n_ctx; r++) {
        or_read_row((uint8_t*)x + r * rb, dt, a, d);
        for (int i = 0; i < d; i++) a[i] = a[i] * s;
        or_write_row(a, (uint8_t*)x + r * rb, dt, d);
    }
    free(a);
}

/* bias_add_inplace (gten/ops.cpp:639-666): x + float(bias). */
void or_bias_add(void* x, int dt, const uint16_t* b, int d, int start, int n_ctx)
{
    const size_t rb = or_row_bytes(dt, d);
    float* a = (float*)malloc((size_t)d * 4);
    for (int r = start; r < n_ctx; r++) {
        or_read_row((uint8_t*)x + r * rb, dt, a, d);
        for (int i = 0; i < d; i++) a[i] = a[i] + or_fp16_to_fp32(b[i]);
        or_write_row(a, (uint8_t*)x + r * rb, dt, d);
    }
    free(a);
}

/* qkv_attn (gten/ops.cpp:1017-1220).  For query row r and head h (kv head
 * h / (n_heads / n_kv_heads)): s_c = dot(q, k_c) * (1/sqrtf(d_head)) for
 * c <= r, -inf for r < c < n_ctx; softmax over the full n_ctx row (max,
 * expf(s - max), sequential sum, divide); the probability row is written in
 * the activation dtype and read back; out = 8-lane fp32 dot of that row with
 * the dequantized V column; the output row is written in the activation
 * dtype. */
void or_qkv_attn(const void* q, const void* k, const void* v, void* out, int dt, int n_heads,
                 int n_kv_heads, int d_head, int start, int n_ctx)
{
    const int qd = n_heads * d_head, kvd = n_kv_heads * d_head;
    const int group = n_heads / n_kv_heads;
    const size_t qrb = or_row_bytes(dt, qd), kvrb = or_row_bytes(dt, kvd), hb = or_row_bytes(dt, d_head);
    const float scale = 1.0f / sqrtf((float)d_head);
    float* s = (float*)malloc((size_t)n_ctx * 4);
    float* p = (float*)malloc((size_t)n_ctx * 4);
    uint8_t* prow = (uint8_t*)malloc(or_row_bytes(dt, n_ctx) + 64);
    float* vt = (float*)malloc((size_t)n_ctx * kvd * 4); /* transposed, dequantized V */
    float* vrow = (float*)malloc((size_t)kvd * 4);
    float* o = (float*)malloc((size_t)qd * 4);
    for (int c = 0; c < n_ctx; c++) {
        or_read_row((const uint8_t*)v + c * kvrb, dt, vrow, kvd);
        for (int j = 0; j < kvd; j++) vt[(size_t)j * n_ctx + c] = vrow[j];
    }
    for (int r = start; r < n_ctx; r++) {
        for (int h = 0; h < n_heads; h++) {
            const int g = h / group;
            const uint8_t* qh = (const uint8_t*)q + r * qrb + h * hb;
            for (int c = 0; c <= r; c++)
                s[c] = or_dot(qh, dt, (const uint8_t*)k + c * kvrb + g * hb, dt, d_head) * scale;
            for (int c = r + 1; c < n_ctx; c++) s[c] = -INFINITY;
            float mx = -INFINITY;
            for (int c = 0; c < n_ctx; c++)
                if (s[c] > mx) mx = s[c];
            float sum = 0.0f;
            for (int c = 0; c < n_ctx; c++) {
                s[c] = expf(s[c] - mx);
                sum += s[c];
            }
            for (int c = 0; c < n_ctx; c++) s[c] = s[c] / sum;
            or_write_row(s, prow, dt, n_ctx);
            or_read_row(prow, dt, p, n_ctx);
            for (int j = 0; j < d_head; j++)
                o[h * d_head + j] = or_dot_f32(p, vt + (size_t)(g * d_head + j) * n_ctx, n_ctx);
        }
        or_write_row(o, (uint8_t*)out + r * qrb, dt, qd);
    }
    free(s); free(p); free(prow); free(vt); free(vrow); free(o);
}

void or_token_embed(const void* table, int wdt, const int32_t* tokens, void* out, int adt, int d,
                    int start, int n_ctx)
{
    const size_t wrb = or_row_bytes(wdt, d), orb = or_row_bytes(adt, d);
    float* a = (float*)malloc((size_t)d * 4);
    for (int r = start; r < n_ctx; r++) {
        const uint8_t* src = (const uint8_t*)table + (size_t)tokens[r] * wrb;
        if (wdt == OR_Q4) {
            or_read_row(src, OR_Q4, a, d);
            or_write_row(a, (uint8_t*)out + r * orb, OR_Q8, d);
        } else {
            memcpy((uint8_t*)out + r * orb, src, wrb);
        }
    }
    free(a);
}

int or_argmax(const float* x, int n)
{
    float mx = -INFINITY;
    int idx = 0;
    for (int i = 0; i < n; i++)
        if (x[i] > mx) { mx = x[i]; idx = i; }
    return idx;
}

/* ---- synthetic data -------------------------------------------------------- */

/* splitmix64 finalizer. */
uint64_t or_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t counter_hash(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    return or_mix64(seed * 0x9E3779B97F4A7C15ull + stream * 0xD1B54A32D192ED03ull + ctr);
}

/* Irwin-Hall: S = sum of 12 uniforms in [0, 2^24) taken 2 per 64-bit hash
 * (bits 40..63 and 8..31); (S - 6*2^24) has unit variance in units of 2^24.
 * value = (float)((double)(S - 6*2^24) * (stddev * 2^-24)). */
void or_gen_normal(uint64_t seed, uint32_t tensor_id, float stddev, int64_t n, float* out)
{
    const double k = (double)stddev * (1.0 / 16777216.0);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        int64_t s = 0;
        for (int j = 0; j < 6; j++) {
            const uint64_t h = counter_hash(seed, tensor_id, (uint64_t)i * 6u + (uint64_t)j);
            s += (int64_t)((h >> 40) & 0xFFFFFFu) + (int64_t)((h >> 8) & 0xFFFFFFu);
        }
        out[i] = (float)((double)(s - 6 * 16777216LL) * k);
    }
}

void or_gen_tokens(uint64_t seed, int n, int vocab, int32_t* out)
{
    for (int i = 0; i < n; i++) {
        const uint64_t h = counter_hash(seed, 0x70CE5u, (uint64_t)i);
        out[i] = (int32_t)(((h >> 32) * (uint64_t)vocab) >> 32);
    }
}
