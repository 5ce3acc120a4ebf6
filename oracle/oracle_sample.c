/*
 * oracle_sample.c -- CPU restatement of the reference's top-k / temperature
 * sampling step (gten/sampler.cpp:63-143) with its random source made
 * reproducible: std::mt19937 seeded with a given 32-bit value instead of
 * std::random_device.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * The reference's step is built from C++ standard library calls; as
 * libstdc++ (GCC 11) implements them, with the reference's arguments:
 *   - std::partial_sort(begin, begin + k, end, greater-by-first): a heap
 *     select over [0, k) (make_heap, then for each later element that
 *     compares greater than the heap top, pop_heap onto it), then sort_heap.
 *     Elements equal to the k-th value enter or leave by the heap's sift
 *     order, which the functions below replay step by step.
 *   - std::exp on double: glibc's exp (called here).
 *   - std::discrete_distribution<int>(probs): sum = accumulate(0.0) over all
 *     n weights, each weight divided by the sum, std::partial_sum of those,
 *     the last entry set to 1.0; a draw is
 *     lower_bound(cumulative, generate_canonical<double, 53>(gen)).  With
 *     fewer than two weights the table is empty and the draw is 0 without
 *     using the generator.
 *   - generate_canonical<double, 53> over mt19937 (32-bit outputs): two
 *     outputs u1, u2; (u1 + u2 * 2^32) rounded to double, times 2^-64; a
 *     result of 1 becomes nextafter(1, 0).
 *   - std::mt19937: the Matsumoto-Nishimura generator (624-word state,
 *     seeding by x_i = 1812433253 (x_{i-1} ^ (x_{i-1} >> 30)) + i).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ---- std::mt19937 ------------------------------------------------------- */

void or_mt_seed(uint32_t seed, uint32_t* st)
{
    st[0] = seed;
    for (uint32_t i = 1; i < 624; i++) st[i] = 1812433253u * (st[i - 1] ^ (st[i - 1] >> 30)) + i;
    st[624] = 624;
}

static void mt_twist(uint32_t* mt)
{
    for (int i = 0; i < 624; i++) {
        const uint32_t y = (mt[i] & 0x80000000u) | (mt[(i + 1) % 624] & 0x7fffffffu);
        mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
    }
}

uint32_t or_mt_next(uint32_t* st)
{
    if (st[624] >= 624) {
        mt_twist(st);
        st[624] = 0;
    }
    uint32_t z = st[st[624]++];
    z ^= z >> 11;
    z ^= (z << 7) & 0x9d2c5680u;
    z ^= (z << 15) & 0xefc60000u;
    z ^= z >> 18;
    return z;
}

/* generate_canonical<double, 53>(mt19937) */
double or_mt_canonical(uint32_t* st)
{
    double sum = 0.0, tmp = 1.0;
    for (int k = 0; k < 2; k++) {
        sum += (double)or_mt_next(st) * tmp;
        tmp *= 4294967296.0;
    }
    double r = sum / tmp;
    if (r >= 1.0) r = nextafter(1.0, 0.0);
    return r;
}

/* ---- std::partial_sort's heap over (value, index) pairs ------------------- */

typedef struct {
    double v;
    int i;
} pair_t;

/* the reference's comparator: a before b when a.first > b.first */
static int before(const pair_t* a, const pair_t* b) { return a->v > b->v; }

/* __push_heap: move the hole up while its parent comes before `val` */
static void push_heap(pair_t* h, long hole, long top, pair_t val)
{
    long parent = (hole - 1) / 2;
    while (hole > top && before(&h[parent], &val)) {
        h[hole] = h[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    h[hole] = val;
}

/* __adjust_heap: sift the hole down to a leaf along the later-ordered child
 * (the right one unless it comes before the left), then push `val` up. */
static void adjust_heap(pair_t* h, long hole, long len, pair_t val)
{
    const long top = hole;
    long child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (before(&h[child], &h[child - 1])) child--;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    push_heap(h, hole, top, val);
}

static void make_heap(pair_t* h, long len)
{
    if (len < 2) return;
    for (long parent = (len - 2) / 2;; parent--) {
        adjust_heap(h, parent, len, h[parent]);
        if (parent == 0) return;
    }
}

/* __pop_heap(first, last, result): result takes the top, the top's slot
 * takes result's old value and sinks */
static void pop_heap(pair_t* h, long len, pair_t* result)
{
    const pair_t val = *result;
    *result = h[0];
    adjust_heap(h, 0, len, val);
}

/* std::partial_sort(a, a + k, a + n, before) */
static void partial_sort(pair_t* a, long k, long n)
{
    make_heap(a, k);
    for (long i = k; i < n; i++)
        if (before(&a[i], &a[0])) pop_heap(a, k, &a[i]);
    for (long len = k; len > 1; len--) pop_heap(a, len - 1, &a[len - 1]);
}

/* ---- one sampling step (gten/sampler.cpp:74-127) ------------------------- */

int or_topk_sample(const float* logits, int n, float temp, int top_k, uint32_t* st, double* probs_out)
{
    /* sampler.cpp:66-67: std::min(top_k, 1000), std::min(temp, 2.0f) */
    if (1000 < top_k) top_k = 1000;
    if (2.0f < temp) temp = 2.0f;
    pair_t* lp = (pair_t*)malloc((size_t)n * sizeof(pair_t));
    for (int j = 0; j < n; j++) {
        lp[j].v = (double)logits[j] / temp; /* sampler.cpp:96-97 */
        lp[j].i = j;
    }
    partial_sort(lp, top_k, n); /* sampler.cpp:100-107 */
    double sum_exp = 0;         /* sampler.cpp:110-117 */
    for (int j = 0; j < top_k; j++) {
        lp[j].v = exp(lp[j].v);
        sum_exp += lp[j].v;
    }
    for (int j = 0; j < top_k; j++) lp[j].v = lp[j].v / sum_exp;
    double* w = (double*)calloc((size_t)n, sizeof(double)); /* sampler.cpp:119-124 */
    for (int j = 0; j < top_k; j++) w[lp[j].i] = lp[j].v;
    free(lp);
    /* std::discrete_distribution (sampler.cpp:126-127) */
    int tok = 0;
    if (n >= 2) {
        double sum = 0.0;
        for (int j = 0; j < n; j++) sum += w[j];
        for (int j = 0; j < n; j++) w[j] = w[j] / sum;
        if (probs_out) memcpy(probs_out, w, (size_t)n * sizeof(double));
        for (int j = 1; j < n; j++) w[j] = w[j - 1] + w[j];
        w[n - 1] = 1.0;
        const double p = or_mt_canonical(st);
        long first = 0, len = n; /* lower_bound */
        while (len > 0) {
            const long half = len >> 1, mid = first + half;
            if (w[mid] < p) {
                first = mid + 1;
                len = len - half - 1;
            } else {
                len = half;
            }
        }
        tok = (int)first;
    } else if (probs_out) {
        for (int j = 0; j < n; j++) probs_out[j] = 0.0;
    }
    free(w);
    return tok;
}

/* ---- glibc exp as the reference calls it ---------------------------------- */

double or_exp(double x) { return exp(x); }

/* Inputs of the exp checks: a fixed xorshift stream, mixing the full range
 * of bit patterns, [-750, 710] (overflow, underflow and subnormal results)
 * and the logit range [-40, 40]. */
static double exp_probe(uint64_t seed, int64_t i)
{
    uint64_t s = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(i + 1);
    s ^= s >> 30;
    s *= 0xBF58476D1CE4E5B9ull;
    s ^= s >> 27;
    s *= 0x94D049BB133111EBull;
    s ^= s >> 31;
    const double u = (double)(s >> 11) * 0x1p-53;
    double x;
    switch (i & 3) {
    case 0: memcpy(&x, &s, 8); return x;
    case 1: return -750.0 + 1460.0 * u;
    default: return -40.0 + 80.0 * u;
    }
}

void or_exp_probe_inputs(uint64_t seed, int64_t start, int64_t n, double* x)
{
    for (int64_t i = 0; i < n; i++) x[i] = exp_probe(seed, start + i);
}

static int same_double(double a, double b)
{
    uint64_t ua, ub;
    memcpy(&ua, &a, 8);
    memcpy(&ub, &b, 8);
    return ua == ub || (isnan(a) && isnan(b));
}

int64_t or_check_exp_fn(double (*fn)(double), uint64_t seed, int64_t count, double* first_x)
{
    int64_t cnt = 0;
    int64_t f = -1;
#pragma omp parallel for reduction(+ : cnt) schedule(static)
    for (int64_t i = 0; i < count; i++) {
        const double x = exp_probe(seed, i);
        if (!same_double(exp(x), fn(x))) {
            cnt++;
#pragma omp critical
            if (f < 0 || i < f) f = i;
        }
    }
    *first_x = f < 0 ? 0.0 : exp_probe(seed, f);
    return cnt;
}

int64_t or_exp_mismatches(const double* x, const double* y, int64_t n, int64_t* first)
{
    int64_t cnt = 0, f = -1;
#pragma omp parallel for reduction(+ : cnt) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        if (!same_double(exp(x[i]), y[i])) {
            cnt++;
#pragma omp critical
            if (f < 0 || i < f) f = i;
        }
    }
    *first = f;
    return cnt;
}
