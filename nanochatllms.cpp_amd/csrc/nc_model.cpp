// nc_model.cpp -- the reference's decoder models on one MI355X.
//
// One class covers the four model families of the reference (tinyllama/,
// zephyr/, minicpm/, openelm/): they share the pre-norm block structure and
// differ in the norm kind, qkv bias, partial RoPE, QK norm, tied embeddings,
// per-layer widths and MiniCPM's scalings.  The dataflow and every
// requantization point follow the reference's block forwards
// (tinyllama/tinyllama.cpp:88-138, zephyr/zephyr.cpp:24-76,
// minicpm/minicpm.cpp:42-110, openelm/openelm.cpp:33-146); the kernels fuse
// neighbouring ops but reproduce each intermediate write/read of the
// activation dtype.
//
// HBM layout per model:
//   weights: q|k|v rows and gate|up rows stored as one fused matrix each
//            (one matvec launch), o and down separate, norms fp16;
//   per layer: K and V caches [max_ctx, kv_dim] and the two residual stream
//            outputs [max_ctx, d] in the activation dtype (rows = positions);
//   scratch shared by the layers for the rows being processed.
// Decode keeps the token stream on the device: argmax writes the next token
// where the next step's embedding reads it, so steps need no host round trip.
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <memory>
#include <vector>

#include "nc_decode.h"
#include "nc_kernels.h"

namespace nc {

namespace {

struct Layer {
    int hq, hkv, qd, kvd, f;
    nc_tensor qkv{}, o{}, gu{}, down{};
    // chunk-major copies read by the prefill matmul (data == nullptr: none)
    nc_tensor cqkv{}, co{}, cgu{}, cdown{};
    uint16_t *attn_norm = nullptr, *attn_norm_b = nullptr, *mlp_norm = nullptr, *mlp_norm_b = nullptr;
    uint16_t *bq = nullptr, *bk = nullptr, *bv = nullptr, *qn = nullptr, *kn = nullptr;
    uint8_t *kc = nullptr, *vc = nullptr, *res1 = nullptr, *res2 = nullptr;
};

__global__ void k_fill_u16(uint16_t* p, uint16_t v, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_f32_to_f16(const float* in, uint16_t* out, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __builtin_bit_cast(uint16_t, (_Float16)in[i]);
}

// fp32 rows -> rows [row_off, row_off + rows) of an F16 weight of npad rows.
__global__ void k_f16_rows(const float* __restrict__ w, int rows, int cols, int row_off, int npad,
                           uint16_t* __restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)rows * cols) return;
    const int r = (int)(i / cols), c = (int)(i - (int64_t)r * cols);
    const int g = c >> 6, m = (c >> 3) & 7, j = c & 7;
    out[(((size_t)g * npad + row_off + r) * 8 + j) * 8 + m] = __builtin_bit_cast(uint16_t, (_Float16)w[i]);
}

}  // namespace

// .gten checkpoint magic number (the converters' GTEN_MAGIC_NUMBER,
// tinyllama/tinyllama_to_gten.py:7; checked in load_from_ckpt).
constexpr int64_t kGtenMagic = 0x454c49464e455447;

class Decoder {
public:
    nc_model_config cfg{};
    int adt = NC_Q8;
    int d = 0;
    hipStream_t st = nullptr;
    std::vector<void*> allocs;
    nc_tensor emb{}, lm{};
    uint16_t *norm_w = nullptr, *norm_b = nullptr;
    std::vector<Layer> L;
    float* rope = nullptr;
    int d_half = 0;
    uint8_t *x0 = nullptr, *xn = nullptr, *q_act = nullptr, *attn = nullptr, *m_act = nullptr;
    // The fused decode step's rows at fixed addresses (read without waiting
    // for the device-held position): the embedding of the step's token, the
    // residual sums after attention and after the MLP, and the position's
    // RoPE row.
    uint8_t *cur_x0 = nullptr, *cur1 = nullptr, *cur2 = nullptr;
    float* cur_rope = nullptr;
    float *qkv_raw = nullptr, *o_raw = nullptr, *gu_raw = nullptr, *down_raw = nullptr, *logits = nullptr;
    int32_t* tokens = nullptr;
    int n_cur = 0;        // tokens in the sequence processed so far
    int n_prompt = 0;     // prompt length of the current generation
    int max_qkv = 0, max_qd = 0, max_f = 0;
    // Single-row steps run the fused decode kernels (nc_decode.hip) when the
    // shapes allow it (Q8 activations, RMS norms); NC_DECODE_FUSED=0 keeps
    // the op-by-op path.
    bool fused = false;
    unsigned long long* am_scratch = nullptr;  // zeroed argmax scratch of the greedy step
    // Top-k sampling: the lm head writes logits only (sample_head), and the
    // sampler draws from the device-held mt19937 state rng (625 words) with
    // the device-held setting sample_set = {k, temp}, so one captured
    // sampling step serves every setting.
    bool sample_head = false;
    uint32_t* rng = nullptr;
    double* sample_set = nullptr;
    hipGraphExec_t sample_graph = nullptr;
    // Pinned host staging for every upload from host memory: the copy is a
    // DMA from memory the model owns, and each upload waits for its copy
    // before it returns (upload()), so no queued copy outlives its source.
    uint8_t* hstage = nullptr;
    size_t hstage_bytes = 0;
    // The lm head (lm, or emb when tied) in the head layout, read by the
    // fused step's lm-head kernel; rebuilt from the weight whenever it
    // changes (refresh_head).  data == nullptr: no copy.
    nc_tensor hl{};
    // The layers' chunk-major copies need rebuilding (a weight changed since).
    bool chunks_dirty = true;

    // Matvec launch timing: a start/end event pair recorded on the model's
    // stream around every matvec launch while profiling is on.
    struct Profile {
        bool on = false;
        std::vector<hipEvent_t> ev;
        std::vector<double> bytes;
        std::vector<int> kind;  // NC_PROF_* role, + NC_PROF_FUSED for the fused kernels
        size_t used = 0;
    } prof;

    // The captured step graphs live as long as the model: each is captured
    // on first use and only destroyed here, after the stream has drained.
    ~Decoder()
    {
        if (st) (void)hipStreamSynchronize(st);
        if (step_graph) (void)hipGraphExecDestroy(step_graph);
        if (sample_graph) (void)hipGraphExecDestroy(sample_graph);
        for (hipEvent_t e : prof.ev) (void)hipEventDestroy(e);
        for (void* p : allocs) (void)hipFree(p);
        if (hstage) (void)hipHostFree(hstage);
    }

    // Copies n host bytes to device memory through the pinned staging
    // buffer and waits for the copy (and everything queued before it).
    int upload(void* dst, const void* src, size_t n, const char* what)
    {
        NC_CHECK_ARG(n <= hstage_bytes, "%s: %zu bytes exceed the %zu-byte staging buffer", what, n, hstage_bytes);
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, what);
        std::memcpy(hstage, src, n);
        e = hipMemcpyAsync(dst, hstage, n, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return e == hipSuccess ? NC_OK : hip_fail(e, what);
    }

    // Waits for the stream when it leaves scope: calls that queue copies
    // into caller memory drain them on every return path.
    struct Drain {
        hipStream_t s;
        ~Drain() { (void)hipStreamSynchronize(s); }
    };

    // Algorithmic HBM bytes of one matvec launch: every weight byte once,
    // plus each activation row read and each fp32 output row written.
    static double matvec_bytes(const nc_tensor* w, int rows)
    {
        const double N = w->rows, K = w->cols;
        double wb, xb;
        if (w->dtype == NC_F16) { wb = 2.0 * N * K; xb = 2.0 * K; }
        else { wb = N * (K / 32) * (w->dtype == NC_Q8 ? 34.0 : 18.0); xb = (K / 32) * 34.0; }
        return wb + rows * (xb + 4.0 * N);
    }

    // fp16 decode row: the norm (after the residual add when braw, the
    // branch scaled as the model scales it) fused into the fp16 matvec that
    // consumes it; glu: the gate|up product with the SwiGLU epilogue, m row
    // out.
    int mv_ln(const uint8_t* a, const float* braw, uint8_t* h_out, const uint16_t* nw, const uint16_t* nb,
              const nc_tensor* w, float* out, uint8_t* m_out, bool glu, int role, const int* dpos)
    {
        const int pd = pitch(d);
        const int kind = norm_kind() == kNormLayer ? 0 : 1;
        const float bs = branch_scale();
        const bool timed = prof.on && prof.used + 2 <= prof.ev.size();
        int s = timed ? dmv_f16_nrm_launch(kind, a, pd, braw, bs, h_out, pd, nw, nb, w, out, m_out, glu, st, dpos,
                                           prof.ev[prof.used], prof.ev[prof.used + 1])
                      : dmv_f16_nrm_launch(kind, a, pd, braw, bs, h_out, pd, nw, nb, w, out, m_out, glu, st, dpos);
        if (s) return s;
        if (timed) {
            prof.used += 2;
            prof.bytes.push_back(matvec_bytes(w, 1));
            prof.kind.push_back(role | NC_PROF_FUSED);
        }
        return NC_OK;
    }

    // The norms of an fp16 model's single-row steps run inside the q|k|v and
    // gate|up matvecs (all but the final norm).
    bool ln_fused(int R) const
    {
        if (R != 1 || adt != NC_F16) return false;
        for (int l = 0; l < cfg.n_layers; l++)
            if (!dmv_f16_nrm_supported(&L[l].qkv, d, false) || !dmv_f16_nrm_supported(&L[l].gu, d, true)) return false;
        return true;
    }

    // fp16 decode row: gate|up product with the SwiGLU epilogue in one
    // launch, fp16 m row out.
    int mv_glu(const uint8_t* x, const nc_tensor* w, uint8_t* m_out)
    {
        const bool timed = prof.on && prof.used + 2 <= prof.ev.size();
        int s = timed ? matvec_f16_glu(x, w, m_out, st, prof.ev[prof.used], prof.ev[prof.used + 1])
                      : matvec_f16_glu(x, w, m_out, st);
        if (s) return s;
        if (timed) {
            prof.used += 2;
            prof.bytes.push_back(matvec_bytes(w, 1));
            prof.kind.push_back(NC_PROF_GATE_UP);
        }
        return NC_OK;
    }

    int mv(const uint8_t* x, int x_pitch, int rows, const nc_tensor* w, float* out, int out_pitch, int role,
           const nc_tensor* wc = nullptr)
    {
        const bool timed = prof.on && prof.used + 2 <= prof.ev.size();
        if (wc && !wc->data) wc = nullptr;
        int s = timed ? matvec_raw(x, adt, x_pitch, rows, w, out, out_pitch, st, prof.ev[prof.used],
                                   prof.ev[prof.used + 1], wc)
                      : matvec_raw(x, adt, x_pitch, rows, w, out, out_pitch, st, nullptr, nullptr, wc);
        if (s) return s;
        if (timed) {
            prof.used += 2;
            prof.bytes.push_back(matvec_bytes(w, rows));
            prof.kind.push_back(role);
        }
        return NC_OK;
    }

    int profile_begin(int max_launches)
    {
        NC_CHECK_ARG(max_launches > 0, "profile_begin: %d launches", max_launches);
        while (prof.ev.size() < (size_t)max_launches * 2) {
            hipEvent_t e;
            hipError_t r = hipEventCreate(&e);
            if (r != hipSuccess) return hip_fail(r, "hipEventCreate");
            prof.ev.push_back(e);
        }
        prof.used = 0;
        prof.bytes.clear();
        prof.kind.clear();
        prof.on = true;
        return NC_OK;
    }

    int profile_end(int* launches, double* total_ms, double* total_bytes, double* min_ms, double* max_ms)
    {
        prof.on = false;
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "profile_end");
        double tot = 0, mn = 1e30, mx = 0, by = 0;
        for (size_t i = 0; i + 1 < prof.used; i += 2) {
            float ms = 0;
            if ((e = hipEventElapsedTime(&ms, prof.ev[i], prof.ev[i + 1])) != hipSuccess)
                return hip_fail(e, "hipEventElapsedTime");
            tot += ms;
            mn = std::min(mn, (double)ms);
            mx = std::max(mx, (double)ms);
        }
        for (double b : prof.bytes) by += b;
        *launches = (int)(prof.used / 2);
        *total_ms = tot;
        *total_bytes = by;
        *min_ms = prof.used ? mn : 0;
        *max_ms = mx;
        return NC_OK;
    }

    int profile_launches(int cap, float* ms, double* bytes, int* kind, int* n_out)
    {
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "profile_launches");
        const int n = std::min(cap, (int)(prof.used / 2));
        for (int i = 0; i < n; i++) {
            if ((e = hipEventElapsedTime(&ms[i], prof.ev[2 * i], prof.ev[2 * i + 1])) != hipSuccess)
                return hip_fail(e, "hipEventElapsedTime");
            bytes[i] = prof.bytes[i];
            kind[i] = prof.kind[i];
        }
        *n_out = n;
        return NC_OK;
    }

    bool tied() const { return cfg.arch == NC_ARCH_MINICPM || cfg.arch == NC_ARCH_OPENELM; }
    int pitch(int cols) const { return act_pitch(adt, cols); }

    int alloc(void** p, size_t bytes)
    {
        int s = nc_malloc(p, bytes ? bytes : 16);
        if (s) return s;
        allocs.push_back(*p);
        hipError_t e = hipMemsetAsync(*p, 0, bytes ? bytes : 16, st);
        return e == hipSuccess ? NC_OK : hip_fail(e, "hipMemsetAsync");
    }
    template <class T>
    int alloc_t(T** p, size_t bytes)
    {
        void* v;
        int s = alloc(&v, bytes);
        *p = static_cast<T*>(v);
        return s;
    }

    int alloc_weight(nc_tensor* t, int dtype, int rows, int cols)
    {
        size_t cb, db;
        int s = nc_weight_bytes(dtype, rows, cols, &cb, &db);
        if (s) return s;
        t->dtype = dtype;
        t->rows = rows;
        t->cols = cols;
        t->pitch = 0;
        if ((s = alloc(&t->data, cb))) return s;
        if (db && (s = alloc(&t->deltas, db))) return s;
        return NC_OK;
    }

    int create(const nc_model_config* c)
    {
        cfg = *c;
        NC_CHECK_ARG(c->wdtype == NC_F16 || c->wdtype == NC_Q8 || c->wdtype == NC_Q4, "model: weight dtype %d",
                     c->wdtype);
        NC_CHECK_ARG(c->n_layers > 0 && c->n_layers <= NC_MAX_LAYERS, "model: %d layers", c->n_layers);
        NC_CHECK_ARG(c->d_head == 64, "model: head size %d (kernels are built for 64)", c->d_head);
        NC_CHECK_ARG(c->n_embd % 64 == 0 && c->max_ctx > 0 && c->n_vocab > 0, "model: bad shape");
        NC_CHECK_ARG(c->max_ctx <= kAttnMaxCtx, "model: max_ctx %d (the attention kernels take up to %d positions)",
                     c->max_ctx, kAttnMaxCtx);
        NC_CHECK_ARG(c->arch >= NC_ARCH_LLAMA && c->arch <= NC_ARCH_OPENELM, "model: arch %d", c->arch);
        if (!initialized()) {
            int s = nc_init(0);
            if (s) return s;
        }
        st = stream_of(nullptr);
        // staging for the largest upload: a prompt of max_ctx tokens (the
        // generator state of 625 words and the small fields fit too)
        hstage_bytes = std::max((size_t)8192, (size_t)(c->max_ctx + 1) * 4);
        hipError_t he = hipHostMalloc((void**)&hstage, hstage_bytes, hipHostMallocDefault);
        if (he != hipSuccess) {
            hstage = nullptr;
            return hip_fail(he, "hipHostMalloc");
        }
        adt = c->wdtype == NC_F16 ? NC_F16 : NC_Q8;
        if (const char* g = std::getenv("NC_DECODE_GRAPH")) use_graph = std::atoi(g) != 0;
        d = c->n_embd;
        const int mc = c->max_ctx;
        int s;
        if ((s = alloc_weight(&emb, c->wdtype, c->n_vocab, d))) return s;
        if (!tied() && (s = alloc_weight(&lm, c->wdtype, c->n_vocab, d))) return s;
        if ((s = alloc_t(&norm_w, (size_t)d * 2))) return s;
        if (c->arch == NC_ARCH_ZEPHYR && (s = alloc_t(&norm_b, (size_t)d * 2))) return s;
        L.resize(c->n_layers);
        for (int l = 0; l < c->n_layers; l++) {
            Layer& y = L[l];
            y.hq = c->n_heads[l];
            y.hkv = c->n_kv_heads[l];
            y.f = c->n_ffn[l];
            NC_CHECK_ARG(y.hq > 0 && y.hkv > 0 && y.hq % y.hkv == 0 && y.f % 64 == 0, "model: layer %d shape", l);
            y.qd = y.hq * 64;
            y.kvd = y.hkv * 64;
            max_qkv = std::max(max_qkv, y.qd + 2 * y.kvd);
            max_qd = std::max(max_qd, y.qd);
            max_f = std::max(max_f, y.f);
            if ((s = alloc_weight(&y.qkv, c->wdtype, y.qd + 2 * y.kvd, d))) return s;
            if ((s = alloc_weight(&y.o, c->wdtype, d, y.qd))) return s;
            if ((s = alloc_weight(&y.gu, c->wdtype, 2 * y.f, d))) return s;
            if ((s = alloc_weight(&y.down, c->wdtype, d, y.f))) return s;
            // the prefill matmul's chunk-major copies
            for (auto wc : {std::make_pair(&y.qkv, &y.cqkv), std::make_pair(&y.o, &y.co), std::make_pair(&y.gu, &y.cgu),
                            std::make_pair(&y.down, &y.cdown)})
                if (chunk_layout_supported(wc.first) &&
                    (s = alloc_weight(wc.second, c->wdtype, wc.first->rows, wc.first->cols)))
                    return s;
            if ((s = alloc_t(&y.attn_norm, (size_t)d * 2)) || (s = alloc_t(&y.mlp_norm, (size_t)d * 2))) return s;
            if (c->arch == NC_ARCH_ZEPHYR) {
                if ((s = alloc_t(&y.attn_norm_b, (size_t)d * 2)) || (s = alloc_t(&y.mlp_norm_b, (size_t)d * 2))) return s;
                if ((s = alloc_t(&y.bq, (size_t)y.qd * 2)) || (s = alloc_t(&y.bk, (size_t)y.kvd * 2)) ||
                    (s = alloc_t(&y.bv, (size_t)y.kvd * 2)))
                    return s;
            }
            if (c->arch == NC_ARCH_OPENELM)
                if ((s = alloc_t(&y.qn, 128)) || (s = alloc_t(&y.kn, 128))) return s;
            if ((s = alloc_t(&y.kc, (size_t)mc * pitch(y.kvd))) || (s = alloc_t(&y.vc, (size_t)mc * pitch(y.kvd))))
                return s;
            if ((s = alloc_t(&y.res1, (size_t)mc * pitch(d))) || (s = alloc_t(&y.res2, (size_t)mc * pitch(d)))) return s;
        }
        if ((s = alloc_t(&x0, (size_t)mc * pitch(d))) || (s = alloc_t(&xn, (size_t)mc * pitch(d))) ||
            (s = alloc_t(&q_act, (size_t)mc * pitch(max_qd))) || (s = alloc_t(&attn, (size_t)mc * pitch(max_qd))) ||
            (s = alloc_t(&m_act, (size_t)mc * pitch(max_f))) ||
            (s = alloc_t(&qkv_raw, (size_t)mc * max_qkv * 4)) || (s = alloc_t(&o_raw, (size_t)mc * d * 4)) ||
            (s = alloc_t(&gu_raw, (size_t)mc * 2 * max_f * 4)) || (s = alloc_t(&down_raw, (size_t)mc * d * 4)) ||
            (s = alloc_t(&logits, (size_t)c->n_vocab * 4)) || (s = alloc_t(&tokens, (size_t)(mc + 1) * 4)))
            return s;
        if ((s = alloc_t(&am_scratch, (size_t)kDmvArgmaxWords * 8))) return s;
        if ((s = alloc_t(&cur_x0, pitch(d))) || (s = alloc_t(&cur1, pitch(d))) || (s = alloc_t(&cur2, pitch(d))))
            return s;
        fused = fused_supported();
        if (const char* f = std::getenv("NC_DECODE_FUSED")) fused = fused && std::atoi(f) != 0;
        // the fused step's lm head reads a copy of its weight in the head layout
        if (fused && head_layout_supported(c->wdtype, c->n_vocab, d)) {
            size_t cb, db;
            if ((s = head_layout_bytes(c->wdtype, c->n_vocab, d, &cb, &db)) || (s = alloc(&hl.data, cb)) ||
                (s = alloc(&hl.deltas, db)))
                return s;
            hl.dtype = c->wdtype;
            hl.rows = c->n_vocab;
            hl.cols = d;
        }
        // RoPE table from the host libm, the reference's expression
        d_half = static_cast<int>((float)c->d_head * c->rope_pct) / 2;
        std::vector<float> tab((size_t)mc * std::max(d_half, 1) * 2);
        if ((s = nc_rope_table(mc, c->d_head, c->rope_pct, tab.data()))) return s;
        if ((s = alloc_t(&rope, tab.size() * 4))) return s;
        if ((s = alloc_t(&cur_rope, (size_t)std::max(d_half, 1) * 8))) return s;
        hipError_t e = hipMemcpyAsync(rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return e == hipSuccess ? NC_OK : hip_fail(e, "rope table upload");
    }

    // ------------------------------------------------------------ weights --

    // Location of weight (layer, slot): the fused matrix and its row offset,
    // or an fp16 vector.
    struct Loc {
        nc_tensor* mat = nullptr;
        int row_off = 0, rows = 0, cols = 0;
        uint16_t* vec = nullptr;
        int n = 0;
        int kind = 0;  // 0 matrix, 1 gain (1.0), 2 zero bias, 3 random fp16 vector
    };

    int locate(int layer, int slot, Loc* o)
    {
        *o = Loc{};
        if (layer < 0) {
            switch ((unsigned)slot) {
            case NC_TID_EMB: o->mat = &emb; o->rows = cfg.n_vocab; o->cols = d; return NC_OK;
            case NC_TID_LM:
                if (tied()) return fail(NC_ERR_ARG, "model: lm head is tied to the embedding");
                o->mat = &lm; o->rows = cfg.n_vocab; o->cols = d; return NC_OK;
            case NC_TID_NORM: o->vec = norm_w; o->n = d; o->kind = 1; return NC_OK;
            case NC_TID_NORM_B:
                if (!norm_b) return fail(NC_ERR_ARG, "model: no final norm bias");
                o->vec = norm_b; o->n = d; o->kind = 2; return NC_OK;
            default: return fail(NC_ERR_ARG, "model: global slot %#x", (unsigned)slot);
            }
        }
        NC_CHECK_ARG(layer < cfg.n_layers, "model: layer %d", layer);
        Layer& y = L[layer];
        switch (slot) {
        case NC_W_Q: o->mat = &y.qkv; o->rows = y.qd; o->cols = d; return NC_OK;
        case NC_W_K: o->mat = &y.qkv; o->row_off = y.qd; o->rows = y.kvd; o->cols = d; return NC_OK;
        case NC_W_V: o->mat = &y.qkv; o->row_off = y.qd + y.kvd; o->rows = y.kvd; o->cols = d; return NC_OK;
        case NC_W_O: o->mat = &y.o; o->rows = d; o->cols = y.qd; return NC_OK;
        case NC_W_GATE: o->mat = &y.gu; o->rows = y.f; o->cols = d; return NC_OK;
        case NC_W_UP: o->mat = &y.gu; o->row_off = y.f; o->rows = y.f; o->cols = d; return NC_OK;
        case NC_W_DOWN: o->mat = &y.down; o->rows = d; o->cols = y.f; return NC_OK;
        case NC_W_ATTN_NORM: o->vec = y.attn_norm; o->n = d; o->kind = 1; return NC_OK;
        case NC_W_MLP_NORM: o->vec = y.mlp_norm; o->n = d; o->kind = 1; return NC_OK;
        case NC_W_ATTN_NORM_B: o->vec = y.attn_norm_b; o->n = d; o->kind = 2; break;
        case NC_W_MLP_NORM_B: o->vec = y.mlp_norm_b; o->n = d; o->kind = 2; break;
        case NC_W_Q_BIAS: o->vec = y.bq; o->n = y.qd; o->kind = 3; break;
        case NC_W_K_BIAS: o->vec = y.bk; o->n = y.kvd; o->kind = 3; break;
        case NC_W_V_BIAS: o->vec = y.bv; o->n = y.kvd; o->kind = 3; break;
        case NC_W_Q_NORM: o->vec = y.qn; o->n = 64; o->kind = 1; break;
        case NC_W_K_NORM: o->vec = y.kn; o->n = 64; o->kind = 1; break;
        default: return fail(NC_ERR_ARG, "model: slot %d", slot);
        }
        if (!o->vec) return fail(NC_ERR_ARG, "model: this architecture has no slot %d", slot);
        return NC_OK;
    }

    // Byte offsets of the sub-matrix in a fused Q4/Q8 weight.
    static size_t code_off(const nc_tensor* m, int row_off)
    {
        return (size_t)row_off * (m->cols / 32) * (m->dtype == NC_Q8 ? 32 : 16);
    }

    int init_synthetic(uint64_t seed)
    {
        size_t max_n = (size_t)cfg.n_vocab * d;
        for (const Layer& y : L)
            max_n = std::max(max_n, std::max((size_t)2 * y.f * d, (size_t)(y.qd + 2 * y.kvd) * d));
        float* tmp = nullptr;
        int s = nc_malloc((void**)&tmp, max_n * 4);
        if (s) return s;
        std::unique_ptr<void, void (*)(void*)> guard(tmp, [](void* p) { (void)hipFree(p); });
        auto one = [&](int layer, int slot) -> int {
            Loc o;
            int r = locate(layer, slot, &o);
            if (r) return NC_OK;  // slot not present in this architecture
            const uint32_t tid = layer < 0 ? (uint32_t)slot : (uint32_t)(layer * 32 + slot);
            if (o.mat) {
                const int64_t n = (int64_t)o.rows * o.cols;
                if ((r = nc_gen_normal(seed, tid, 0.02f, n, tmp, st))) return r;
                if (o.mat->dtype == NC_F16) {
                    hipLaunchKernelGGL(k_f16_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, tmp, o.rows,
                                       o.cols, o.row_off, (o.mat->rows + 7) & ~7, (uint16_t*)o.mat->data);
                    return launch_status("k_f16_rows");
                }
                nc_tensor sub = *o.mat;
                sub.rows = o.rows;
                sub.data = (uint8_t*)o.mat->data + code_off(o.mat, o.row_off);
                sub.deltas = (uint16_t*)o.mat->deltas + (size_t)o.row_off * (o.cols / 32);
                return nc_weight_quantize(tmp, &sub, st);
            }
            const unsigned grid = (unsigned)((o.n + 255) / 256);
            if (o.kind == 3) {
                if ((r = nc_gen_normal(seed, tid, 0.02f, o.n, tmp, st))) return r;
                hipLaunchKernelGGL(k_f32_to_f16, dim3(grid), dim3(256), 0, st, tmp, o.vec, (int64_t)o.n);
            } else {
                hipLaunchKernelGGL(k_fill_u16, dim3(grid), dim3(256), 0, st, o.vec,
                                   (uint16_t)(o.kind == 1 ? 0x3C00u : 0u), (int64_t)o.n);
            }
            return launch_status("weight fill");
        };
        chunks_dirty = true;
        const unsigned globals[4] = {NC_TID_EMB, NC_TID_NORM, NC_TID_NORM_B, NC_TID_LM};
        for (unsigned g : globals)
            if ((s = one(-1, (int)g))) return s;
        for (int l = 0; l < cfg.n_layers; l++)
            for (int slot = 0; slot <= NC_W_K_NORM; slot++)
                if ((s = one(l, slot))) return s;
        if ((s = refresh_head())) return s;
        hipError_t e = hipStreamSynchronize(st);
        return e == hipSuccess ? NC_OK : hip_fail(e, "init_synthetic");
    }

    // The chunk-major copies of the layer weights, rebuilt from the weights
    // when one changed (before a prefill reads them).
    int refresh_chunks()
    {
        if (!chunks_dirty) return NC_OK;
        for (Layer& y : L)
            for (auto wc : {std::make_pair(&y.qkv, &y.cqkv), std::make_pair(&y.o, &y.co),
                            std::make_pair(&y.gu, &y.cgu), std::make_pair(&y.down, &y.cdown)})
                if (wc.second->data) {
                    int s = chunk_layout_launch(wc.first, wc.second->data, wc.second->deltas, st);
                    if (s) return s;
                }
        chunks_dirty = false;
        return NC_OK;
    }

    // The head-layout copy of the lm head, rebuilt from the weight.
    int refresh_head()
    {
        if (!hl.data) return NC_OK;
        return head_layout_launch(tied() ? &emb : &lm, hl.data, hl.deltas, st);
    }

    int set_weight(int layer, int slot, const void* ref, size_t n_bytes)
    {
        const bool head = layer < 0 && (slot == NC_TID_LM || (slot == NC_TID_EMB && tied()));
        int s = set_weight_only(layer, slot, ref, n_bytes);
        if (s || !head) return s;
        if ((s = refresh_head())) return s;
        hipError_t e = hipStreamSynchronize(st);
        return e == hipSuccess ? NC_OK : hip_fail(e, "set_weight: head layout");
    }

    int set_weight_only(int layer, int slot, const void* ref, size_t n_bytes)
    {
        chunks_dirty = true;
        Loc o;
        int s = locate(layer, slot, &o);
        if (s) return s;
        hipError_t e = hipSuccess;
        if (o.vec) {
            NC_CHECK_ARG(n_bytes == (size_t)o.n * 2, "set_weight: %zu bytes for %d fp16 values", n_bytes, o.n);
            e = hipMemcpy(o.vec, ref, n_bytes, hipMemcpyHostToDevice);
            return e == hipSuccess ? NC_OK : hip_fail(e, "set_weight");
        }
        const int dt = o.mat->dtype;
        const size_t want = dt == NC_F16 ? (size_t)o.rows * o.cols * 2
                                         : (size_t)o.rows * (o.cols / 32) * (dt == NC_Q8 ? 34 : 18);
        NC_CHECK_ARG(n_bytes == want, "set_weight: payload %zu bytes, expected %zu", n_bytes, want);
        if (dt == NC_F16) {
            // per 64-column group, the sub-matrix rows are one contiguous run
            const int npad = (o.mat->rows + 7) & ~7, G = o.cols / 64;
            const uint16_t* src = static_cast<const uint16_t*>(ref);
            std::vector<uint16_t> run((size_t)o.rows * 64);
            for (int g = 0; g < G && e == hipSuccess; g++) {
                for (int r = 0; r < o.rows; r++)
                    for (int m = 0; m < 8; m++)
                        for (int j = 0; j < 8; j++) run[((size_t)r * 8 + j) * 8 + m] = src[(size_t)r * o.cols + 64 * g + 8 * m + j];
                e = hipMemcpy((uint16_t*)o.mat->data + ((size_t)g * npad + o.row_off) * 64, run.data(), run.size() * 2,
                              hipMemcpyHostToDevice);
            }
            return e == hipSuccess ? NC_OK : hip_fail(e, "set_weight");
        }
        size_t cb, db;
        if ((s = nc_weight_bytes(dt, o.rows, o.cols, &cb, &db))) return s;
        std::vector<uint8_t> codes(cb), deltas(db);
        if ((s = nc_weight_from_reference(ref, dt, o.rows, o.cols, codes.data(), deltas.data()))) return s;
        e = hipMemcpy((uint8_t*)o.mat->data + code_off(o.mat, o.row_off), codes.data(), cb, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy((uint16_t*)o.mat->deltas + (size_t)o.row_off * (o.cols / 32), deltas.data(), db,
                          hipMemcpyHostToDevice);
        return e == hipSuccess ? NC_OK : hip_fail(e, "set_weight");
    }

    // ------------------------------------------------------- checkpoint --

    // The tensors of a .gten checkpoint in file order, as each model's
    // load_from_ckpt reads them (tinyllama/tinyllama.cpp:131-187,
    // zephyr/zephyr.cpp:79-150, minicpm/minicpm.cpp:113-166,
    // openelm/openelm.cpp:201-262).
    std::vector<std::pair<int, int>> gten_order() const
    {
        std::vector<std::pair<int, int>> o;
        const int a = cfg.arch;
        o.push_back({-1, NC_TID_EMB});
        for (int l = 0; l < cfg.n_layers; l++) {
            if (a == NC_ARCH_ZEPHYR) {
                for (int s : {NC_W_Q, NC_W_Q_BIAS, NC_W_K, NC_W_K_BIAS, NC_W_V, NC_W_V_BIAS, NC_W_O, NC_W_GATE, NC_W_UP,
                              NC_W_DOWN, NC_W_ATTN_NORM, NC_W_ATTN_NORM_B, NC_W_MLP_NORM, NC_W_MLP_NORM_B})
                    o.push_back({l, s});
            } else {
                for (int s : {NC_W_Q, NC_W_K, NC_W_V, NC_W_O, NC_W_GATE, NC_W_UP, NC_W_DOWN}) o.push_back({l, s});
                if (a == NC_ARCH_OPENELM) {
                    o.push_back({l, NC_W_Q_NORM});
                    o.push_back({l, NC_W_K_NORM});
                }
                o.push_back({l, NC_W_ATTN_NORM});
                o.push_back({l, NC_W_MLP_NORM});
            }
        }
        o.push_back({-1, NC_TID_NORM});
        if (a == NC_ARCH_ZEPHYR) o.push_back({-1, NC_TID_NORM_B});
        if (!tied()) o.push_back({-1, NC_TID_LM});
        return o;
    }

    // Payload bytes of one tensor in the reference's storage
    // (Tensor::nbytes: Q8 / Q4 blocks of 34 / 18 bytes, or fp16 values).
    int ref_bytes(int layer, int slot, size_t* n)
    {
        Loc o;
        int s = locate(layer, slot, &o);
        if (s) return s;
        if (o.vec) {
            *n = (size_t)o.n * 2;
        } else {
            const int dt = o.mat->dtype;
            *n = dt == NC_F16 ? (size_t)o.rows * o.cols * 2 : (size_t)o.rows * (o.cols / 32) * (dt == NC_Q8 ? 34 : 18);
        }
        return NC_OK;
    }

    // load_from_ckpt: the magic number, then per tensor in file order a
    // layer header and a weight record (read_layer_header /
    // read_into_weight, gten/utils.cpp:29-61) -- name size, name, payload
    // size, payload -- with the reference's checks (magic, payload size,
    // plus a truncated file) as errors.  Records before a failing one have
    // already replaced their weights.
    int load_gten(const char* path)
    {
        std::ifstream f(path, std::ios::binary);
        if (!f) return fail(NC_ERR_ARG, "load_gten: cannot open `%s`", path);
        int64_t magic = 0;
        f.read(reinterpret_cast<char*>(&magic), sizeof(magic));
        if (!f || magic != kGtenMagic)
            return fail(NC_ERR_ARG, "Magic number in the binary does not match the expected one.");
        std::vector<char> payload;
        auto read_name = [&](std::string* name) {
            int32_t n = 0;
            f.read(reinterpret_cast<char*>(&n), sizeof(n));
            if (!f || n < 0 || n > (1 << 20)) return false;
            name->resize(n);
            f.read(name->data(), n);
            return (bool)f;
        };
        for (const auto& [layer, slot] : gten_order()) {
            std::string layer_name, weight_name;
            if (!read_name(&layer_name) || !read_name(&weight_name))
                return fail(NC_ERR_ARG, "load_gten: `%s` ends before tensor (%d, %#x)", path, layer, slot);
            int32_t size = 0;
            f.read(reinterpret_cast<char*>(&size), sizeof(size));
            if (!f) return fail(NC_ERR_ARG, "load_gten: `%s` ends before tensor (%d, %#x)", path, layer, slot);
            size_t want;
            int s = ref_bytes(layer, slot, &want);
            if (s) return s;
            if (size < 0 || (size_t)size != want)
                return fail(NC_ERR_ARG, "Weight `%s` data size: %d does not match the expected size: %zu.",
                            weight_name.c_str(), size, want);
            payload.resize(want);
            f.read(payload.data(), (std::streamsize)want);
            if (!f) return fail(NC_ERR_ARG, "load_gten: `%s` ends inside weight `%s`", path, weight_name.c_str());
            if ((s = set_weight(layer, slot, payload.data(), want))) return s;
        }
        return NC_OK;
    }

    // Inverse of set_weight: the stored weight in the reference's bytes.
    int get_weight(int layer, int slot, void* ref, size_t n_bytes)
    {
        Loc o;
        int s = locate(layer, slot, &o);
        if (s) return s;
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "get_weight");
        if (o.vec) {
            NC_CHECK_ARG(n_bytes == (size_t)o.n * 2, "get_weight: %zu bytes for %d fp16 values", n_bytes, o.n);
            e = hipMemcpy(ref, o.vec, n_bytes, hipMemcpyDeviceToHost);
            return e == hipSuccess ? NC_OK : hip_fail(e, "get_weight");
        }
        const int dt = o.mat->dtype;
        const size_t want = dt == NC_F16 ? (size_t)o.rows * o.cols * 2
                                         : (size_t)o.rows * (o.cols / 32) * (dt == NC_Q8 ? 34 : 18);
        NC_CHECK_ARG(n_bytes == want, "get_weight: buffer %zu bytes, expected %zu", n_bytes, want);
        uint8_t* out = static_cast<uint8_t*>(ref);
        if (dt == NC_F16) {
            const int npad = (o.mat->rows + 7) & ~7, G = o.cols / 64;
            std::vector<uint16_t> run((size_t)o.rows * 64);
            uint16_t* dst = reinterpret_cast<uint16_t*>(out);
            for (int g = 0; g < G; g++) {
                e = hipMemcpy(run.data(), (uint16_t*)o.mat->data + ((size_t)g * npad + o.row_off) * 64, run.size() * 2,
                              hipMemcpyDeviceToHost);
                if (e != hipSuccess) return hip_fail(e, "get_weight");
                for (int r = 0; r < o.rows; r++)
                    for (int m = 0; m < 8; m++)
                        for (int j = 0; j < 8; j++) dst[(size_t)r * o.cols + 64 * g + 8 * m + j] = run[((size_t)r * 8 + j) * 8 + m];
            }
            return NC_OK;
        }
        size_t cb, db;
        if ((s = nc_weight_bytes(dt, o.rows, o.cols, &cb, &db))) return s;
        std::vector<uint8_t> codes(cb);
        std::vector<uint16_t> deltas(db / 2);
        e = hipMemcpy(codes.data(), (uint8_t*)o.mat->data + code_off(o.mat, o.row_off), cb, hipMemcpyDeviceToHost);
        if (e == hipSuccess)
            e = hipMemcpy(deltas.data(), (uint16_t*)o.mat->deltas + (size_t)o.row_off * (o.cols / 32), db,
                          hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(e, "get_weight");
        const size_t nblk = db / 2;
        for (size_t b = 0; b < nblk; b++) {
            if (dt == NC_Q8) {
                uint8_t* blk = out + b * 34;
                std::memcpy(blk, &deltas[b], 2);
                for (int el = 0; el < 32; el++) {
                    const int k = (el & 7) >> 1, pos = (el & 1) + (((el & 15) >> 3) << 1);
                    blk[2 + el] = codes[b * 32 + (2 * k + (el >> 4)) * 4 + pos];
                }
            } else {
                uint8_t* blk = out + b * 18;
                std::memcpy(blk, &deltas[b], 2);
                for (int j = 0; j < 16; j++) {
                    const int k = (j & 7) >> 1, pos = (j & 1) + ((j >> 3) << 1);
                    blk[2 + j] = codes[b * 16 + k * 4 + pos];
                }
            }
        }
        return NC_OK;
    }

    // ------------------------------------------------------------ forward --

    int norm_kind() const { return cfg.arch == NC_ARCH_ZEPHYR ? kNormLayer : kNormRms; }
    float branch_scale() const
    {
        // MiniCPMConfig::scale_depth / std::sqrt(n_layers) with the reference's
        // constants (minicpm/minicpm.h:14,19; minicpm/minicpm.cpp:57)
        return cfg.arch == NC_ARCH_MINICPM ? (float)((double)1.4f / std::sqrt(40.0)) : 1.0f;
    }

    // Model::logits for rows [sp, n): tokens already on the device.  The
    // last row's logits land in `logits`.  With dpos (graph capture of a
    // decode step) the single row's position is read on the device instead
    // and sp / n are unused.
    int forward(int sp, int n, int* dpos = nullptr)
    {
        const int R = dpos ? 1 : n - sp;
        if (R == 1 && fused) return forward_fused(sp, dpos);
        int s;
        if (R >= kGemmMinRows && (s = refresh_chunks())) return s;
        const int pd = pitch(d);
        const size_t off = dpos ? 0 : (size_t)sp * pd;  // host-side offset of position-indexed rows
        const bool minicpm = cfg.arch == NC_ARCH_MINICPM;
        const float bs = branch_scale();
        // embedding (+ MiniCPM's x12, minicpm.cpp:96)
        if ((s = embed_launch(&emb, dpos ? tokens : tokens + sp, x0 + off, pd, adt, R, minicpm ? 12.0f : 1.0f, st,
                              dpos)))
            return s;
        const bool lnf = ln_fused(R);
        // first attention norm on the embeddings
        if (!lnf && (s = norm_launch(norm_kind(), adt, false, x0 + off, pd, nullptr, 0, 1.0f, nullptr, 0,
                                     L[0].attn_norm, L[0].attn_norm_b, xn, pd, d, d, R, 1.0f, st, dpos)))
            return s;
        const uint8_t* xin = x0;
        for (int l = 0; l < cfg.n_layers; l++) {
            Layer& y = L[l];
            const int pq = pitch(y.qd), pkv = pitch(y.kvd), pf = pitch(y.f);
            const int nqkv = y.qd + 2 * y.kvd;
            if (lnf) {
                // this layer's attention norm; from the second layer on after
                // the previous layer's residual add (out = h + mlp)
                const bool first = l == 0;
                if ((s = mv_ln(first ? x0 + off : L[l - 1].res1 + off, first ? nullptr : down_raw,
                               first ? nullptr : L[l - 1].res2 + off, y.attn_norm, y.attn_norm_b, &y.qkv, qkv_raw,
                               nullptr, false, NC_PROF_QKV, dpos)))
                    return s;
            } else if ((s = mv(xn, pd, R, &y.qkv, qkv_raw, nqkv, NC_PROF_QKV, &y.cqkv))) {
                return s;
            }
            if (R == 1 && adt == NC_F16 && attn_decode_supported(y.hq, y.hkv, cfg.max_ctx)) {
                // fp16 decode row: q/k/v post-processing and attention in one launch
                if ((s = attn_decode_f16_launch(qkv_raw, y.hq, y.hkv, y.bq, y.bk, y.bv, y.qn, y.kn, rope, d_half, sp,
                                                dpos, y.kc, y.vc, pkv, attn, cfg.max_ctx, st)))
                    return s;
            } else {
                if ((s = qkv_post_launch(adt, qkv_raw, nqkv, y.hq, y.hkv, y.bq, y.bk, y.bv, y.qn, y.kn, rope, d_half,
                                         sp, R, q_act, pq, y.kc, pkv, y.vc, pkv, st, dpos)))
                    return s;
                if ((s = attn_launch(adt, q_act, pq, y.kc, pkv, y.vc, pkv, attn, pq, y.hq, y.hkv, sp, n, st, dpos,
                                     cfg.max_ctx)))
                    return s;
            }
            if ((s = mv(attn, pq, R, &y.o, o_raw, d, NC_PROF_O, &y.co))) return s;
            // h = x + attn (MiniCPM: attn scaled first), then the MLP norm and gate|up
            if (lnf) {
                if ((s = mv_ln(xin + off, o_raw, y.res1 + off, y.mlp_norm, y.mlp_norm_b, &y.gu, nullptr, m_act, true,
                               NC_PROF_GATE_UP, dpos)))
                    return s;
            } else {
                if ((s = norm_launch(norm_kind(), adt, true, xin + off, pd, o_raw, d, bs, y.res1 + off, pd,
                                     y.mlp_norm, y.mlp_norm_b, xn, pd, d, d, R, 1.0f, st, dpos)))
                    return s;
                if (R == 1 && adt == NC_F16 && matvec_f16_glu_supported(&y.gu)) {
                    if ((s = mv_glu(xn, &y.gu, m_act))) return s;
                } else {
                    if ((s = mv(xn, pd, R, &y.gu, gu_raw, 2 * y.f, NC_PROF_GATE_UP, &y.cgu))) return s;
                    if ((s = silu_mul_launch(adt, gu_raw, 2 * y.f, y.f, m_act, pf, R, st))) return s;
                }
            }
            if ((s = mv(m_act, pf, R, &y.down, down_raw, d, NC_PROF_DOWN, &y.cdown))) return s;
            // out = h + mlp, then the next layer's attention norm (or the final norm)
            const bool last = l + 1 == cfg.n_layers;
            const uint16_t* nw = last ? norm_w : L[l + 1].attn_norm;
            const uint16_t* nb = last ? norm_b : L[l + 1].attn_norm_b;
            const float post = last && minicpm ? 1.0f / 9 : 1.0f;  // minicpm.cpp:104-105
            // (fused: the next layer's q|k|v launch does this add and norm)
            if ((!lnf || last) && (s = norm_launch(norm_kind(), adt, true, y.res1 + off, pd, down_raw, d, bs,
                                                   y.res2 + off, pd, nw, nb, xn, pd, d, d, R, post, st, dpos)))
                return s;
            xin = y.res2;
        }
        // lm head on the last row only, fp32 out (gten/modules.cpp:48-59,111-122)
        const nc_tensor* head = tied() ? &emb : &lm;
        return mv(xn + (size_t)(R - 1) * pd, pd, 1, head, logits, cfg.n_vocab, NC_PROF_LM_HEAD);
    }

    // The fused kernels' norm prologues: the first layer's (a stored row) and
    // the others' (a residual add first).
    int pro_first() const { return norm_kind() == kNormLayer ? PRO_LN : PRO_RMS; }
    int pro_res_add() const { return norm_kind() == kNormLayer ? PRO_RES_LN : PRO_RES_RMS; }

    bool fused_supported() const
    {
        if (adt != NC_Q8) return false;
        const int wt = cfg.wdtype, pr = pro_res_add();
        for (const Layer& y : L)
            if (!decode_matvec_supported(wt, d, y.qd + 2 * y.kvd, pr, EPI_RAW) ||
                !decode_matvec_supported(wt, d, y.qd + 2 * y.kvd, pro_first(), EPI_RAW) ||
                !decode_matvec_supported(wt, y.qd, d, PRO_X, EPI_RAW) ||
                !decode_matvec_supported(wt, d, 2 * y.f, pr, EPI_SWIGLU) ||
                !decode_matvec_supported(wt, y.f, d, PRO_X, EPI_RAW))
                return false;
        return decode_matvec_supported(wt, d, cfg.n_vocab, pr, EPI_ARGMAX);
    }

    // Algorithmic HBM bytes of one fused launch: weights once, the prologue
    // inputs, the residual row written and the fp32 outputs.
    static double fused_bytes(const nc_tensor* w, int pro, int epi)
    {
        const double N = w->rows, K = w->cols, row = (K / 32) * 34.0;
        double b = N * (K / 32) * (w->dtype == NC_Q8 ? 34.0 : 18.0);
        b += epi == EPI_SWIGLU ? (N / 64) * 34.0 : 4.0 * N;
        // the input row (two with the residual add, and its fp32 addend),
        // the norm gains (and layer_norm's biases)
        if (pro == PRO_X) b += row;
        if (pro == PRO_RMS) b += row + 2.0 * K;
        if (pro == PRO_RES_RMS) b += 2.0 * row + 4.0 * K + 2.0 * K;
        if (pro == PRO_LN) b += row + 4.0 * K;
        if (pro == PRO_RES_LN) b += 2.0 * row + 4.0 * K + 4.0 * K;
        return b;
    }

    int dmv(DmvArgs a, const nc_tensor* w, int pro, int epi, int role)
    {
        a.wq = (const uint32_t*)w->data;
        a.wd = (const uint16_t*)w->deltas;
        a.N = w->rows;
        a.nb = w->cols / 32;
        const bool timed = prof.on && prof.used + 2 <= prof.ev.size();
        int s = timed ? decode_matvec(a, w->dtype, pro, epi, st, prof.ev[prof.used], prof.ev[prof.used + 1])
                      : decode_matvec(a, w->dtype, pro, epi, st);
        if (s) return s;
        if (timed) {
            prof.used += 2;
            prof.bytes.push_back(fused_bytes(w, pro, epi));
            prof.kind.push_back(role | NC_PROF_FUSED);
        }
        return NC_OK;
    }

    // One decode step (row `pos`, or *dpos under graph replay) with the fused
    // kernels.  Each matvec builds its own input row: layer l's qkv takes
    // the previous layer's MLP residual add and the attention norm, o takes
    // the attention output, gate|up the attention residual add and the MLP
    // norm (and ends with SwiGLU), down the SwiGLU row; the lm head takes the last residual
    // add and the final norm and writes the greedy token to tokens[pos + 1]
    // (advancing *dpos).  Residual rows are stored where forward() stores
    // them (res1 / res2 at the position), with the same requantization
    // points.
    int forward_fused(int pos, int* dpos)
    {
        const int pd = pitch(d);
        const bool minicpm = cfg.arch == NC_ARCH_MINICPM;
        const float bs = branch_scale();
        int s;
        // Under graph replay (dpos) the previous step's lm head has stored
        // this step's embedding row (cur_x0) and RoPE row (cur_rope); a
        // direct step embeds its token first.
        if (!dpos && (s = embed_launch(&emb, tokens + pos, x0 + (size_t)pos * pd, pd, adt, 1, minicpm ? 12.0f : 1.0f,
                                       st, nullptr, cur_x0)))
            return s;
        DmvArgs base;
        base.pos = pos;
        base.dpos = dpos;
        base.res_pitch = pd;
        base.bscale = bs;
        const int pr = pro_res_add();
        for (int l = 0; l < cfg.n_layers; l++) {
            Layer& y = L[l];
            const int pkv = pitch(y.kvd);
            DmvArgs a = base;
            a.norm_w = y.attn_norm;
            a.norm_b = y.attn_norm_b;
            a.raw = qkv_raw;
            if (l == 0) {
                a.x = cur_x0;
                a.x_pitch = 0;
                if ((s = dmv(a, &y.qkv, pro_first(), EPI_RAW, NC_PROF_QKV))) return s;
            } else {
                a.res_in = L[l - 1].res1;
                a.res_cur = cur1;
                a.raw_in = down_raw;
                a.res_out = L[l - 1].res2;
                a.res_cur_out = cur2;
                if ((s = dmv(a, &y.qkv, pr, EPI_RAW, NC_PROF_QKV))) return s;
            }
            if ((s = attn_decode_launch(qkv_raw, y.hq, y.hkv, y.bq, y.bk, y.bv, y.qn, y.kn, rope, d_half, pos, dpos,
                                        y.kc, y.vc, pkv, attn, cfg.max_ctx, st, dpos ? cur_rope : nullptr)))
                return s;
            a = base;
            a.x = attn;
            a.raw = o_raw;
            if ((s = dmv(a, &y.o, PRO_X, EPI_RAW, NC_PROF_O))) return s;
            a = base;
            a.res_in = l == 0 ? x0 : L[l - 1].res2;
            a.res_cur = l == 0 ? cur_x0 : cur2;
            a.raw_in = o_raw;
            a.res_out = y.res1;
            a.res_cur_out = cur1;
            a.norm_w = y.mlp_norm;
            a.norm_b = y.mlp_norm_b;
            a.m_out = m_act;
            if ((s = dmv(a, &y.gu, pr, EPI_SWIGLU, NC_PROF_GATE_UP))) return s;
            a = base;
            a.x = m_act;
            a.raw = down_raw;
            if ((s = dmv(a, &y.down, PRO_X, EPI_RAW, NC_PROF_DOWN))) return s;
        }
        DmvArgs a = base;
        a.res_in = L[cfg.n_layers - 1].res1;
        a.res_cur = cur1;
        a.raw_in = down_raw;
        a.res_out = L[cfg.n_layers - 1].res2;
        a.norm_w = norm_w;
        a.norm_b = norm_b;
        a.post_scale = minicpm ? 1.0f / 9 : 1.0f;  // minicpm.cpp:104-105
        a.raw = logits;
        // the head-layout copy of the lm head when there is one
        const nc_tensor* head = hl.data ? &hl : (tied() ? &emb : &lm);
        a.head = hl.data ? 1 : 0;
        // a sampling step: logits only, the sampler picks the token
        if (sample_head) return dmv(a, head, pr, EPI_RAW, NC_PROF_LM_HEAD);
        a.tokens = tokens;
        a.pos_out = dpos;
        a.amax = am_scratch;
        // the next step's embedding and RoPE rows, from the greedy token (the
        // embedding rows in the embedding's own layout)
        if (dpos) next_input_fields(&a, dpos);
        return dmv(a, head, pr, EPI_ARGMAX, NC_PROF_LM_HEAD);
    }

    // The fields of the next step's embedding and RoPE rows (the greedy
    // lm head's epilogue, or k_next_inputs after a sampler).
    void next_input_fields(DmvArgs* a, int* dpos)
    {
        a->nb = d / 32;
        a->tokens = tokens;
        a->pos_out = dpos;
        a->emb_codes = (const uint32_t*)emb.data;
        a->emb_deltas = (const uint16_t*)emb.deltas;
        a->emb_scale = cfg.arch == NC_ARCH_MINICPM ? 12.0f : 1.0f;
        a->emb_cur = cur_x0;
        a->emb_rows = x0;
        a->emb_pitch = pitch(d);
        a->max_ctx = cfg.max_ctx;
        a->rope_table = rope;
        a->rope_cur = cur_rope;
        a->rope_half = d_half;
    }

    // One decode step as a HIP graph: forward at the device-held position,
    // then the greedy token written behind it and the position advanced, so
    // consecutive replays decode consecutive tokens with no host work.
    hipGraphExec_t step_graph = nullptr;
    int* step_pos = nullptr;  // device copy of the decode position

    int capture_step_graph()
    {
        int s;
        if (!step_pos && (s = alloc_t(&step_pos, 16))) return s;
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "capture: sync");
        if ((e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal)) != hipSuccess)
            return hip_fail(e, "hipStreamBeginCapture");
        const bool was_on = prof.on;
        prof.on = false;
        s = forward(0, 0, step_pos);
        if (!s && !fused) s = argmax_advance_launch(logits, cfg.n_vocab, tokens, step_pos, am_scratch, st);
        prof.on = was_on;
        hipGraph_t g = nullptr;
        e = hipStreamEndCapture(st, &g);
        if (s) {
            if (g) (void)hipGraphDestroy(g);
            return s;
        }
        if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
        e = hipGraphInstantiate(&step_graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        return e == hipSuccess ? NC_OK : hip_fail(e, "hipGraphInstantiate");
    }

    int logits_call(const int32_t* toks, int n, int sp, float* out)
    {
        NC_CHECK_ARG(toks && out && n > 0 && n <= cfg.max_ctx && sp >= 0 && sp < n,
                     "logits: %d tokens from %d with max_ctx %d", n, sp, cfg.max_ctx);
        NC_CHECK_ARG(sp == 0 || sp <= n_cur, "logits: start_pos %d beyond the %d cached rows", sp, n_cur);
        topk_on = false;
        Drain drain{st};
        int s = upload(tokens, toks, (size_t)n * 4, "token upload");
        if (s || (s = forward(sp, n))) return s;
        n_cur = n;
        hipError_t e = hipMemcpyAsync(out, logits, (size_t)cfg.n_vocab * 4, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return e == hipSuccess ? NC_OK : hip_fail(e, "logits download");
    }

    int prefill(const int32_t* prompt, int np)
    {
        NC_CHECK_ARG(prompt && np > 0 && np < cfg.max_ctx + 1, "prefill: %d prompt tokens, max_ctx %d", np, cfg.max_ctx);
        topk_on = false;
        int s = upload(tokens, prompt, (size_t)np * 4, "token upload");
        if (s || (s = forward(0, np))) return s;
        if (s) return s;
        if ((s = argmax_launch(logits, cfg.n_vocab, tokens + np, st))) return s;
        n_cur = np;
        n_prompt = np;
        return NC_OK;
    }

    // n_steps more greedy steps; the pending token sits at tokens[n_cur].
    // Steps replay the captured step graph; while matvec profiling is on they
    // are launched directly so each matvec can be bracketed by events.
    bool use_graph = true;

    int decode(int n_steps)
    {
        NC_CHECK_ARG(n_cur > 0, "decode: no prefill");
        NC_CHECK_ARG(n_cur + n_steps <= cfg.max_ctx, "decode: %d + %d steps exceed max_ctx %d", n_cur, n_steps,
                     cfg.max_ctx);
        if (n_steps <= 0) return NC_OK;
        int s;
        if (use_graph && !prof.on) {
            if (!step_graph && (s = capture_step_graph())) return s;
            const int pos = n_cur;
            if ((s = upload(step_pos, &pos, 4, "decode: position upload"))) return s;
            hipError_t e = hipSuccess;
            if (fused) {
                // the first replayed step's inputs (later steps' come from the
                // lm head before them): its token's embedding and RoPE row
                if ((s = embed_launch(&emb, tokens + pos, x0 + (size_t)pos * pitch(d), pitch(d), adt, 1,
                                      cfg.arch == NC_ARCH_MINICPM ? 12.0f : 1.0f, st, nullptr, cur_x0)))
                    return s;
                if (d_half > 0 && (e = hipMemcpyAsync(cur_rope, rope + (size_t)pos * d_half * 2, (size_t)d_half * 8,
                                                      hipMemcpyDeviceToDevice, st)) != hipSuccess)
                    return hip_fail(e, "decode: rope row");
            }
            for (int i = 0; i < n_steps; i++)
                if ((e = hipGraphLaunch(step_graph, st)) != hipSuccess) return hip_fail(e, "hipGraphLaunch");
            n_cur += n_steps;
            return NC_OK;
        }
        for (int i = 0; i < n_steps; i++) {
            const int n = n_cur + 1;
            if ((s = forward(n - 1, n))) return s;
            if (!fused && (s = argmax_launch(logits, cfg.n_vocab, tokens + n, st))) return s;
            n_cur = n;
        }
        return NC_OK;
    }

    // One sampling step after the logits of position pos: the sampler writes
    // tokens[pos + 1] (pos from the device when dpos is given, which it then
    // advances) and, for the fused step, the next step's input rows.
    int sample_after(float temp, int k, int* dpos, int pos, const double* dset = nullptr)
    {
        int s = sample_topk_launch(logits, cfg.n_vocab, temp, k, rng, tokens, dpos, pos, nullptr, st, dset);
        if (s || !fused || !dpos) return s;
        DmvArgs a;
        next_input_fields(&a, dpos);
        return next_inputs_launch(a, cfg.wdtype, st);
    }

    // A decode step that samples instead of taking the greedy token, as a
    // HIP graph; the sampler reads its setting from sample_set.
    int capture_sample_graph()
    {
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "capture: sync");
        if ((e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal)) != hipSuccess)
            return hip_fail(e, "hipStreamBeginCapture");
        const bool was_on = prof.on;
        prof.on = false;
        sample_head = true;
        int s = forward(0, 0, step_pos);
        sample_head = false;
        if (!s) s = sample_after(0.0f, 0, step_pos, 0, sample_set);
        prof.on = was_on;
        hipGraph_t g = nullptr;
        e = hipStreamEndCapture(st, &g);
        if (s) {
            if (g) (void)hipGraphDestroy(g);
            return s;
        }
        if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
        e = hipGraphInstantiate(&sample_graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        return e == hipSuccess ? NC_OK : hip_fail(e, "hipGraphInstantiate");
    }

    // topk_sample (gten/sampler.cpp:63-143) with std::mt19937(seed): the
    // prompt's logits, then n_gen sampled tokens, each step's logits on the
    // device.  top_k and temp are clamped as the reference clamps them.
    int generate_topk(const int32_t* prompt, int np, int n_gen, float temp, int top_k, uint32_t seed)
    {
        NC_CHECK_ARG(prompt && np > 0 && n_gen > 0 && np + n_gen - 1 <= cfg.max_ctx,
                     "generate_topk: %d prompt + %d tokens, max_ctx %d", np, n_gen, cfg.max_ctx);
        int s = topk_begin(prompt, np, temp, top_k, seed);
        return s ? s : topk_steps(n_gen - 1);
    }

    // The sampled loop in parts: the prompt and its sampled token, then
    // more sampled steps (each reading the setting and generator state the
    // first part left on the device).
    bool topk_on = false, topk_graph = false;
    float topk_t = 0.0f;
    int topk_k = 0;

    int topk_begin(const int32_t* prompt, int np, float temp, int top_k, uint32_t seed)
    {
        const int k = 1000 < top_k ? 1000 : top_k;
        const float t = 2.0f < temp ? 2.0f : temp;
        topk_on = false;
        NC_CHECK_ARG(prompt && np > 0 && np <= cfg.max_ctx, "generate_topk: %d prompt tokens, max_ctx %d", np,
                     cfg.max_ctx);
        NC_CHECK_ARG(k >= 1 && k <= cfg.n_vocab && t > 0.0f, "generate_topk: top_k %d, temperature %g", top_k,
                     (double)temp);
        int s;
        if (!rng && (s = alloc_t(&rng, 625 * 4))) return s;
        if (!step_pos && (s = alloc_t(&step_pos, 16))) return s;
        if (!sample_set && (s = alloc_t(&sample_set, 16))) return s;
        uint32_t st0[625];
        mt_seed_host(seed, st0);
        const double set[2] = {(double)k, (double)t};
        if ((s = upload(rng, st0, sizeof(st0), "generate_topk: generator upload")) ||
            (s = upload(sample_set, set, sizeof(set), "generate_topk: setting upload")) ||
            (s = upload(tokens, prompt, (size_t)np * 4, "generate_topk: token upload")))
            return s;
        if ((s = forward(0, np))) return s;
        n_cur = np;
        n_prompt = np;
        const bool graph = use_graph && !prof.on;
        const int first = np - 1;
        if (graph && (s = upload(step_pos, &first, 4, "generate_topk: position upload"))) return s;
        if ((s = sample_after(t, k, graph ? step_pos : nullptr, first))) return s;
        topk_on = true;
        topk_graph = graph;
        topk_t = t;
        topk_k = k;
        return NC_OK;
    }

    int topk_steps(int n_steps)
    {
        NC_CHECK_ARG(topk_on, "sample_steps: no sampled prompt");
        NC_CHECK_ARG(n_steps >= 0 && n_cur + n_steps <= cfg.max_ctx, "sample_steps: %d + %d steps exceed max_ctx %d",
                     n_cur, n_steps, cfg.max_ctx);
        int s;
        hipError_t e = hipSuccess;
        // the first part chose the graph (device position) or direct path
        if (topk_graph) {
            if (!sample_graph && (s = capture_sample_graph())) return s;
            for (int i = 0; i < n_steps; i++)
                if ((e = hipGraphLaunch(sample_graph, st)) != hipSuccess) return hip_fail(e, "hipGraphLaunch");
            n_cur += n_steps;
            return NC_OK;
        }
        for (int i = 0; i < n_steps; i++) {
            const int n = n_cur + 1;
            sample_head = true;
            s = forward(n - 1, n);
            sample_head = false;
            if (s || (s = sample_after(topk_t, topk_k, nullptr, n - 1))) return s;
            n_cur = n;
        }
        return NC_OK;
    }

    // Generated tokens so far: tokens[n_prompt + 1 .. n_cur + 1).
    int fetch_generated(int32_t* out, int max_out, int* n_out)
    {
        const int cnt = std::min(max_out, n_cur + 1 - n_prompt);
        hipError_t e = hipMemcpyAsync(out, tokens + n_prompt, (size_t)cnt * 4, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return hip_fail(e, "token download");
        int k = 0;
        while (k < cnt && out[k] != cfg.eos) k++;  // greedy_sample stops at eos
        *n_out = k;
        return NC_OK;
    }

    int layer_out(int layer, int row, void* ref)
    {
        NC_CHECK_ARG(layer >= 0 && layer < cfg.n_layers && row >= 0 && row < cfg.max_ctx, "layer_out: %d/%d", layer,
                     row);
        const int pd = pitch(d);
        std::vector<uint8_t> buf(pd);
        hipError_t e = hipStreamSynchronize(st);
        if (e == hipSuccess) e = hipMemcpy(buf.data(), L[layer].res2 + (size_t)row * pd, pd, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(e, "layer_out");
        return nc_act_to_reference(buf.data(), ref, adt, 1, d);
    }
};

}  // namespace nc

using nc::Decoder;

extern "C" {

int nc_model_create(const nc_model_config* cfg, void** model)
{
    NC_CHECK_ARG(cfg && model, "model_create: null argument");
    *model = nullptr;
    auto* m = new Decoder();
    int s = m->create(cfg);
    if (s) {
        delete m;
        return s;
    }
    *model = m;
    return NC_OK;
}

int nc_model_free(void* model)
{
    delete static_cast<Decoder*>(model);
    return NC_OK;
}

int nc_model_init_synthetic(void* model, uint64_t seed)
{
    NC_CHECK_ARG(model, "model: null");
    return static_cast<Decoder*>(model)->init_synthetic(seed);
}

int nc_model_set_weight(void* model, int layer, int slot, const void* ref_bytes, size_t n_bytes)
{
    NC_CHECK_ARG(model && ref_bytes, "model: null");
    return static_cast<Decoder*>(model)->set_weight(layer, slot, ref_bytes, n_bytes);
}

int nc_model_load_gten(void* model, const char* path)
{
    NC_CHECK_ARG(model && path, "load_gten: null argument");
    return static_cast<Decoder*>(model)->load_gten(path);
}

int nc_model_get_weight(void* model, int layer, int slot, void* ref_bytes, size_t n_bytes)
{
    NC_CHECK_ARG(model && ref_bytes, "model: null");
    return static_cast<Decoder*>(model)->get_weight(layer, slot, ref_bytes, n_bytes);
}

int nc_model_logits(void* model, const int32_t* tokens, int n_tokens, int start_pos, float* logits)
{
    NC_CHECK_ARG(model, "model: null");
    return static_cast<Decoder*>(model)->logits_call(tokens, n_tokens, start_pos, logits);
}

int nc_model_layer_out(void* model, int layer, int row, void* ref_bytes)
{
    NC_CHECK_ARG(model && ref_bytes, "model: null");
    return static_cast<Decoder*>(model)->layer_out(layer, row, ref_bytes);
}

int nc_model_prefill(void* model, const int32_t* prompt, int n_prompt)
{
    NC_CHECK_ARG(model, "model: null");
    return static_cast<Decoder*>(model)->prefill(prompt, n_prompt);
}

int nc_model_decode(void* model, int n_steps, int32_t* out)
{
    NC_CHECK_ARG(model, "model: null");
    auto* m = static_cast<Decoder*>(model);
    int s = m->decode(n_steps);
    if (s || !out) return s;
    int n;
    return m->fetch_generated(out, m->n_cur + 1 - m->n_prompt, &n);
}

int nc_model_profile_begin(void* model, int max_launches)
{
    NC_CHECK_ARG(model, "model: null");
    return static_cast<Decoder*>(model)->profile_begin(max_launches);
}

int nc_model_profile_launches(void* model, int cap, float* ms, double* bytes, int* kind, int* n_out)
{
    NC_CHECK_ARG(model && cap >= 0 && ms && bytes && kind && n_out, "profile_launches: null argument");
    return static_cast<Decoder*>(model)->profile_launches(cap, ms, bytes, kind, n_out);
}

int nc_model_profile_end(void* model, int* launches, double* total_ms, double* total_bytes, double* min_ms,
                         double* max_ms)
{
    NC_CHECK_ARG(model && launches && total_ms && total_bytes && min_ms && max_ms, "model: null");
    return static_cast<Decoder*>(model)->profile_end(launches, total_ms, total_bytes, min_ms, max_ms);
}

int nc_model_generate(void* model, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out, int* n_out)
{
    NC_CHECK_ARG(model && out && n_out && n_gen > 0, "model_generate: bad arguments");
    auto* m = static_cast<Decoder*>(model);
    NC_CHECK_ARG(n_prompt + n_gen - 1 <= m->cfg.max_ctx, "model_generate: %d + %d exceeds max_ctx %d", n_prompt, n_gen,
                 m->cfg.max_ctx);
    int s = m->prefill(prompt, n_prompt);
    if (!s) s = m->decode(n_gen - 1);
    if (!s) s = m->fetch_generated(out, n_gen, n_out);
    return s;
}

int nc_model_sample_begin(void* model, const int32_t* prompt, int n_prompt, float temp, int top_k, uint32_t seed)
{
    NC_CHECK_ARG(model, "model: null");
    return static_cast<Decoder*>(model)->topk_begin(prompt, n_prompt, temp, top_k, seed);
}

int nc_model_sample_steps(void* model, int n_steps, int32_t* out)
{
    NC_CHECK_ARG(model, "model: null");
    auto* m = static_cast<Decoder*>(model);
    int s = m->topk_steps(n_steps);
    if (s || !out) return s;
    int n;
    return m->fetch_generated(out, m->n_cur + 1 - m->n_prompt, &n);
}

int nc_model_get_config(void* model, nc_model_config* cfg)
{
    NC_CHECK_ARG(model && cfg, "model_get_config: null");
    *cfg = static_cast<Decoder*>(model)->cfg;
    return NC_OK;
}

int nc_model_generate_topk(void* model, const int32_t* prompt, int n_prompt, int n_gen, float temp, int top_k,
                           uint32_t seed, int32_t* out, int* n_out)
{
    NC_CHECK_ARG(model && out && n_out, "model_generate_topk: bad arguments");
    auto* m = static_cast<Decoder*>(model);
    int s = m->generate_topk(prompt, n_prompt, n_gen, temp, top_k, seed);
    if (!s) s = m->fetch_generated(out, n_gen, n_out);
    return s;
}

}  // extern "C"
