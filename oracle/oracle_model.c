/*
 * oracle_model.c -- the reference's decoder forwards restated on top of the
 * oracle ops (test infrastructure; see oracle.h).
 *
 * Dataflow and requantization points follow tinyllama/tinyllama.cpp:88-138,
 * zephyr/zephyr.cpp:24-76, minicpm/minicpm.cpp:42-110 and
 * openelm/openelm.cpp:33-146 (with the RoPE output buffer typed in the
 * activation dtype, which is what openelm.cpp:22-23 intends for Q8 models).
 * Each module owns a [max_ctx, d] activation buffer like the reference's
 * Linear/RMSNorm/... m_acv (gten/modules.cpp:78-87), so the K and V buffers
 * are the KV cache and rows before start_pos are reused as-is.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    void* w[OR_W_NSLOTS];
    /* activation buffers, [max_ctx, dim] in the activation dtype */
    uint8_t *attn_norm, *q, *k, *v, *qn, *kn, *qr, *kr, *attn, *o, *res1, *mlp_norm, *gate, *up,
        *down, *res2;
} or_layer;

struct or_model {
    or_config cfg;
    int adt;
    void* emb;
    void* norm_w;
    void* norm_b;
    void* lm; /* NULL when the embedding is tied */
    or_layer* L;
    uint8_t *x0, *xf, *scratch;
    float* logits;
};

static int is_tied(const or_config* c) { return c->arch == OR_ARCH_MINICPM || c->arch == OR_ARCH_OPENELM; }

int or_weight_shape(const or_config* c, int layer, int slot, int* rows, int* cols, int* dtype)
{
    const int d = c->n_embd;
    if (layer < 0) {
        switch ((unsigned)slot) {
        case OR_TID_EMB: *rows = c->n_vocab; *cols = d; *dtype = c->wdtype; return 1;
        case OR_TID_NORM: *rows = 1; *cols = d; *dtype = OR_F16; return 1;
        case OR_TID_NORM_B: *rows = 1; *cols = d; *dtype = OR_F16; return c->arch == OR_ARCH_ZEPHYR;
        case OR_TID_LM: *rows = c->n_vocab; *cols = d; *dtype = c->wdtype; return !is_tied(c);
        default: return 0;
        }
    }
    const int qd = c->n_heads[layer] * c->d_head, kvd = c->n_kv_heads[layer] * c->d_head;
    const int f = c->n_ffn[layer];
    *dtype = c->wdtype;
    *rows = 1;
    switch (slot) {
    case OR_W_Q: *rows = qd; *cols = d; return 1;
    case OR_W_K: *rows = kvd; *cols = d; return 1;
    case OR_W_V: *rows = kvd; *cols = d; return 1;
    case OR_W_O: *rows = d; *cols = qd; return 1;
    case OR_W_GATE: *rows = f; *cols = d; return 1;
    case OR_W_UP: *rows = f; *cols = d; return 1;
    case OR_W_DOWN: *rows = d; *cols = f; return 1;
    case OR_W_ATTN_NORM: case OR_W_MLP_NORM: *cols = d; *dtype = OR_F16; return 1;
    case OR_W_ATTN_NORM_B: case OR_W_MLP_NORM_B: *cols = d; *dtype = OR_F16; return c->arch == OR_ARCH_ZEPHYR;
    case OR_W_Q_BIAS: *cols = qd; *dtype = OR_F16; return c->arch == OR_ARCH_ZEPHYR;
    case OR_W_K_BIAS: case OR_W_V_BIAS: *cols = kvd; *dtype = OR_F16; return c->arch == OR_ARCH_ZEPHYR;
    case OR_W_Q_NORM: case OR_W_K_NORM: *cols = c->d_head; *dtype = OR_F16; return c->arch == OR_ARCH_OPENELM;
    default: return 0;
    }
}

static size_t tensor_bytes(int rows, int cols, int dt) { return (size_t)rows * or_row_bytes(dt, cols); }

static uint32_t tensor_id(int layer, int slot) { return layer < 0 ? (uint32_t)slot : (uint32_t)(layer * 32 + slot); }

void or_make_weight(const or_config* c, uint64_t seed, int layer, int slot, void* out)
{
    int rows, cols, dt;
    if (!or_weight_shape(c, layer, slot, &rows, &cols, &dt)) return;
    const int64_t n = (int64_t)rows * cols;
    const int is_gain = (layer >= 0 && (slot == OR_W_ATTN_NORM || slot == OR_W_MLP_NORM || slot == OR_W_Q_NORM ||
                                       slot == OR_W_K_NORM)) ||
                        (layer < 0 && (unsigned)slot == OR_TID_NORM);
    const int is_zero = (layer >= 0 && (slot == OR_W_ATTN_NORM_B || slot == OR_W_MLP_NORM_B)) ||
                        (layer < 0 && (unsigned)slot == OR_TID_NORM_B);
    if (is_gain || is_zero) {
        for (int64_t i = 0; i < n; i++) ((uint16_t*)out)[i] = is_gain ? 0x3C00u : 0u;
        return;
    }
    float* f = (float*)malloc((size_t)n * 4);
    or_gen_normal(seed, tensor_id(layer, slot), 0.02f, n, f);
    if (dt == OR_F16) or_fp32_to_fp16_array(f, (uint16_t*)out, n);
    else if (dt == OR_Q8) or_q8_quantize_weights(f, n / OR_QBLOCK, (uint8_t*)out);
    else if (dt == OR_Q4) or_q4_quantize_weights(f, n / OR_QBLOCK, (uint8_t*)out);
    free(f);
}

static void* alloc_weight(const or_config* c, int layer, int slot)
{
    int rows, cols, dt;
    if (!or_weight_shape(c, layer, slot, &rows, &cols, &dt)) return NULL;
    return calloc(1, tensor_bytes(rows, cols, dt));
}

or_model* or_model_create(const or_config* cfg)
{
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->cfg = *cfg;
    const or_config* c = &m->cfg;
    m->adt = c->wdtype == OR_F16 ? OR_F16 : OR_Q8;
    const int mc = c->max_ctx, d = c->n_embd, adt = m->adt;
    m->emb = alloc_weight(c, -1, OR_TID_EMB);
    m->norm_w = alloc_weight(c, -1, OR_TID_NORM);
    m->norm_b = alloc_weight(c, -1, OR_TID_NORM_B);
    m->lm = alloc_weight(c, -1, OR_TID_LM);
    m->L = (or_layer*)calloc((size_t)c->n_layers, sizeof(or_layer));
#define ACT(cols) ((uint8_t*)calloc(1, tensor_bytes(mc, (cols), adt)))
    for (int l = 0; l < c->n_layers; l++) {
        or_layer* L = &m->L[l];
        for (int s = 0; s < OR_W_NSLOTS; s++) L->w[s] = alloc_weight(c, l, s);
        const int qd = c->n_heads[l] * c->d_head, kvd = c->n_kv_heads[l] * c->d_head, f = c->n_ffn[l];
        L->attn_norm = ACT(d); L->q = ACT(qd); L->k = ACT(kvd); L->v = ACT(kvd);
        if (c->arch == OR_ARCH_OPENELM) { L->qn = ACT(qd); L->kn = ACT(kvd); L->qr = ACT(qd); L->kr = ACT(kvd); }
        L->attn = ACT(qd); L->o = ACT(d); L->res1 = ACT(d); L->mlp_norm = ACT(d);
        L->gate = ACT(f); L->up = ACT(f); L->down = ACT(d); L->res2 = ACT(d);
    }
    m->x0 = ACT(d); m->xf = ACT(d); m->scratch = ACT(d);
#undef ACT
    m->logits = (float*)calloc((size_t)c->n_vocab, 4);
    return m;
}

void or_model_free(or_model* m)
{
    if (!m) return;
    for (int l = 0; l < m->cfg.n_layers; l++) {
        or_layer* L = &m->L[l];
        for (int s = 0; s < OR_W_NSLOTS; s++) free(L->w[s]);
        free(L->attn_norm); free(L->q); free(L->k); free(L->v); free(L->qn); free(L->kn); free(L->qr);
        free(L->kr); free(L->attn); free(L->o); free(L->res1); free(L->mlp_norm); free(L->gate);
        free(L->up); free(L->down); free(L->res2);
    }
    free(m->L); free(m->emb); free(m->norm_w); free(m->norm_b); free(m->lm);
    free(m->x0); free(m->xf); free(m->scratch); free(m->logits);
    free(m);
}

void* or_model_weight(or_model* m, int layer, int slot)
{
    if (layer >= 0) return m->L[layer].w[slot];
    switch ((unsigned)slot) {
    case OR_TID_EMB: return m->emb;
    case OR_TID_NORM: return m->norm_w;
    case OR_TID_NORM_B: return m->norm_b;
    case OR_TID_LM: return m->lm;
    default: return NULL;
    }
}

void or_model_init_synthetic(or_model* m, uint64_t seed)
{
    const or_config* c = &m->cfg;
    const unsigned globals[4] = {OR_TID_EMB, OR_TID_NORM, OR_TID_NORM_B, OR_TID_LM};
    for (int g = 0; g < 4; g++)
        if (or_model_weight(m, -1, (int)globals[g])) or_make_weight(c, seed, -1, (int)globals[g], or_model_weight(m, -1, (int)globals[g]));
    for (int l = 0; l < c->n_layers; l++)
        for (int s = 0; s < OR_W_NSLOTS; s++)
            if (m->L[l].w[s]) or_make_weight(c, seed, l, s, m->L[l].w[s]);
}

static void norm_op(or_model* m, const void* x, void* out, const void* w, const void* b, int sp, int n)
{
    if (m->cfg.arch == OR_ARCH_ZEPHYR)
        or_layer_norm(x, m->adt, (const uint16_t*)w, (const uint16_t*)b, out, m->cfg.n_embd, sp, n);
    else
        or_rms_norm(x, m->adt, (const uint16_t*)w, out, m->cfg.n_embd, sp, n);
}

/* Linear::forward (gten/modules.cpp:89-104): matmul into the Act buffer,
 * then the fp16 bias added in place when present. */
static void linear(or_model* m, const void* x, int K, const void* w, const void* bias, void* out, int N,
                   int sp, int n)
{
    or_matmul(x, m->adt, w, m->cfg.wdtype, out, m->adt, K, N, sp, n, NULL);
    if (bias) or_bias_add(out, m->adt, (const uint16_t*)bias, N, sp, n);
}

static void block_forward(or_model* m, int l, const void* x, int sp, int n)
{
    const or_config* c = &m->cfg;
    or_layer* L = &m->L[l];
    const int d = c->n_embd, adt = m->adt, dh = c->d_head;
    const int hq = c->n_heads[l], hkv = c->n_kv_heads[l], qd = hq * dh, kvd = hkv * dh, f = c->n_ffn[l];
    const int minicpm = c->arch == OR_ARCH_MINICPM;
    /* scale_depth / std::sqrt(n_layers) with MiniCPMConfig's constants
     * (1.4f, 40 layers), evaluated in double and stored as float
     * (minicpm/minicpm.h:14,19; minicpm/minicpm.cpp:57). */
    const float branch_scale = (float)((double)1.4f / sqrt(40.0));

    if (minicpm) memcpy(m->scratch, x, tensor_bytes(n, d, adt)); /* copy_tensor, minicpm.cpp:54 */

    norm_op(m, x, L->attn_norm, L->w[OR_W_ATTN_NORM], L->w[OR_W_ATTN_NORM_B], sp, n);
    linear(m, L->attn_norm, d, L->w[OR_W_Q], L->w[OR_W_Q_BIAS], L->q, qd, sp, n);
    linear(m, L->attn_norm, d, L->w[OR_W_K], L->w[OR_W_K_BIAS], L->k, kvd, sp, n);
    const uint8_t *qa, *ka;
    if (c->arch == OR_ARCH_OPENELM) {
        linear(m, L->attn_norm, d, L->w[OR_W_V], NULL, L->v, kvd, sp, n);
        /* per-head QK RMSNorm (openelm.cpp:44-49), then RoPE into separate buffers */
        or_rms_norm_heads(L->q, adt, (const uint16_t*)L->w[OR_W_Q_NORM], L->qn, hq, dh, sp, n);
        or_rms_norm_heads(L->k, adt, (const uint16_t*)L->w[OR_W_K_NORM], L->kn, hkv, dh, sp, n);
        or_rotary_emb(L->qn, L->qr, adt, qd, dh, c->rope_pct, sp, n);
        or_rotary_emb(L->kn, L->kr, adt, kvd, dh, c->rope_pct, sp, n);
        qa = L->qr; ka = L->kr;
    } else {
        or_rotary_emb(L->q, L->q, adt, qd, dh, c->rope_pct, sp, n);
        or_rotary_emb(L->k, L->k, adt, kvd, dh, c->rope_pct, sp, n);
        linear(m, L->attn_norm, d, L->w[OR_W_V], L->w[OR_W_V_BIAS], L->v, kvd, sp, n);
        qa = L->q; ka = L->k;
    }
    or_qkv_attn(qa, ka, L->v, L->attn, adt, hq, hkv, dh, sp, n);
    linear(m, L->attn, qd, L->w[OR_W_O], NULL, L->o, d, sp, n);
    if (minicpm) {
        or_scale(L->o, adt, branch_scale, d, sp, n);
        or_add(m->scratch, L->o, L->res1, adt, d, sp, n);
        memcpy(m->scratch, L->res1, tensor_bytes(n, d, adt));
    } else {
        or_add(x, L->o, L->res1, adt, d, sp, n);
    }

    norm_op(m, L->res1, L->mlp_norm, L->w[OR_W_MLP_NORM], L->w[OR_W_MLP_NORM_B], sp, n);
    linear(m, L->mlp_norm, d, L->w[OR_W_GATE], NULL, L->gate, f, sp, n);
    linear(m, L->mlp_norm, d, L->w[OR_W_UP], NULL, L->up, f, sp, n);
    or_silu(L->gate, L->gate, adt, f, sp, n);
    or_multiply(L->gate, L->up, L->gate, adt, f, sp, n);
    linear(m, L->gate, f, L->w[OR_W_DOWN], NULL, L->down, d, sp, n);
    if (minicpm) {
        or_scale(L->down, adt, branch_scale, d, sp, n);
        or_add(L->down, m->scratch, L->res2, adt, d, sp, n);
    } else {
        or_add(L->res1, L->down, L->res2, adt, d, sp, n);
    }
}

void or_model_logits(or_model* m, const int32_t* tokens, int n, int sp, float* logits)
{
    const or_config* c = &m->cfg;
    const int d = c->n_embd, adt = m->adt;
    or_token_embed(m->emb, c->wdtype, tokens, m->x0, adt, d, sp, n);
    if (c->arch == OR_ARCH_MINICPM) or_scale(m->x0, adt, 12.0f, d, sp, n); /* minicpm.cpp:96 */
    const uint8_t* x = m->x0;
    for (int l = 0; l < c->n_layers; l++) {
        block_forward(m, l, x, sp, n);
        x = m->L[l].res2;
    }
    norm_op(m, x, m->xf, m->norm_w, m->norm_b, sp, n);
    if (c->arch == OR_ARCH_MINICPM) or_scale(m->xf, adt, 1.0f / 9, d, sp, n); /* minicpm.cpp:104-105 */
    /* lm head on the last row only, fp32 out (gten/modules.cpp:48-59,111-122) */
    const void* head = m->lm ? m->lm : m->emb;
    const uint8_t* last = m->xf + (size_t)(n - 1) * or_row_bytes(adt, d);
    or_matmul(last, adt, head, c->wdtype, m->logits, OR_F32, d, c->n_vocab, 0, 1, NULL);
    memcpy(logits, m->logits, (size_t)c->n_vocab * 4);
}

const void* or_model_layer_out(or_model* m, int layer, int row)
{
    return m->L[layer].res2 + (size_t)row * or_row_bytes(m->adt, m->cfg.n_embd);
}

size_t or_model_act_row_bytes(or_model* m) { return or_row_bytes(m->adt, m->cfg.n_embd); }

/* topk_sample's loop (gten/sampler.cpp:84-134) with a seeded generator. */
int or_generate_topk(or_model* m, const int32_t* prompt, int n_prompt, int n_gen, float temp, int top_k,
                     uint32_t seed, int32_t* out)
{
    uint32_t st[625];
    or_mt_seed(seed, st);
    const int total = n_prompt + n_gen;
    int32_t* toks = (int32_t*)malloc((size_t)total * 4);
    float* lg = (float*)malloc((size_t)m->cfg.n_vocab * 4);
    memcpy(toks, prompt, (size_t)n_prompt * 4);
    int n = n_prompt, produced = 0;
    for (int i = 0; i < n_gen; i++) {
        or_model_logits(m, toks, n, i == 0 ? 0 : n - 1, lg);
        const int t = or_topk_sample(lg, m->cfg.n_vocab, temp, top_k, st, NULL);
        if (t == m->cfg.eos) break;
        out[produced++] = t;
        toks[n++] = t;
    }
    free(toks);
    free(lg);
    return produced;
}

int or_generate_greedy(or_model* m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out)
{
    const int total = n_prompt + n_gen;
    int32_t* toks = (int32_t*)malloc((size_t)total * 4);
    float* lg = (float*)malloc((size_t)m->cfg.n_vocab * 4);
    memcpy(toks, prompt, (size_t)n_prompt * 4);
    int n = n_prompt, produced = 0;
    for (int i = 0; i < n_gen; i++) {
        or_model_logits(m, toks, n, i == 0 ? 0 : n - 1, lg);
        const int t = or_argmax(lg, m->cfg.n_vocab);
        if (t == m->cfg.eos) break;
        out[produced++] = t;
        toks[n++] = t;
    }
    free(toks);
    free(lg);
    return produced;
}
