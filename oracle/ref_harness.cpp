// ref_harness.cpp -- C entry points around the reference's own gten code.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile together with the
// reference's sources where they lie (src/gten/{ops,quants,tensor,modules,
// utils}.cpp and the model block sources), never copied, into
// oracle/_ref/libgten_ref.so.  It lets the tests run the reference's ops and
// block forwards on the same inputs as the oracle restatement and the HIP
// path.  The reference's nanochat.cpp main (which shells out to a network
// downloader) is not built.
//
// Model tops (embedding -> blocks -> final norm -> lm head) are composed here
// exactly as TinyLLama::logits (tinyllama/tinyllama.cpp:122-138) and its
// siblings do, because those classes hard-code their vocab / layer counts;
// the per-layer blocks are the reference's own classes.  OpenELM's
// SelfAttention_Elm types its RoPE output buffer fp16 (openelm.cpp:22-23,
// gten/modules.cpp:247-249), which makes Q8 models abort in qkv_attn
// (gten/ops.cpp:1216); the OpenELM block is therefore composed here from the
// reference's modules and ops with that buffer typed in the activation dtype.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <iostream>
#include <memory>
#include <random>
#include <sstream>
#include <utility>
#include <vector>

#include "gten/gten.h"
#include "gten/sampler.h"
#include "gten/tokenizer.h"
#include "minicpm/minicpm.h"
#include "tinyllama/tinyllama.h"
#include "zephyr/zephyr.h"

extern "C" {
#include "oracle.h"
}

using namespace gten;

static Dtype to_dtype(int dt)
{
    switch (dt) {
    case OR_I32: return kInt32;
    case OR_F16: return kFloat16;
    case OR_F32: return kFloat32;
    case OR_Q8: return kQint8;
    default: return kQint4;
    }
}

static Tensor view2d(const void* p, int rows, int cols, int dt) { return Tensor(p, {rows, cols}, to_dtype(dt)); }
static Tensor view1d(const void* p, int n, int dt) { return Tensor(p, {n}, to_dtype(dt)); }

extern "C" {

float ref_fp16_to_fp32(uint16_t h) { return gten::fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return gten::fp32_to_fp16(f); }

void ref_q8_quantize_row(const float* x, uint8_t* blocks, int n)
{
    ops::q8_quantize_row(x, reinterpret_cast<Q8Block*>(blocks), n);
}

void ref_q8_dequantize_row(const uint8_t* blocks, float* out, int n)
{
    ops::q8_dequantize_row(reinterpret_cast<const Q8Block*>(blocks), out, n);
}

void ref_q4_dequantize_row(const uint8_t* blocks, float* out, int n)
{
    ops::q4_dequantize_row(reinterpret_cast<const Q4Block*>(blocks), out, n);
}

void ref_matmul(const void* x, int xdt, const void* w, int wdt, void* out, int odt, int K, int N, int start,
                int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, K, xdt), tw = view2d(w, N, K, wdt), to = view2d(out, n_ctx, N, odt);
    ops::matmul_2d(tx, tw, to, start);
}

void ref_rms_norm(const void* x, int dt, const uint16_t* w, void* out, int d, int start, int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, d, dt), tw = view1d(w, d, OR_F16), to = view2d(out, n_ctx, d, dt);
    ops::rms_norm(tx, tw, to, start);
}

void ref_rms_norm_heads(const void* x, int dt, const uint16_t* w, void* out, int n_heads, int d_head, int start,
                        int n_ctx)
{
    Tensor tx = Tensor(x, {n_ctx, n_heads, d_head}, to_dtype(dt));
    Tensor tw = view1d(w, d_head, OR_F16), to = view2d(out, n_ctx, n_heads * d_head, dt);
    ops::rms_norm(tx, tw, to, start);
}

void ref_layer_norm(const void* x, int dt, const uint16_t* w, const uint16_t* b, void* out, int d, int start,
                    int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, d, dt), tw = view1d(w, d, OR_F16), tb = view1d(b, d, OR_F16);
    Tensor to = view2d(out, n_ctx, d, dt);
    ops::layer_norm(tx, tw, tb, to, start);
}

void ref_rotary_emb(void* x, void* out, int dt, int d, int d_head, float pct, int start, int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, d, dt), to = view2d(out, n_ctx, d, dt);
    ops::rotary_emb(tx, to, d_head, pct, start);
}

void ref_silu(const void* x, void* out, int dt, int d, int start, int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, d, dt), to = view2d(out, n_ctx, d, dt);
    ops::silu(tx, to, start);
}

void ref_multiply(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx)
{
    Tensor ta = view2d(a, n_ctx, d, dt), tb = view2d(b, n_ctx, d, dt), to = view2d(out, n_ctx, d, dt);
    ops::multiply(ta, tb, to, start);
}

void ref_add(const void* a, const void* b, void* out, int dt, int d, int start, int n_ctx)
{
    Tensor ta = view2d(a, n_ctx, d, dt), tb = view2d(b, n_ctx, d, dt), to = view2d(out, n_ctx, d, dt);
    ops::add(ta, tb, to, start);
}

void ref_scale(void* x, int dt, float s, int d, int start, int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, d, dt);
    ops::scale(tx, s, start);
}

void ref_bias_add(void* x, int dt, const uint16_t* b, int d, int start, int n_ctx)
{
    Tensor tx = view2d(x, n_ctx, d, dt), tb = view1d(b, d, OR_F16);
    ops::bias_add_inplace(tx, tb, start);
}

// The reference addresses probability rows with element strides used as byte
// offsets (gten/ops.cpp:1033-1034,1083), so max_ctx is chosen large enough
// that no two rows overlap.
void ref_qkv_attn(const void* q, const void* k, const void* v, void* out, int dt, int n_heads, int n_kv_heads,
                  int d_head, int start, int n_ctx)
{
    const int max_ctx = std::max(2 * n_ctx, ((n_ctx + 31) / 32) * 34);
    Tensor tq = view2d(q, n_ctx, n_heads * d_head, dt);
    Tensor tk = view2d(k, n_ctx, n_kv_heads * d_head, dt);
    Tensor tv = view2d(v, n_ctx, n_kv_heads * d_head, dt);
    Tensor qk = Tensor({n_heads, max_ctx, max_ctx}, to_dtype(dt));
    qk.resize({n_heads, n_ctx, n_ctx});
    Tensor to = view2d(out, n_ctx, n_heads * d_head, dt);
    ops::qkv_attn(tq, tk, tv, qk, to, max_ctx, start);
}

void ref_token_embed(const void* table, int wdt, const int32_t* tokens, void* out, int adt, int d, int vocab,
                     int start, int n_ctx)
{
    Tensor tw = view2d(table, vocab, d, wdt), tt = view1d(tokens, n_ctx, OR_I32), to = view2d(out, n_ctx, d, adt);
    ops::token_embed(tw, tt, to, start);
}

}  // extern "C"

// ---------------------------------------------------------------- models ---

namespace {

void fill(const or_config* c, uint64_t seed, int layer, int slot, Tensor& t)
{
    int rows, cols, dt;
    if (!or_weight_shape(c, layer, slot, &rows, &cols, &dt)) return;
    or_make_weight(c, seed, layer, slot, t.data_ptr<void>());
}

// OpenELM block: SelfAttention_Elm::forward + OpenELMBlock::forward
// (openelm/openelm.cpp:33-58,90-108) on the reference's modules and ops.
struct ElmBlock {
    RMSNorm attn_norm;
    Linear q, k, v, o;
    RMSNorm3D q_norm, k_norm;
    Tensor q_rope, k_rope, qk, qkv;
    Residual inp_res;
    RMSNorm mlp_norm;
    Linear gate, up, down;
    SiLU silu;
    Multiply mul;
    Residual attn_res;
    int n_heads, max_ctx;

    ElmBlock(int hq, int kvd, int d, int f, int mc, ModuleDtype dt)
        : attn_norm(d, mc, dt), q(d, hq * 64, mc, dt), k(d, kvd, mc, dt), v(d, kvd, mc, dt), o(hq * 64, d, mc, dt),
          q_norm(d, 64, mc, dt), k_norm(d, 64, mc, dt), q_rope({mc, hq * 64}, dt.adtype),
          k_rope({mc, kvd}, dt.adtype), qk({hq, mc, mc}, dt.adtype), qkv({mc, hq * 64}, dt.adtype),
          inp_res(mc, d, dt.adtype), mlp_norm(d, mc, dt), gate(d, f, mc, dt), up(d, f, mc, dt),
          down(f, d, mc, dt), silu(mc, f, dt.adtype, true), mul(mc, f, dt.adtype, true),
          attn_res(mc, d, dt.adtype), n_heads(hq), max_ctx(mc)
    {
    }

    Tensor attn_forward(const Tensor& inp, int sp)
    {
        Tensor tq = q.forward(inp, sp);
        Tensor tk = k.forward(inp, sp);
        Tensor tv = v.forward(inp, sp);
        const int n_ctx = tq.dimsize(0);
        Tensor qv = tq.view({n_ctx, tq.dimsize(1) / 64, 64});
        tq = q_norm.forward(qv);
        Tensor kv = tk.view({n_ctx, tk.dimsize(1) / 64, 64});
        tk = k_norm.forward(kv);
        q_rope.resize({n_ctx, tq.dimsize(1)});
        ops::rotary_emb(tq, q_rope, 64, 1.0f, sp);
        k_rope.resize({n_ctx, tk.dimsize(1)});
        ops::rotary_emb(tk, k_rope, 64, 1.0f, sp);
        qk.resize({n_heads, n_ctx, n_ctx});
        qkv.resize({n_ctx, q_rope.dimsize(1)});
        ops::qkv_attn(q_rope, k_rope, tv, qk, qkv, max_ctx, sp);
        return o.forward(qkv, sp);
    }

    Tensor forward(Tensor& inp, int sp)
    {
        Tensor h = inp_res.forward(inp, attn_forward(attn_norm.forward(inp, sp), sp), sp);
        const Tensor hn = mlp_norm.forward(h, sp);
        Tensor w1 = gate.forward(hn, sp);
        const Tensor w3 = up.forward(hn, sp);
        Tensor sw1 = silu.forward(w1, sp);
        const Tensor w1w2 = mul.forward(sw1, w3, sp);
        return attn_res.forward(h, down.forward(w1w2, sp), sp);
    }
};

struct RefModel {
    or_config cfg;
    ModuleDtype dtype;
    std::unique_ptr<Embedding> emb;
    std::unique_ptr<TiedEmbedding> tied;
    std::unique_ptr<RMSNorm> rms;
    std::unique_ptr<LayerNorm> ln;
    std::unique_ptr<EmbeddingLinear> lm;
    std::vector<TinyLLamaBlock> llama;
    std::vector<ZephyrBlock> zephyr;
    std::vector<MiniCPMAttentionBlock> minicpm;
    std::vector<std::unique_ptr<ElmBlock>> elm;
    Tensor res_scratch;
    std::vector<Tensor> layer_out;
    size_t act_row_bytes;
};

}  // namespace

extern "C" {

void* ref_model_create(const or_config* c, uint64_t seed)
{
    auto* m = new RefModel();
    m->cfg = *c;
    m->dtype = c->wdtype == OR_F16 ? mFloat16 : (c->wdtype == OR_Q8 ? mQint8 : mQint4);
    const ModuleDtype dt = m->dtype;
    const int mc = c->max_ctx, d = c->n_embd, V = c->n_vocab;
    const ModuleDtype norm_dt = {kFloat16, dt.adtype};
    m->layer_out.resize(c->n_layers);
    m->act_row_bytes = or_row_bytes(c->wdtype == OR_F16 ? OR_F16 : OR_Q8, d);
    switch (c->arch) {
    case OR_ARCH_LLAMA:
        m->emb.reset(new Embedding(V, d, mc, dt));
        m->rms.reset(new RMSNorm(d, mc, norm_dt));
        m->lm.reset(new EmbeddingLinear(d, V, mc, {dt.wdtype, kFloat32}));
        m->llama.reserve(c->n_layers);
        for (int l = 0; l < c->n_layers; l++)
            m->llama.push_back(TinyLLamaBlock(c->n_heads[l], d, c->n_kv_heads[l], c->n_ffn[l], mc, dt));
        break;
    case OR_ARCH_ZEPHYR:
        m->emb.reset(new Embedding(V, d, mc, dt));
        m->ln.reset(new LayerNorm(d, mc, norm_dt));
        m->lm.reset(new EmbeddingLinear(d, V, mc, {dt.wdtype, kFloat32}));
        m->zephyr.reserve(c->n_layers);
        for (int l = 0; l < c->n_layers; l++)
            m->zephyr.push_back(ZephyrBlock(c->n_heads[l], d, c->n_kv_heads[l], c->n_ffn[l], mc, dt, c->rope_pct));
        break;
    case OR_ARCH_MINICPM:
        m->tied.reset(new TiedEmbedding(V, d, mc, dt));
        m->rms.reset(new RMSNorm(d, mc, norm_dt));
        m->res_scratch = Tensor({mc, d}, dt.adtype);
        m->minicpm.reserve(c->n_layers);
        for (int l = 0; l < c->n_layers; l++)
            m->minicpm.push_back(MiniCPMAttentionBlock(c->n_heads[l], d, c->n_kv_heads[l], c->n_ffn[l], mc, dt));
        break;
    default:
        m->tied.reset(new TiedEmbedding(V, d, mc, dt));
        m->rms.reset(new RMSNorm(d, mc, norm_dt));
        for (int l = 0; l < c->n_layers; l++)
            m->elm.emplace_back(new ElmBlock(c->n_heads[l], c->n_kv_heads[l] * 64, d, c->n_ffn[l], mc, dt));
        break;
    }

    // weights, in the generator's tensor numbering
    if (m->emb) fill(c, seed, -1, OR_TID_EMB, m->emb->m_weight);
    if (m->tied) fill(c, seed, -1, OR_TID_EMB, m->tied->m_weight);
    if (m->lm) fill(c, seed, -1, OR_TID_LM, m->lm->m_weight);
    if (m->rms) fill(c, seed, -1, OR_TID_NORM, m->rms->m_weight);
    if (m->ln) { fill(c, seed, -1, OR_TID_NORM, m->ln->m_weight); fill(c, seed, -1, OR_TID_NORM_B, m->ln->m_bias); }
    for (int l = 0; l < c->n_layers; l++) {
        Linear *q, *k, *v, *o, *g, *u, *dn;
        if (c->arch == OR_ARCH_LLAMA) {
            auto& b = m->llama[l];
            q = &b.m_self_attn.m_query; k = &b.m_self_attn.m_key; v = &b.m_self_attn.m_value; o = &b.m_self_attn.m_qkv_proj;
            g = &b.m_mlp_gate_proj; u = &b.m_mlp_up_proj; dn = &b.m_mlp_down_proj;
            fill(c, seed, l, OR_W_ATTN_NORM, b.m_attn_norm.m_weight);
            fill(c, seed, l, OR_W_MLP_NORM, b.m_mlp_norm.m_weight);
        } else if (c->arch == OR_ARCH_ZEPHYR) {
            auto& b = m->zephyr[l];
            q = &b.m_self_attn.m_query; k = &b.m_self_attn.m_key; v = &b.m_self_attn.m_value; o = &b.m_self_attn.m_qkv_proj;
            g = &b.m_mlp_gate_proj; u = &b.m_mlp_up_proj; dn = &b.m_mlp_down_proj;
            fill(c, seed, l, OR_W_ATTN_NORM, b.m_attn_norm.m_weight);
            fill(c, seed, l, OR_W_ATTN_NORM_B, b.m_attn_norm.m_bias);
            fill(c, seed, l, OR_W_MLP_NORM, b.m_mlp_norm.m_weight);
            fill(c, seed, l, OR_W_MLP_NORM_B, b.m_mlp_norm.m_bias);
            fill(c, seed, l, OR_W_Q_BIAS, q->m_bias);
            fill(c, seed, l, OR_W_K_BIAS, k->m_bias);
            fill(c, seed, l, OR_W_V_BIAS, v->m_bias);
        } else if (c->arch == OR_ARCH_MINICPM) {
            auto& b = m->minicpm[l];
            q = &b.m_self_attn.m_query; k = &b.m_self_attn.m_key; v = &b.m_self_attn.m_value; o = &b.m_self_attn.m_qkv_proj;
            g = &b.m_mlp_gate_proj; u = &b.m_mlp_up_proj; dn = &b.m_mlp_down_proj;
            fill(c, seed, l, OR_W_ATTN_NORM, b.m_input_norm.m_weight);
            fill(c, seed, l, OR_W_MLP_NORM, b.m_post_attn_norm.m_weight);
        } else {
            auto& b = *m->elm[l];
            q = &b.q; k = &b.k; v = &b.v; o = &b.o; g = &b.gate; u = &b.up; dn = &b.down;
            fill(c, seed, l, OR_W_ATTN_NORM, b.attn_norm.m_weight);
            fill(c, seed, l, OR_W_MLP_NORM, b.mlp_norm.m_weight);
            fill(c, seed, l, OR_W_Q_NORM, b.q_norm.m_weight);
            fill(c, seed, l, OR_W_K_NORM, b.k_norm.m_weight);
        }
        fill(c, seed, l, OR_W_Q, q->m_weight);
        fill(c, seed, l, OR_W_K, k->m_weight);
        fill(c, seed, l, OR_W_V, v->m_weight);
        fill(c, seed, l, OR_W_O, o->m_weight);
        fill(c, seed, l, OR_W_GATE, g->m_weight);
        fill(c, seed, l, OR_W_UP, u->m_weight);
        fill(c, seed, l, OR_W_DOWN, dn->m_weight);
    }
    return m;
}

void ref_model_free(void* p) { delete static_cast<RefModel*>(p); }

// Model::logits(tokens, start_pos): the last row's fp32 logits into `logits`.
void ref_model_logits(void* p, const int32_t* tokens, int n, int sp, float* logits)
{
    auto* m = static_cast<RefModel*>(p);
    const or_config* c = &m->cfg;
    Tensor toks(tokens, {n}, kInt32);
    Tensor x;
    switch (c->arch) {
    case OR_ARCH_LLAMA:
        x = m->emb->forward(toks, sp);
        for (int l = 0; l < c->n_layers; l++) m->layer_out[l] = x = m->llama[l].forward(x, sp);
        x = m->rms->forward(x, sp);
        x = m->lm->forward(x);
        break;
    case OR_ARCH_ZEPHYR:
        x = m->emb->forward(toks, sp);
        for (int l = 0; l < c->n_layers; l++) m->layer_out[l] = x = m->zephyr[l].forward(x, sp);
        x = m->ln->forward(x, sp);
        x = m->lm->forward(x);
        break;
    case OR_ARCH_MINICPM: {
        x = m->tied->forward_embed(toks, sp);
        ops::scale(x, minicpm_cfg.scale_emb, sp);
        for (int l = 0; l < c->n_layers; l++) m->layer_out[l] = x = m->minicpm[l].forward(x, m->res_scratch, sp);
        x = m->rms->forward(x, sp);
        const float scaler = 1.0f / (minicpm_cfg.n_embd / minicpm_cfg.dim_model_base);
        ops::scale(x, scaler, sp);
        x = m->tied->forward_proj(x);
        break;
    }
    default:
        x = m->tied->forward_embed(toks, sp);
        for (int l = 0; l < c->n_layers; l++) m->layer_out[l] = x = m->elm[l]->forward(x, sp);
        x = m->rms->forward(x, sp);
        x = m->tied->forward_proj(x);
        break;
    }
    std::memcpy(logits, x.data_ptr<float>(), (size_t)c->n_vocab * 4);
}

const void* ref_model_layer_out(void* p, int layer, int row)
{
    auto* m = static_cast<RefModel*>(p);
    return m->layer_out[layer].data_ptr<uint8_t>() + (size_t)row * m->act_row_bytes;
}

// greedy_sample (gten/sampler.cpp:11-60) without the tokenizer.
int ref_generate_greedy(void* p, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out)
{
    auto* m = static_cast<RefModel*>(p);
    std::vector<int32_t> toks(prompt, prompt + n_prompt);
    toks.reserve(n_prompt + n_gen);
    std::vector<float> lg(m->cfg.n_vocab);
    int produced = 0;
    for (int i = 0; i < n_gen; i++) {
        const int n = (int)toks.size();
        ref_model_logits(p, toks.data(), n, i == 0 ? 0 : n - 1, lg.data());
        float mx = -std::numeric_limits<float>::infinity();
        int idx = 0;
        for (int j = 0; j < m->cfg.n_vocab; j++)
            if (lg[j] > mx) { mx = lg[j]; idx = j; }
        if (idx == m->cfg.eos) break;
        out[produced++] = idx;
        toks.push_back(idx);
    }
    return produced;
}

// Model::load_from_ckpt with the reference's record readers
// (gten::read_layer_header / read_into_weight, gten/utils.cpp:29-61) over
// this harness's modules, in each model's file order
// (tinyllama/tinyllama.cpp:131-187, zephyr/zephyr.cpp:79-150,
// minicpm/minicpm.cpp:113-166, openelm/openelm.cpp:201-262).  Returns 0, or
// -1 for a file that does not open or has the wrong magic number (the
// reference asserts on those; a wrong payload size still exits the process
// inside read_into_weight, so callers pass well-formed files only).
int ref_model_load_gten(void* p, const char* path)
{
    auto* m = static_cast<RefModel*>(p);
    std::ifstream f(path, std::ios::binary);
    if (!f) return -1;
    int64_t magic = 0;
    f.read(reinterpret_cast<char*>(&magic), sizeof(magic));
    if (magic != 0x454c49464e455447) return -1;
    const ModuleDtype dt = m->dtype;
    const ModuleDtype norm_dt = {kFloat16, dt.adtype};
    auto rec = [&](Tensor& t, const ModuleDtype& d) {
        read_layer_header(f);
        read_into_weight(f, t, d);
    };
    rec(m->emb ? m->emb->m_weight : m->tied->m_weight, dt);
    const or_config* c = &m->cfg;
    for (int l = 0; l < c->n_layers; l++) {
        if (c->arch == OR_ARCH_LLAMA) {
            auto& b = m->llama[l];
            for (Linear* x : {&b.m_self_attn.m_query, &b.m_self_attn.m_key, &b.m_self_attn.m_value,
                              &b.m_self_attn.m_qkv_proj, &b.m_mlp_gate_proj, &b.m_mlp_up_proj, &b.m_mlp_down_proj})
                rec(x->m_weight, dt);
            rec(b.m_attn_norm.m_weight, norm_dt);
            rec(b.m_mlp_norm.m_weight, norm_dt);
        } else if (c->arch == OR_ARCH_ZEPHYR) {
            auto& b = m->zephyr[l];
            for (Linear* x : {&b.m_self_attn.m_query, &b.m_self_attn.m_key, &b.m_self_attn.m_value}) {
                rec(x->m_weight, dt);
                rec(x->m_bias, norm_dt);
            }
            for (Linear* x : {&b.m_self_attn.m_qkv_proj, &b.m_mlp_gate_proj, &b.m_mlp_up_proj, &b.m_mlp_down_proj})
                rec(x->m_weight, dt);
            rec(b.m_attn_norm.m_weight, norm_dt);
            rec(b.m_attn_norm.m_bias, norm_dt);
            rec(b.m_mlp_norm.m_weight, norm_dt);
            rec(b.m_mlp_norm.m_bias, norm_dt);
        } else if (c->arch == OR_ARCH_MINICPM) {
            auto& b = m->minicpm[l];
            for (Linear* x : {&b.m_self_attn.m_query, &b.m_self_attn.m_key, &b.m_self_attn.m_value,
                              &b.m_self_attn.m_qkv_proj, &b.m_mlp_gate_proj, &b.m_mlp_up_proj, &b.m_mlp_down_proj})
                rec(x->m_weight, dt);
            rec(b.m_input_norm.m_weight, norm_dt);
            rec(b.m_post_attn_norm.m_weight, norm_dt);
        } else {
            auto& b = *m->elm[l];
            for (Linear* x : {&b.q, &b.k, &b.v, &b.o, &b.gate, &b.up, &b.down}) rec(x->m_weight, dt);
            rec(b.q_norm.m_weight, norm_dt);
            rec(b.k_norm.m_weight, norm_dt);
            rec(b.attn_norm.m_weight, norm_dt);
            rec(b.mlp_norm.m_weight, norm_dt);
        }
    }
    if (m->rms) rec(m->rms->m_weight, norm_dt);
    if (m->ln) {
        rec(m->ln->m_weight, norm_dt);
        rec(m->ln->m_bias, norm_dt);
    }
    if (m->lm) rec(m->lm->m_weight, dt);
    return f ? 0 : -1;
}

// topk_sample's per-step sampling (gten/sampler.cpp:90-127) with the
// standard library calls the reference makes -- std::partial_sort, std::exp,
// std::discrete_distribution<int> -- over a std::mt19937 the caller seeds
// (the reference seeds it from std::random_device, sampler.cpp:70-71).
void* ref_rng_create(uint32_t seed) { return new std::mt19937(seed); }
void ref_rng_free(void* g) { delete static_cast<std::mt19937*>(g); }
uint32_t ref_rng_next(void* g) { return (uint32_t)(*static_cast<std::mt19937*>(g))(); }

int ref_topk_sample(void* g, const float* logits, int n, float temp, int top_k, double* probs_out)
{
    auto& gen = *static_cast<std::mt19937*>(g);
    top_k = std::min(top_k, 1000);
    temp = std::min(temp, 2.0f);
    std::vector<std::pair<double, int>> lp;
    lp.reserve(n);
    for (int j = 0; j < n; ++j) lp.emplace_back((double)logits[j] / temp, j);
    std::partial_sort(lp.begin(), lp.begin() + top_k, lp.end(),
                      [](const std::pair<double, int>& a, const std::pair<double, int>& b) { return a.first > b.first; });
    lp.resize(top_k);
    double sum_exp = 0;
    for (auto& e : lp) {
        e.first = std::exp(e.first);
        sum_exp += e.first;
    }
    for (auto& e : lp) e.first = e.first / sum_exp;
    std::vector<double> w(n, 0.0);
    for (const auto& e : lp) w[e.second] = e.first;
    std::discrete_distribution<int> dist(w.begin(), w.end());
    if (probs_out) {
        const std::vector<double> pr = n >= 2 ? dist.probabilities() : std::vector<double>(n, 0.0);
        std::copy(pr.begin(), pr.end(), probs_out);
    }
    return dist(gen);
}

// topk_sample's loop (sampler.cpp:84-134) over this harness's model.
int ref_generate_topk(void* p, const int32_t* prompt, int n_prompt, int n_gen, float temp, int top_k, uint32_t seed,
                      int32_t* out)
{
    auto* m = static_cast<RefModel*>(p);
    std::mt19937 gen(seed);
    std::vector<int32_t> toks(prompt, prompt + n_prompt);
    std::vector<float> lg(m->cfg.n_vocab);
    int produced = 0;
    for (int i = 0; i < n_gen; i++) {
        const int n = (int)toks.size();
        ref_model_logits(p, toks.data(), n, i == 0 ? 0 : n - 1, lg.data());
        const int t = ref_topk_sample(&gen, lg.data(), m->cfg.n_vocab, temp, top_k, nullptr);
        if (t == m->cfg.eos) break;
        out[produced++] = t;
        toks.push_back(t);
    }
    return produced;
}

// The reference's tokenizers (gten/tokenizer.cpp) as nanochat.cpp builds
// them (nanochat.cpp:189-229), behind a C interface for the tests.
struct RefTokenizer {
    std::unique_ptr<gten::LLamaTokenizer> llama;
    std::unique_ptr<gten::Gpt2Tokenizer> gpt2;
    gten::Tokenizer* t = nullptr;
};

void* ref_tok_llama_create(const char* path, int vocab_size, int eos, const char* prompt_prefix,
                           const char* prompt_suffix, const int32_t* tokens_prefix, int n_prefix,
                           const int32_t* tokens_suffix, int n_suffix)
{
    auto* r = new RefTokenizer;
    r->llama = std::make_unique<gten::LLamaTokenizer>(
            path, vocab_size, eos, std::string(prompt_prefix), std::string(prompt_suffix),
            std::vector<int>(tokens_prefix, tokens_prefix + n_prefix),
            std::vector<int>(tokens_suffix, tokens_suffix + n_suffix));
    r->t = r->llama.get();
    return r;
}

void* ref_tok_gpt2_create(const char* path, int vocab_size, int eos)
{
    auto* r = new RefTokenizer;
    r->gpt2 = std::make_unique<gten::Gpt2Tokenizer>(std::string(path), vocab_size, eos);
    r->t = r->gpt2.get();
    return r;
}

// Number of tokens of Tokenizer::encode(text); the first `cap` go to out.
int ref_tok_encode(void* p, const char* text, int32_t* out, int cap)
{
    std::string s(text);
    const std::vector<int> v = static_cast<RefTokenizer*>(p)->t->encode(s);
    for (int i = 0; i < (int)v.size() && i < cap; i++) out[i] = v[i];
    return (int)v.size();
}

const char* ref_tok_decode(void* p, int prev_token, int token)
{
    return static_cast<RefTokenizer*>(p)->t->decode(prev_token, token);
}

void ref_tok_free(void* p) { delete static_cast<RefTokenizer*>(p); }

}  // extern "C"

namespace {

// A harness model behind the reference's Model interface (gten/abc.h), so
// that the reference's own greedy_sample drives it.
class HarnessModel : public gten::Model {
public:
    HarnessModel(void* m, int inference_ctx, int train_ctx) : Model(inference_ctx, train_ctx), m_(m) {}
    Tensor logits(const Tensor& tokens, const int start_pos) override
    {
        Tensor out({static_cast<RefModel*>(m_)->cfg.n_vocab}, kFloat32);
        ref_model_logits(m_, tokens.data_ptr<int32_t>(), tokens.numel(), start_pos, out.data_ptr<float>());
        return out;
    }
    void load_from_ckpt(std::ifstream&) override {}
    void print_perf(const int) override {}

private:
    void* m_;
};

}  // namespace

extern "C" {

// gten::greedy_sample (gten/sampler.cpp:11-60) itself, prompt text in, the
// text it writes to std::cerr out (`cap` bytes at most; returns the full
// length).
int ref_greedy_sample_text(void* model, void* tok, const char* prompt, int inference_ctx, int train_ctx, char* out,
                           int cap)
{
    HarnessModel hm(model, inference_ctx, train_ctx);
    std::ostringstream os;
    std::streambuf* old = std::cerr.rdbuf(os.rdbuf());
    std::string p(prompt);
    gten::greedy_sample(p, &hm, static_cast<RefTokenizer*>(tok)->t, false);
    std::cerr.rdbuf(old);
    const std::string s = os.str();
    std::memcpy(out, s.data(), std::min<size_t>(s.size(), (size_t)cap));
    return (int)s.size();
}

}  // extern "C"
