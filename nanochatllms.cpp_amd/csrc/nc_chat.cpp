// nc_chat.cpp -- the text path of the reference's samplers, greedy_sample
// and topk_sample (gten/sampler.cpp:11-143): prompt text in, generated text
// out, on the library's own public entry points -- the tokenizer
// (nc_tokenizer_*) and the model's split generation (nc_model_prefill +
// nc_model_decode, nc_model_sample_begin + nc_model_sample_steps).  The
// device runs ahead of the host in chunks of steps with no host round trip
// inside a chunk; the host then walks the new tokens in order, stops at the
// tokenizer's eos as the reference's loop does, and hands each token's
// decode(prev, token) to the caller's sink.  Steps the device ran past eos
// are discarded (the next call starts again from position 0).
#include <algorithm>
#include <cstring>
#include <vector>

#include "nc_runtime.h"

namespace {

// Steps between host checks: 1, 2, 4, ... up to kChunkMax, so the first
// words come back after a step or two and long answers pay one host round
// trip per kChunkMax tokens.
constexpr int kChunkMax = 16;

// start(prompt, n): runs the prompt and leaves the first generated token on
// the device; steps(n, out): n more steps, then every token generated since
// the prompt into out.
template <class Start, class Steps>
int sample_text(void* model, void* tokenizer, const char* prompt, int n_predict, nc_text_sink sink, void* user,
                int* n_tokens, Start&& start, Steps&& steps)
{
    NC_CHECK_ARG(model && tokenizer && prompt && n_tokens, "sample: null argument");
    *n_tokens = 0;
    nc_model_config cfg;
    int s = nc_model_get_config(model, &cfg);
    if (s) return s;
    if (n_predict <= 0) n_predict = cfg.max_ctx;
    NC_CHECK_ARG(n_predict <= cfg.max_ctx, "sample: n_predict %d exceeds the model's max_ctx %d", n_predict,
                 cfg.max_ctx);
    const int eos = nc_tokenizer_eos(tokenizer);

    // tokens = tokenizer->encode(prompt)
    int np = 0;
    std::vector<int32_t> toks(std::strlen(prompt) + 64);
    s = nc_tokenizer_encode(tokenizer, prompt, toks.data(), (int)toks.size(), &np);
    if (s && np > (int)toks.size()) {
        toks.resize(np);
        s = nc_tokenizer_encode(tokenizer, prompt, toks.data(), np, &np);
    }
    if (s) return s;
    NC_CHECK_ARG(np > 0, "sample: the prompt encodes to no tokens");

    // for (i < n_predict - tokens.size()): one token per iteration, eos ends
    const int max_iters = n_predict - np;
    if (max_iters > 0) {
        if ((s = start(toks.data(), np))) return s;
        std::vector<int32_t> gen(max_iters);
        int have = 1;   // tokens on the device (the prompt's own first)
        int done = 0;   // tokens the host has walked
        int chunk = 1;
        int prev = 1;
        bool stop = false;
        while (!stop) {
            // every token so far; the first chunk only fetches
            const int more = done == 0 ? 0 : std::min(chunk, max_iters - have);
            if ((s = steps(more, gen.data()))) return s;
            have += more;
            for (; done < have; done++) {
                const int tok = gen[done];
                if (tok == eos) {
                    stop = true;
                    break;
                }
                if (sink) sink(nc_tokenizer_decode(tokenizer, prev, tok), user);
                prev = tok;
                *n_tokens += 1;
            }
            if (have >= max_iters) stop = true;
            chunk = std::min(2 * chunk, kChunkMax);
        }
    }
    if (sink) sink("\n", user);
    return NC_OK;
}

}  // namespace

extern "C" {

int nc_greedy_sample(void* model, void* tokenizer, const char* prompt, int n_predict, nc_text_sink sink, void* user,
                     int* n_tokens)
{
    return sample_text(
            model, tokenizer, prompt, n_predict, sink, user, n_tokens,
            [&](const int32_t* p, int n) { return nc_model_prefill(model, p, n); },
            [&](int n, int32_t* out) { return nc_model_decode(model, n, out); });
}

int nc_topk_sample(void* model, void* tokenizer, const char* prompt, int n_predict, float temp, int top_k,
                   uint32_t seed, nc_text_sink sink, void* user, int* n_tokens)
{
    return sample_text(
            model, tokenizer, prompt, n_predict, sink, user, n_tokens,
            [&](const int32_t* p, int n) { return nc_model_sample_begin(model, p, n, temp, top_k, seed); },
            [&](int n, int32_t* out) { return nc_model_sample_steps(model, n, out); });
}

}  // extern "C"
