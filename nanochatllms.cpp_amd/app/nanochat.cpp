// nanochat.cpp -- the package's chat program, as the reference's main
// (src/nanochat.cpp:36-263) runs it: a model from its .gten checkpoint, the
// model's tokenizer (nanochat.cpp:189-229), then one prompt (-p) or a chat
// loop (a prompt per line, "q" quits), each answered by greedy_sample
// (-greedy) or topk_sample, streamed to stderr as the reference streams it.
// Everything goes through the library's C-ABI (include/gten_hip.h).
//
// The reference shells out to a downloader first; this program reads what
// is already on disk: --model-dir (default ./models, the reference's
// <name>.<fp16|q8|q4>.gten names) and --tokenizer-dir (default
// ./assets/tokenizers).  topk_sample draws from std::mt19937 seeded by
// std::random_device as the reference does, or by --seed.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <random>
#include <string>

#include "../../include/gten_hip.h"

namespace {

const char* kUsage = R"(
USAGE:
./nanochat [options] -m MODEL_NAME -p PROMPT  for a single prompt or
./nanochat [options] -m MODEL_NAME for a chat interface.

Available MODEL_NAME options are [tinyllama, zephyr, minicpm, openelm_sm, openelm_md, openelm_lg].

Optional args.
-f16 :     Use float-16 model and inference. [default]
-q8  :     Use 8-bit quantized model.
-q4  :     Use 4-bit quantized model.
-greedy :  Greedy sampling instead of top-k.
-showstat  : Show inference performance stats.
--temp T   : Temperature to use during sampling. It must be greater than 0.
--npred  N : Max number of tokens to generate. Minimum is 1.
--topk K   : Top tokens to randomly select from during prediction. Minimum is 1.
--seed S   : Seed of the sampler (default: std::random_device).
--model-dir D, --tokenizer-dir D, --device N
)";

// The reference's model configurations: tinyllama/tinyllama.h:12-24,
// zephyr/zephyr.h:10-23, minicpm/minicpm.h:9-24, openelm/openelm.h:13-51.
// Returns the train context (max_ctx of the header), 0 for an unknown name.
int model_config(const std::string& name, nc_model_config* c)
{
    std::memset(c, 0, sizeof(*c));
    c->d_head = 64;
    c->rope_pct = 1.0f;
    auto uniform = [&](int layers, int hq, int hkv, int ffn) {
        c->n_layers = layers;
        for (int l = 0; l < layers; l++) {
            c->n_heads[l] = hq;
            c->n_kv_heads[l] = hkv;
            c->n_ffn[l] = ffn;
        }
    };
    if (name == "tinyllama") {
        c->arch = NC_ARCH_LLAMA;
        c->n_vocab = 32003;
        c->n_embd = 2048;
        c->eos = 32002;
        uniform(22, 32, 4, 5632);
        return 2048;
    }
    if (name == "zephyr") {
        c->arch = NC_ARCH_ZEPHYR;
        c->n_vocab = 100352;
        c->n_embd = 2048;
        c->eos = 100257;
        c->rope_pct = 0.25f;
        uniform(24, 32, 32, 5632);
        return 4096;
    }
    if (name == "minicpm") {
        c->arch = NC_ARCH_MINICPM;
        c->n_vocab = 122753;
        c->n_embd = 2304;
        c->eos = 2;
        uniform(40, 36, 36, 5760);
        return 2048;
    }
    static const int sm_q[] = {12, 12, 12, 12, 12, 16, 16, 16, 16, 16, 16, 16, 20, 20, 20, 20};
    static const int sm_kv[] = {3, 3, 3, 3, 3, 4, 4, 4, 4, 4, 4, 4, 5, 5, 5, 5};
    static const int sm_f[] = {768, 1024, 1280, 1536, 1792, 2048, 2560, 2816,
                               3072, 3328, 3584, 3840, 4352, 4608, 4864, 5120};
    static const int md_q[] = {12, 12, 12, 16, 16, 16, 16, 16, 16, 16, 20, 20, 20, 20, 20, 20, 24, 24, 24, 24};
    static const int md_kv[] = {3, 3, 3, 4, 4, 4, 4, 4, 4, 4, 5, 5, 5, 5, 5, 5, 6, 6, 6, 6};
    static const int md_f[] = {768,  1024, 1280, 1536, 1792, 2304, 2560, 2816, 3072, 3328,
                               3584, 3840, 4096, 4352, 4608, 5120, 5376, 5632, 5888, 6144};
    static const int lg_q[] = {16, 16, 16, 20, 20, 20, 20, 20, 20, 20, 24, 24, 24, 24,
                               24, 24, 24, 24, 28, 28, 28, 28, 28, 28, 32, 32, 32, 32};
    static const int lg_kv[] = {4, 4, 4, 5, 5, 5, 5, 5, 5, 5, 6, 6, 6, 6, 6, 6, 6, 6, 7, 7, 7, 7, 7, 7, 8, 8, 8, 8};
    static const int lg_f[] = {1024, 1280, 1536, 1792, 2048, 2304, 2560, 2816, 3072, 3328, 3584, 3840, 4096, 4608,
                               4608, 5120, 5376, 5632, 5888, 6144, 6400, 6656, 6912, 7168, 7424, 7680, 7936, 8192};
    const int *q = nullptr, *kv = nullptr, *f = nullptr;
    if (name == "openelm_sm") {
        c->n_layers = 16, c->n_embd = 1280, q = sm_q, kv = sm_kv, f = sm_f;
    } else if (name == "openelm_md") {
        c->n_layers = 20, c->n_embd = 1536, q = md_q, kv = md_kv, f = md_f;
    } else if (name == "openelm_lg") {
        c->n_layers = 28, c->n_embd = 2048, q = lg_q, kv = lg_kv, f = lg_f;
    } else {
        return 0;
    }
    c->arch = NC_ARCH_OPENELM;
    c->n_vocab = 32000;
    c->eos = 32002;
    for (int l = 0; l < c->n_layers; l++) {
        c->n_heads[l] = q[l];
        c->n_kv_heads[l] = kv[l];
        c->n_ffn[l] = f[l];
    }
    return 2048;
}

const char* tokenizer_file(const std::string& name)
{
    if (name == "zephyr") return "zephyr_tokenizer.bin";
    if (name == "minicpm") return "minicpm_tokenizer.bin";
    return "tinyllama_tokenizer.bin";  // TinyLlama and OpenELM
}

void to_stderr(const char* text, void*) { std::cerr << text << std::flush; }

[[noreturn]] void die(const std::string& what)
{
    std::cerr << "error: " << what << ": " << nc_last_error() << "\n";
    std::exit(EXIT_FAILURE);
}

bool parse_int(const char* s, int* out)
{
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (!end || *end || end == s) return false;
    *out = (int)v;
    return true;
}

}  // namespace

int main(int argc, char** argv)
{
    int wdtype = NC_F16;
    std::string model_name, prompt, model_dir = "./models", tok_dir = "./assets/tokenizers";
    int n_predict = 1024;
    bool greedy = false, showstat = false, have_seed = false;
    float temp = 0.9f;
    int topk = 50, device = 0, seed = 0;
    for (int i = 1; i < argc; i++) {
        const std::string a = argv[i];
        const bool has_val = i + 1 < argc;
        if (a == "--help" || a == "-h") {
            std::cout << kUsage << "\n";
            return 0;
        } else if (a == "-f16") {
            wdtype = NC_F16;
        } else if (a == "-q8") {
            wdtype = NC_Q8;
        } else if (a == "-q4") {
            wdtype = NC_Q4;
        } else if (a == "-greedy") {
            greedy = true;
        } else if (a == "-showstat") {
            showstat = true;
        } else if (a == "-m" && has_val) {
            model_name = argv[++i];
        } else if (a == "-p" && has_val) {
            prompt = argv[++i];
        } else if (a == "--npred" && has_val) {
            if (!parse_int(argv[++i], &n_predict) || n_predict < 1) {
                std::cerr << "npred must be an integer >= 1.\n";
                return -1;
            }
        } else if (a == "--temp" && has_val) {
            char* end = nullptr;
            temp = std::strtof(argv[++i], &end);
            if (!end || *end || !(temp > 0.0f)) {
                std::cerr << "temp value must be greater than zero.\n";
                return -1;
            }
        } else if (a == "--topk" && has_val) {
            if (!parse_int(argv[++i], &topk) || topk < 1) {
                std::cerr << "topk must be gte 1.\n";
                return -1;
            }
        } else if (a == "--seed" && has_val) {
            if (!parse_int(argv[++i], &seed)) {
                std::cerr << "Invalid seed value.\n";
                return -1;
            }
            have_seed = true;
        } else if (a == "--model-dir" && has_val) {
            model_dir = argv[++i];
        } else if (a == "--tokenizer-dir" && has_val) {
            tok_dir = argv[++i];
        } else if (a == "--device" && has_val) {
            if (!parse_int(argv[++i], &device)) return -1;
        } else {
            std::cerr << "error: Unknown or incomplete argument: " << a << "\n" << kUsage;
            return EXIT_FAILURE;
        }
    }
    nc_model_config cfg;
    const int train_ctx = model_name.empty() ? 0 : model_config(model_name, &cfg);
    if (!train_ctx) {
        std::cerr << "error: Unknown or missing model name: " << model_name << ".\n" << kUsage << "\n";
        return EXIT_FAILURE;
    }
    // the model's inference context: greedy_sample / topk_sample generate up
    // to min(inference ctx, train ctx) positions (sampler.cpp:13,68)
    cfg.wdtype = wdtype;
    cfg.max_ctx = std::min(n_predict, std::min(train_ctx, NC_MAX_CTX));
    const char* dt = wdtype == NC_F16 ? "fp16" : (wdtype == NC_Q8 ? "q8" : "q4");
    const std::string ckpt = model_dir + "/" + model_name + "." + dt + ".gten";
    const std::string tok_path = tok_dir + "/" + tokenizer_file(model_name);

    if (nc_init(device)) die("nc_init");
    void* model = nullptr;
    void* tok = nullptr;
    if (nc_model_create(&cfg, &model)) die("model");
    if (nc_model_load_gten(model, ckpt.c_str())) die("checkpoint " + ckpt);
    if (nc_tokenizer_load_for_model(model_name.c_str(), tok_path.c_str(), &tok)) die("tokenizer " + tok_path);

    std::mt19937 seeder(have_seed ? (uint32_t)seed : std::random_device{}());
    auto answer = [&](const std::string& p) {
        int n = 0;
        const auto t0 = std::chrono::steady_clock::now();
        const int s = greedy ? nc_greedy_sample(model, tok, p.c_str(), 0, to_stderr, nullptr, &n)
                             : nc_topk_sample(model, tok, p.c_str(), 0, temp, topk, (uint32_t)seeder(), to_stderr,
                                              nullptr, &n);
        if (s) die("sample");
        if (showstat) {
            const double ms =
                    std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            std::cerr << "\n" << n << " tokens in " << ms << " ms (" << (ms > 0 ? n * 1000.0 / ms : 0.0)
                      << " tokens/s, prompt included)\n";
        }
    };
    if (prompt.empty()) {
        std::cout << "Chat interface. Write your prompt and press enter to submit. Enter q or press ctrl+c to quit.\n";
        std::string line;
        while (true) {
            std::cerr << "\n\n[You]: ";
            if (!std::getline(std::cin, line) || line == "q") break;
            std::cerr << "\n[" + model_name + "-Chat]: \n\n";
            answer(line);
        }
    } else {
        answer(prompt);
    }
    nc_tokenizer_free(tok);
    nc_model_free(model);
    return 0;
}
