// nc_tokenizer.cpp -- the reference's two tokenizers on the host, with its
// results: text -> token ids in front of the decode path, token id -> text
// behind it (gten/tokenizer.cpp, configured per model as nanochat.cpp:
// 189-229 does).
//
// * BPE with scores (LLamaTokenizer, gten/tokenizer.cpp:25-248; TinyLlama,
//   MiniCPM, OpenELM): the text with the prompt prefix and suffix around
//   it; a " " token first for non-empty text; each UTF-8 code point (at most
//   4 bytes) looked up as a piece, or its bytes as tokens byte + 3; then,
//   while any adjacent pair concatenates to a piece, the pair whose piece has
//   the highest score (above -1e10; the leftmost on ties) is merged; the
//   token prefix and suffix around the result.  Pieces are found as the
//   reference finds them: the vocabulary sorted by strcmp with glibc's
//   qsort (a stable merge sort at these sizes: equal pieces stay in id
//   order) and glibc's bsearch probe sequence, so a piece that occurs twice
//   resolves to the same id.  Decoding strips the leading space after BOS
//   (id 1) and turns "<0xHH>" pieces into the byte.
// * Greedy longest match (Gpt2Tokenizer, gten/tokenizer.cpp:251-334;
//   Zephyr): words by the reference's std::regex pattern, searched on the
//   remaining text as the reference loops; each word split from the left
//   into the longest vocabulary entry, each followed by the next character
//   on its own (the reference's loop takes its single-character branch after
//   every match); characters without an entry are dropped; token prefix and
//   suffix around the result.  A word that occurs
//   twice in the vocabulary maps to its last id (later entries overwrite).
//
// The merge loop keeps each adjacent pair's merged piece and score and, after
// a merge, recomputes only the two pairs next to it; the pair chosen at each
// step is the one the reference's full rescan would choose.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <regex>
#include <string>
#include <unordered_map>
#include <vector>

#include "nc_runtime.h"

namespace nc {

class TokenizerImpl {
public:
    virtual ~TokenizerImpl() = default;
    virtual int encode(const std::string& text, std::vector<int32_t>* out) = 0;
    virtual const char* decode(int prev_token, int token) = 0;
    int vocab_size = 0;
    int eos = -1;
    std::vector<int32_t> tokens_prefix, tokens_suffix;
};

class BpeTokenizer final : public TokenizerImpl {
public:
    int load(const char* path, int n)
    {
        vocab_size = n;
        for (int i = 0; i < 256; i++) {
            byte_pieces_[2 * i] = (char)i;
            byte_pieces_[2 * i + 1] = '\0';
        }
        FILE* f = std::fopen(path, "rb");
        if (!f) return fail(NC_ERR_ARG, "tokenizer: cannot open `%s`", path);
        std::unique_ptr<FILE, int (*)(FILE*)> guard(f, std::fclose);
        uint32_t max_len = 0;
        if (std::fread(&max_len, 4, 1, f) != 1) return fail(NC_ERR_ARG, "tokenizer: `%s` is empty", path);
        pieces_.resize(n);
        scores_.resize(n);
        for (int i = 0; i < n; i++) {
            int32_t len = 0;
            if (std::fread(&scores_[i], 4, 1, f) != 1 || std::fread(&len, 4, 1, f) != 1 || len < 0 ||
                len > (1 << 20))
                return fail(NC_ERR_ARG, "tokenizer: `%s` ends at piece %d of %d", path, i, n);
            pieces_[i].assign((size_t)len, '\0');
            if (len && std::fread(&pieces_[i][0], (size_t)len, 1, f) != 1)
                return fail(NC_ERR_ARG, "tokenizer: `%s` ends inside piece %d", path, i);
        }
        // strcmp order, equal pieces in id order (a stable sort)
        sorted_.resize(n);
        for (int i = 0; i < n; i++) sorted_[i] = i;
        std::stable_sort(sorted_.begin(), sorted_.end(),
                         [&](int a, int b) { return std::strcmp(pieces_[a].c_str(), pieces_[b].c_str()) < 0; });
        return NC_OK;
    }

    // glibc bsearch over the sorted pieces: the id of the entry it stops at
    int lookup(const char* s) const
    {
        size_t l = 0, u = sorted_.size();
        while (l < u) {
            const size_t idx = (l + u) / 2;
            const int c = std::strcmp(s, pieces_[sorted_[idx]].c_str());
            if (c < 0) u = idx;
            else if (c > 0) l = idx + 1;
            else return sorted_[idx];
        }
        return -1;
    }

    int encode(const std::string& text_in, std::vector<int32_t>* out) override
    {
        const std::string text = prompt_prefix + text_in + prompt_suffix;
        std::vector<int32_t> t;
        const char* c0 = text.c_str();
        if (c0[0] != '\0') t.push_back(lookup(" "));
        std::string cp;
        for (const char* c = c0; *c != '\0'; c++) {
            if ((*c & 0xC0) != 0x80) cp.clear();
            cp.push_back(*c);
            if ((c[1] & 0xC0) == 0x80 && cp.size() < 4) continue;
            const int id = lookup(cp.c_str());
            if (id != -1) {
                t.push_back(id);
            } else {
                for (unsigned char b : cp) t.push_back((int32_t)b + 3);
            }
            cp.clear();
        }
        for (int32_t id : t)
            if (id < 0 || id >= vocab_size) return fail(NC_ERR_ARG, "tokenizer: piece id %d outside the vocabulary", id);
        merge(&t);
        out->assign(tokens_prefix.begin(), tokens_prefix.end());
        out->insert(out->end(), t.begin(), t.end());
        out->insert(out->end(), tokens_suffix.begin(), tokens_suffix.end());
        return NC_OK;
    }

    const char* decode(int prev_token, int token) override
    {
        if (token >= vocab_size || token < 0) return "";
        const char* piece = pieces_[token].c_str();
        if (prev_token == 1 && piece[0] == ' ') piece++;
        unsigned char b;
        if (std::sscanf(piece, "<0x%02hhX>", &b) == 1) piece = byte_pieces_ + 2 * b;
        return piece;
    }

    std::string prompt_prefix, prompt_suffix;

private:
    struct Pair {
        int id;       // merged piece, or -1
        float score;
    };

    Pair pair_of(int a, int b) const
    {
        const std::string s = std::string(pieces_[a].c_str()) + pieces_[b].c_str();
        const int id = lookup(s.c_str());
        return {id, id != -1 ? scores_[id] : 0.0f};
    }

    void merge(std::vector<int32_t>* tp)
    {
        std::vector<int32_t>& t = *tp;
        if (t.size() < 2) return;
        std::vector<Pair> p(t.size() - 1);
        for (size_t i = 0; i + 1 < t.size(); i++) p[i] = pair_of(t[i], t[i + 1]);
        for (;;) {
            float best = -1e10f;
            long bi = -1;
            for (size_t i = 0; i < p.size(); i++)
                if (p[i].id != -1 && p[i].score > best) {
                    best = p[i].score;
                    bi = (long)i;
                }
            if (bi < 0) return;
            t[bi] = p[bi].id;
            t.erase(t.begin() + bi + 1);
            p.erase(p.begin() + bi);
            if (bi > 0) p[bi - 1] = pair_of(t[bi - 1], t[bi]);
            if ((size_t)bi < p.size()) p[bi] = pair_of(t[bi], t[bi + 1]);
        }
    }

    std::vector<std::string> pieces_;
    std::vector<float> scores_;
    std::vector<int> sorted_;
    char byte_pieces_[512];
};

class WordTokenizer final : public TokenizerImpl {
public:
    int load(const char* path, int n)
    {
        vocab_size = n;
        std::ifstream f(path, std::ios::binary);
        if (!f) return fail(NC_ERR_ARG, "tokenizer: cannot open `%s`", path);
        words_.resize(n);
        int i = 0;
        for (; i < n; i++) {
            uint32_t len = 0;
            f.read(reinterpret_cast<char*>(&len), 4);
            if (!f && f.gcount() == 0 && i > 0) break;  // the file holds fewer words than the vocabulary
            if (!f || len > (1u << 20)) return fail(NC_ERR_ARG, "tokenizer: `%s` is cut inside word %d", path, i);
            words_[i].assign(len, '\0');
            f.read(&words_[i][0], len);
            if (!f) return fail(NC_ERR_ARG, "tokenizer: `%s` ends inside word %d", path, i);
            ids_[words_[i]] = i;
        }
        // Past the end of the file the reference's reads fail and its loop
        // keeps the last word it read (gten/tokenizer.cpp:256-268 as
        // compiled): every remaining id holds that word, and the word maps to
        // the last id.  Zephyr's vocabulary file has 100256 words for 100352
        // ids.
        for (; i < n; i++) {
            words_[i] = words_[i - 1];
            ids_[words_[i]] = i;
        }
        return NC_OK;
    }

    int encode(const std::string& text, std::vector<int32_t>* out) override
    {
        static const std::regex re(
                R"('s|'t|'re|'ve|'m|'ll|'d| ?[[:alpha:]]+| ?[[:digit:]]+| ?[^\s[:alpha:][:digit:]]+|\s+(?!\S)|\s+)");
        out->assign(tokens_prefix.begin(), tokens_prefix.end());
        std::string rest = text;
        std::smatch m;
        while (std::regex_search(rest, m, re)) {
            const std::string word = m.str(0);
            split(word, out);
            rest = m.suffix().str();
        }
        out->insert(out->end(), tokens_suffix.begin(), tokens_suffix.end());
        return NC_OK;
    }

    const char* decode(int, int token) override
    {
        if (token < 0 || token >= vocab_size) return "";
        return words_[token].c_str();
    }

private:
    // The reference's split of one word (gten/tokenizer.cpp:299-324): the
    // longest entry starting at i, then -- unless the word ended -- the next
    // character as a token of its own (dropped when it has no entry), since
    // the loop's single-character branch is taken after every match too.
    void split(const std::string& w, std::vector<int32_t>* out) const
    {
        const size_t n = w.size();
        size_t i = 0;
        while (i < n) {
            for (size_t j = n; j > i; j--) {
                auto it = ids_.find(w.substr(i, j - i));
                if (it != ids_.end()) {
                    out->push_back(it->second);
                    i = j;
                    break;
                }
            }
            if (i == n) break;
            auto it = ids_.find(w.substr(i, 1));
            if (it != ids_.end()) out->push_back(it->second);
            i++;
        }
    }

    std::vector<std::string> words_;
    std::unordered_map<std::string, int32_t> ids_;
};

}  // namespace nc

using nc::TokenizerImpl;

extern "C" {

int nc_tokenizer_load_bpe(const char* path, int vocab_size, int eos, const char* prompt_prefix,
                          const char* prompt_suffix, const int32_t* tokens_prefix, int n_prefix,
                          const int32_t* tokens_suffix, int n_suffix, void** tokenizer)
{
    NC_CHECK_ARG(path && tokenizer && vocab_size > 0 && n_prefix >= 0 && n_suffix >= 0 &&
                         (tokens_prefix || !n_prefix) && (tokens_suffix || !n_suffix),
                 "tokenizer_load_bpe: bad arguments");
    *tokenizer = nullptr;
    auto t = std::make_unique<nc::BpeTokenizer>();
    int s = t->load(path, vocab_size);
    if (s) return s;
    t->eos = eos;
    t->prompt_prefix = prompt_prefix ? prompt_prefix : "";
    t->prompt_suffix = prompt_suffix ? prompt_suffix : "";
    t->tokens_prefix.assign(tokens_prefix, tokens_prefix + n_prefix);
    t->tokens_suffix.assign(tokens_suffix, tokens_suffix + n_suffix);
    *tokenizer = static_cast<TokenizerImpl*>(t.release());
    return NC_OK;
}

int nc_tokenizer_load_words(const char* path, int vocab_size, int eos, const int32_t* tokens_prefix, int n_prefix,
                            const int32_t* tokens_suffix, int n_suffix, void** tokenizer)
{
    NC_CHECK_ARG(path && tokenizer && vocab_size > 0 && n_prefix >= 0 && n_suffix >= 0 &&
                         (tokens_prefix || !n_prefix) && (tokens_suffix || !n_suffix),
                 "tokenizer_load_words: bad arguments");
    *tokenizer = nullptr;
    auto t = std::make_unique<nc::WordTokenizer>();
    int s = t->load(path, vocab_size);
    if (s) return s;
    t->eos = eos;
    t->tokens_prefix.assign(tokens_prefix, tokens_prefix + n_prefix);
    t->tokens_suffix.assign(tokens_suffix, tokens_suffix + n_suffix);
    *tokenizer = static_cast<TokenizerImpl*>(t.release());
    return NC_OK;
}

int nc_tokenizer_load_for_model(const char* model, const char* path, void** tokenizer)
{
    NC_CHECK_ARG(model && path && tokenizer, "tokenizer_load_for_model: bad arguments");
    const std::string m = model;
    // TinyLlama and OpenELM: vocab n_vocab - 3 = 32000 and eos
    // tinyllama_cfg.eos = 32002 (tinyllama/tinyllama.h:13,20)
    if (m == "tinyllama") {
        const int32_t pre[] = {1, 32001}, suf[] = {32002, 29871, 13, 32001, 20255, 13};
        return nc_tokenizer_load_bpe(path, 32000, 32002, "user\n", "", pre, 2, suf, 6, tokenizer);
    }
    if (m == "zephyr") {
        const int32_t pre[] = {27, 91, 882, 91, 29, 397}, suf[] = {100257, 198, 27, 91, 78191, 91, 397};
        return nc_tokenizer_load_words(path, 100352, 100257, pre, 6, suf, 7, tokenizer);
    }
    if (m == "minicpm") return nc_tokenizer_load_bpe(path, 122753, 2, "<用户>", "<AI>", nullptr, 0, nullptr, 0, tokenizer);
    if (m == "openelm_sm" || m == "openelm_md" || m == "openelm_lg") {
        const int32_t pre[] = {1};
        return nc_tokenizer_load_bpe(path, 32000, 32002, "", "", pre, 1, nullptr, 0, tokenizer);
    }
    return nc::fail(NC_ERR_ARG, "tokenizer_load_for_model: unknown model `%s`", model);
}

int nc_tokenizer_encode(void* tokenizer, const char* text, int32_t* out, int cap, int* n_out)
{
    NC_CHECK_ARG(tokenizer && text && n_out && cap >= 0 && (out || !cap), "tokenizer_encode: bad arguments");
    std::vector<int32_t> v;
    int s = static_cast<TokenizerImpl*>(tokenizer)->encode(text, &v);
    if (s) return s;
    *n_out = (int)v.size();
    NC_CHECK_ARG((int)v.size() <= cap, "tokenizer_encode: %zu tokens, room for %d", v.size(), cap);
    std::copy(v.begin(), v.end(), out);
    return NC_OK;
}

const char* nc_tokenizer_decode(void* tokenizer, int prev_token, int token)
{
    return tokenizer ? static_cast<TokenizerImpl*>(tokenizer)->decode(prev_token, token) : "";
}

int nc_tokenizer_eos(void* tokenizer) { return tokenizer ? static_cast<TokenizerImpl*>(tokenizer)->eos : -1; }

int nc_tokenizer_free(void* tokenizer)
{
    delete static_cast<TokenizerImpl*>(tokenizer);
    return NC_OK;
}

}  // extern "C"
