// Byte-level BPE tokenizer over the reference's exported tokenizer.bin /
// merges.bin / chat templates (src/tokenizer.cpp:22-381, formats written by
// export.py:49-188).  Host code behind a C ABI.
//
// Encoding follows the reference's algorithm step by step, because its
// output (not a textbook BPE's) is what the model was run with:
//   1. scan: at '<', the text up to the first '>' within the longest token
//      length is one token if the vocabulary holds it whole; every other
//      byte is its own single-byte token (src/tokenizer.cpp:177-204);
//   2. merge: a priority queue of adjacent pairs ordered by merge rank, then
//      by left position; a popped pair whose left node is gone, is last, or
//      whose two ids changed since it was queued is skipped; a merge writes
//      the merged id into the left node, unlinks the right one and queues
//      the new pairs on both sides (:212-314).
// Lookups use hash maps instead of the reference's bsearch over a strcmp
// sort; for the strings the scan produces (no NUL bytes) both find the same
// id (the lowest one if the vocabulary repeats a string).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <new>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/toyinfer_attn.h"
#include "../../include/toyinfer_tokenizer.h"

struct toyinfer_tokenizer {
    std::vector<std::string> vocab;  // [vocab_size] raw bytes
    std::unordered_map<std::string, uint32_t> index;
    // (left << 32 | right) -> (merged id, rank); a repeated pair keeps the last
    // rank, as the reference's map assignment (src/tokenizer.cpp:35-37).
    std::unordered_map<uint64_t, std::pair<uint32_t, uint32_t>> merges;
    uint32_t num_merges = 0;
    size_t max_token_len = 0;
    std::string system_template, user_template;
};

namespace {

bool read_file(const std::string& path, std::string& out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
    return !f.bad();
}

uint32_t le32(const std::string& b, size_t off) {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(b.data()) + off;
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

// src/tokenizer.cpp:74-124: count, then (length, bytes) per id while the
// file lasts; later ids stay empty.
int load_vocab(toyinfer_tokenizer* t, const std::string& dir, uint32_t vocab_size) {
    std::string b;
    if (!read_file(dir + "/tokenizer.bin", b) || b.size() < 4) return TOYINFER_ERR_IO;
    if (le32(b, 0) > vocab_size) return TOYINFER_ERR_IO;
    t->vocab.assign(vocab_size, std::string());
    size_t off = 4;
    for (uint32_t i = 0; i < vocab_size && off < b.size(); ++i) {
        if (b.size() - off < 4) return TOYINFER_ERR_IO;
        const uint32_t len = le32(b, off);
        off += 4;
        if (b.size() - off < len) return TOYINFER_ERR_IO;
        t->vocab[i].assign(b, off, len);
        off += len;
        if (len > t->max_token_len) t->max_token_len = len;
    }
    for (uint32_t i = vocab_size; i-- > 0;) t->index[t->vocab[i]] = i;  // lowest id wins
    return TOYINFER_OK;
}

// src/tokenizer.cpp:22-39: count, then (left, right, merged) per rank.
int load_merges(toyinfer_tokenizer* t, const std::string& dir) {
    std::string b;
    if (!read_file(dir + "/merges.bin", b) || b.size() < 4) return TOYINFER_ERR_IO;
    const uint32_t n = le32(b, 0);
    if ((b.size() - 4) / 12 < n) return TOYINFER_ERR_IO;
    const uint32_t v = (uint32_t)t->vocab.size();
    t->merges.reserve(n);
    for (uint32_t r = 0; r < n; ++r) {
        const uint32_t a = le32(b, 4 + 12ull * r), c = le32(b, 8 + 12ull * r),
                       m = le32(b, 12 + 12ull * r);
        if (a >= v || c >= v || m >= v) return TOYINFER_ERR_IO;
        t->merges[(uint64_t)a << 32 | c] = {m, r};
    }
    t->num_merges = n;
    return TOYINFER_OK;
}

bool find_token(const toyinfer_tokenizer* t, const std::string& s, uint32_t& id) {
    const auto it = t->index.find(s);
    if (it == t->index.end()) return false;
    id = it->second;
    return true;
}

struct MergeJob {
    uint32_t rank, idx, left, right;
};
// Lower rank first, then the smaller position (src/tokenizer.cpp:228-233).
struct JobAfter {
    bool operator()(const MergeJob& a, const MergeJob& b) const {
        return a.rank != b.rank ? a.rank > b.rank : a.idx > b.idx;
    }
};

// Appends the expansion of `tmpl` with args[] for each "%s" ("%%" is '%').
bool render(const std::string& tmpl, const char* const* args, int nargs, std::string& out) {
    int used = 0;
    for (size_t i = 0; i < tmpl.size(); ++i) {
        if (tmpl[i] != '%') {
            out.push_back(tmpl[i]);
            continue;
        }
        if (i + 1 >= tmpl.size()) return false;
        const char c = tmpl[++i];
        if (c == '%') {
            out.push_back('%');
        } else if (c == 's' && used < nargs) {
            out.append(args[used++]);
        } else {
            return false;
        }
    }
    return true;
}

}  // namespace

extern "C" {

int toyinfer_tokenizer_create(const char* model_dir, uint32_t vocab_size, int thinking,
                              toyinfer_tokenizer** out) {
    if (!out) return TOYINFER_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    if (!model_dir || vocab_size == 0) return TOYINFER_ERR_INVALID_ARGUMENT;
    toyinfer_tokenizer* t = new (std::nothrow) toyinfer_tokenizer();
    if (!t) return TOYINFER_ERR_IO;
    const std::string dir(model_dir);
    int st = load_vocab(t, dir, vocab_size);
    if (st == TOYINFER_OK) st = load_merges(t, dir);
    // src/tokenizer.cpp:126-134: the thinking or the plain pair of templates.
    const std::string sfx = thinking ? "_thinking.txt" : ".txt";
    if (st == TOYINFER_OK && (!read_file(dir + "/template_system" + sfx, t->system_template) ||
                              !read_file(dir + "/template_user" + sfx, t->user_template)))
        st = TOYINFER_ERR_IO;
    if (st != TOYINFER_OK) {
        delete t;
        return st;
    }
    *out = t;
    return TOYINFER_OK;
}

void toyinfer_tokenizer_destroy(toyinfer_tokenizer* t) { delete t; }

int toyinfer_tokenizer_encode(toyinfer_tokenizer* t, const char* text, uint32_t* ids,
                              uint32_t cap, uint32_t* count) {
    if (!t || !text || !count || (cap && !ids)) return TOYINFER_ERR_INVALID_ARGUMENT;
    *count = 0;
    // 1. Special tokens and single bytes.
    std::vector<uint32_t> tok;
    tok.reserve(strlen(text));
    for (const char* ch = text; *ch; ++ch) {
        uint32_t id = 0;
        bool found = false;
        if (*ch == '<') {
            for (size_t i = 0; i < t->max_token_len && ch[i]; ++i) {
                if (ch[i] != '>') continue;
                if (find_token(t, std::string(ch, i + 1), id)) {
                    found = true;
                    ch += i;
                }
                break;
            }
        }
        if (!found && !find_token(t, std::string(1, *ch), id)) return TOYINFER_ERR_INVALID_ARGUMENT;
        tok.push_back(id);
    }
    // 2. Merges over a doubly linked list of nodes.
    const int32_t n = (int32_t)tok.size();
    std::vector<int32_t> prev(n), next(n);
    std::vector<char> valid(n, 1);
    for (int32_t i = 0; i < n; ++i) {
        prev[i] = i - 1;
        next[i] = i + 1 < n ? i + 1 : -1;
    }
    auto pair_of = [&](uint32_t a, uint32_t b, std::pair<uint32_t, uint32_t>& mr) {
        const auto it = t->merges.find((uint64_t)a << 32 | b);
        if (it == t->merges.end()) return false;
        mr = it->second;
        return true;
    };
    std::priority_queue<MergeJob, std::vector<MergeJob>, JobAfter> q;
    std::pair<uint32_t, uint32_t> mr;
    for (int32_t i = 0; i + 1 < n; ++i)
        if (pair_of(tok[i], tok[i + 1], mr)) q.push({mr.second, (uint32_t)i, tok[i], tok[i + 1]});
    int32_t live = n;
    while (!q.empty()) {
        const MergeJob j = q.top();
        q.pop();
        const int32_t c = (int32_t)j.idx;
        if (!valid[c] || next[c] == -1) continue;
        const int32_t r = next[c];
        if (tok[r] != j.right || tok[c] != j.left) continue;
        if (!pair_of(tok[c], tok[r], mr)) return TOYINFER_ERR_IO;
        tok[c] = mr.first;
        valid[r] = 0;
        next[c] = next[r];
        --live;
        if (next[r] != -1) prev[next[r]] = c;
        if (prev[c] != -1 && pair_of(tok[prev[c]], tok[c], mr))
            q.push({mr.second, (uint32_t)prev[c], tok[prev[c]], tok[c]});
        if (next[c] != -1 && pair_of(tok[c], tok[next[c]], mr))
            q.push({mr.second, (uint32_t)c, tok[c], tok[next[c]]});
    }
    *count = (uint32_t)live;
    uint32_t w = 0;
    for (int32_t i = n ? 0 : -1; i != -1 && w < cap; i = next[i]) ids[w++] = tok[i];
    return (uint32_t)live <= cap ? TOYINFER_OK : TOYINFER_ERR_WORKSPACE;
}

const char* toyinfer_tokenizer_decode(const toyinfer_tokenizer* t, uint32_t id, uint32_t* len) {
    if (!t || id >= t->vocab.size()) return nullptr;
    if (len) *len = (uint32_t)t->vocab[id].size();
    return t->vocab[id].c_str();
}

int toyinfer_tokenizer_render_prompt(const toyinfer_tokenizer* t, const char* user_prompt,
                                     const char* system_prompt, char* buf, size_t cap,
                                     size_t* len) {
    if (!t || !user_prompt || !len || (cap && !buf)) return TOYINFER_ERR_INVALID_ARGUMENT;
    std::string out;
    const char* args[2] = {system_prompt, user_prompt};
    const bool ok = system_prompt ? render(t->system_template, args, 2, out)
                                  : render(t->user_template, args + 1, 1, out);
    if (!ok) return TOYINFER_ERR_INVALID_ARGUMENT;
    *len = out.size();
    if (cap == 0) return TOYINFER_ERR_WORKSPACE;
    const size_t w = out.size() < cap ? out.size() : cap - 1;
    memcpy(buf, out.data(), w);
    buf[w] = '\0';
    return out.size() < cap ? TOYINFER_OK : TOYINFER_ERR_WORKSPACE;
}

uint32_t toyinfer_tokenizer_vocab_size(const toyinfer_tokenizer* t) {
    return t ? (uint32_t)t->vocab.size() : 0;
}
uint32_t toyinfer_tokenizer_num_merges(const toyinfer_tokenizer* t) {
    return t ? t->num_merges : 0;
}

}  // extern "C"
