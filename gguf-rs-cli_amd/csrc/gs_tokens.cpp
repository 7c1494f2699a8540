// gs_tokens.cpp -- token id -> text and the stop-token set (declared in
// include/gs_tokens.h).  Host code: the text step after the sampler in
// gguf-rs-cli (src/tokenizer/bpe.rs:180-208, src/tokenizer/chat.rs:9-72).
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/gs_sampler.h"
#include "../../include/gs_tokens.h"

struct gs_vocab {
    uint32_t model;
    std::vector<uint64_t> off;           // raw token bytes
    std::string raw;
    std::vector<uint64_t> doff;          // decoded text of each token
    std::string dec;
    std::unordered_map<std::string, uint32_t> to_id;
};

namespace {

// Appends code point c as UTF-8.
void put_utf8(std::string &o, uint32_t c)
{
    if (c < 0x80) {
        o.push_back((char)c);
    } else if (c < 0x800) {
        o.push_back((char)(0xC0 | (c >> 6)));
        o.push_back((char)(0x80 | (c & 0x3F)));
    } else if (c < 0x10000) {
        o.push_back((char)(0xE0 | (c >> 12)));
        o.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
        o.push_back((char)(0x80 | (c & 0x3F)));
    } else {
        o.push_back((char)(0xF0 | (c >> 18)));
        o.push_back((char)(0x80 | ((c >> 12) & 0x3F)));
        o.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
        o.push_back((char)(0x80 | (c & 0x3F)));
    }
}

// Length of the valid UTF-8 sequence starting at s[i] (1-4), or 0 with
// *bad = the length of its maximal subpart (the longest prefix of a valid
// sequence, at least 1): the Unicode "substitution of maximal subparts"
// that String::from_utf8_lossy follows.  Ranges of well-formed sequences:
// Unicode Table 3-7.
size_t utf8_seq(const unsigned char *s, size_t n, size_t i, size_t *bad)
{
    const unsigned c = s[i];
    size_t need;
    unsigned lo = 0x80, hi = 0xBF;
    if (c < 0x80) return 1;
    if (c >= 0xC2 && c <= 0xDF) need = 1;
    else if (c == 0xE0) { need = 2; lo = 0xA0; }
    else if (c >= 0xE1 && c <= 0xEC) need = 2;
    else if (c == 0xED) { need = 2; hi = 0x9F; }
    else if (c >= 0xEE && c <= 0xEF) need = 2;
    else if (c == 0xF0) { need = 3; lo = 0x90; }
    else if (c >= 0xF1 && c <= 0xF3) need = 3;
    else if (c == 0xF4) { need = 3; hi = 0x8F; }
    else { *bad = 1; return 0; }
    for (size_t k = 1; k <= need; k++) {
        const unsigned b = i + k < n ? s[i + k] : 0x100;   // past the end: no continuation
        const unsigned l = k == 1 ? lo : 0x80, h = k == 1 ? hi : 0xBF;
        if (b < l || b > h) { *bad = k; return 0; }
    }
    return need + 1;
}

// Decodes one UTF-8 scalar (a valid sequence of length len).
uint32_t utf8_get(const unsigned char *s, size_t len)
{
    if (len == 1) return s[0];
    uint32_t c = s[0] & (0x7F >> len);
    for (size_t k = 1; k < len; k++) c = (c << 6) | (s[k] & 0x3F);
    return c;
}

// String::from_utf8_lossy.
std::string utf8_lossy(const std::string &b)
{
    const unsigned char *s = (const unsigned char *)b.data();
    std::string o;
    for (size_t i = 0; i < b.size();) {
        size_t bad = 0;
        const size_t len = utf8_seq(s, b.size(), i, &bad);
        if (len) { o.append(b, i, len); i += len; }
        else { put_utf8(o, 0xFFFD); i += bad; }
    }
    return o;
}

// build_byte_encoder (src/tokenizer/bpe.rs:199-208): bytes 33-126, 161-172 and
// 174-255 map to the code point of the same value; the others, in order, to
// 256, 257, ...  Returned as the inverse: code point -> byte, -1 = unmapped.
std::unordered_map<uint32_t, int> byte_decoder()
{
    std::unordered_map<uint32_t, int> dec;
    bool mapped[256] = {};
    for (int b = 33; b <= 126; b++) mapped[b] = true;
    for (int b = 161; b <= 172; b++) mapped[b] = true;
    for (int b = 174; b <= 255; b++) mapped[b] = true;
    uint32_t n = 0;
    for (int b = 0; b < 256; b++) dec[mapped[b] ? (uint32_t)b : 256u + n++] = b;
    return dec;
}

// The token's text as decode prints it, minus the type and range checks.
std::string decode_token(const std::string &tok, uint32_t model, const std::unordered_map<uint32_t, int> &bdec)
{
    const unsigned char *s = (const unsigned char *)tok.data();
    if (model == GS_TOK_GPT2) {
        // chars -> bytes through the byte decoder (the token is a Rust String,
        // valid UTF-8; chars are its scalars)
        std::string bytes;
        size_t nchar = 0;
        for (size_t i = 0; i < tok.size();) {
            size_t bad = 0;
            size_t len = utf8_seq(s, tok.size(), i, &bad);
            if (!len) len = bad;                        // not UTF-8: the loader's input is
            const uint32_t c = utf8_get(s + i, len);    // always valid; keep going
            nchar++;
            auto it = bdec.find(c);
            if (it != bdec.end()) bytes.push_back((char)it->second);
            i += len;
        }
        return bytes.size() == nchar ? utf8_lossy(bytes) : tok;
    }
    // Llama: U+2581 (E2 96 81) -> ' '
    std::string o;
    for (size_t i = 0; i < tok.size(); i++) {
        if (i + 2 < tok.size() && s[i] == 0xE2 && s[i + 1] == 0x96 && s[i + 2] == 0x81) {
            o.push_back(' ');
            i += 2;
        } else {
            o.push_back((char)s[i]);
        }
    }
    return o;
}

int copy_out(const char *src, size_t n, char *out, size_t cap, size_t *len)
{
    if (len) *len = n;
    if (out && cap) memcpy(out, src, n < cap ? n : cap);
    return GS_OK;
}

} // namespace

extern "C" {

int gs_vocab_create(const char *data, const uint64_t *offsets, size_t n, const uint32_t *types, size_t n_types,
                    uint32_t model, gs_vocab **out)
{
    if (!out || (n && !offsets) || (n_types && !types) || model > GS_TOK_GPT2) return GS_ERR_INVALID;
    *out = nullptr;
    if (n > 0xffffffffull) return GS_ERR_UNSUPPORTED;
    for (size_t i = 0; i < n; i++)
        if (offsets[i + 1] < offsets[i]) return GS_ERR_INVALID;
    if (n && offsets[n] > offsets[0] && !data) return GS_ERR_INVALID;
    gs_vocab *v = new (std::nothrow) gs_vocab();
    if (!v) return GS_ERR_NOMEM;
    try {
        v->model = model;
        const auto bdec = byte_decoder();
        v->off.assign(1, 0);
        v->doff.assign(1, 0);
        v->to_id.reserve(n);
        for (size_t i = 0; i < n; i++) {
            const std::string tok(data + offsets[i], (size_t)(offsets[i + 1] - offsets[i]));
            v->raw += tok;
            v->off.push_back(v->raw.size());
            v->to_id[tok] = (uint32_t)i;                 // collect(): a later duplicate wins
            const uint32_t typ = i < n_types ? types[i] : 0u;
            if (typ != 2 && typ != 3) v->dec += decode_token(tok, model, bdec);   // control/special: ""
            v->doff.push_back(v->dec.size());
        }
    } catch (const std::bad_alloc &) {
        delete v;
        return GS_ERR_NOMEM;
    }
    *out = v;
    return GS_OK;
}

int gs_vocab_destroy(gs_vocab *v)
{
    if (!v) return GS_ERR_INVALID;
    delete v;
    return GS_OK;
}

int gs_vocab_find(const gs_vocab *v, const char *s, size_t len, uint32_t *id)
{
    if (!v || !id || (len && !s)) return GS_ERR_INVALID;
    auto it = v->to_id.find(std::string(s ? s : "", len));
    *id = it == v->to_id.end() ? UINT32_MAX : it->second;
    return GS_OK;
}

int gs_token_decode(const gs_vocab *v, uint32_t id, char *out, size_t cap, size_t *len)
{
    if (!v || (cap && !out)) return GS_ERR_INVALID;
    if ((size_t)id + 1 >= v->doff.size()) return copy_out("", 0, out, cap, len);
    return copy_out(v->dec.data() + v->doff[id], (size_t)(v->doff[id + 1] - v->doff[id]), out, cap, len);
}

int gs_tokens_decode(const gs_vocab *v, const uint32_t *ids, size_t n, char *out, size_t cap, size_t *len)
{
    if (!v || (n && !ids) || (cap && !out)) return GS_ERR_INVALID;
    size_t w = 0;
    for (size_t i = 0; i < n; i++) {
        const uint32_t id = ids[i];
        if ((size_t)id + 1 >= v->doff.size()) continue;
        const size_t a = v->doff[id], m = (size_t)(v->doff[id + 1] - a);
        if (w < cap) memcpy(out + w, v->dec.data() + a, m < cap - w ? m : cap - w);
        w += m;
    }
    if (len) *len = w;
    return GS_OK;
}

int gs_chat_template_detect(const gs_vocab *v, const char *tmpl, uint32_t *kind)
{
    if (!v || !kind) return GS_ERR_INVALID;
    static const struct { const char *mark; uint32_t kind; } by_tmpl[] = {
        {"<|im_start|>", GS_TMPL_CHATML}, {"<|start_header_id|>", GS_TMPL_LLAMA3},
        {"<start_of_turn>", GS_TMPL_GEMMA}, {"<|user|>", GS_TMPL_PHI3}, {"[INST]", GS_TMPL_LLAMA2}};
    static const struct { const char *tok; uint32_t kind; } by_vocab[] = {
        {"<|im_start|>", GS_TMPL_CHATML}, {"<|eot_id|>", GS_TMPL_LLAMA3},
        {"<start_of_turn>", GS_TMPL_GEMMA}, {"<|user|>", GS_TMPL_PHI3}, {"[INST]", GS_TMPL_LLAMA2}};
    if (tmpl)
        for (const auto &m : by_tmpl)
            if (strstr(tmpl, m.mark)) { *kind = m.kind; return GS_OK; }
    for (const auto &m : by_vocab)
        if (v->to_id.count(m.tok)) { *kind = m.kind; return GS_OK; }
    *kind = GS_TMPL_SIMPLE;
    return GS_OK;
}

int gs_stop_tokens(const gs_vocab *v, uint32_t kind, const uint32_t *eos, size_t n_eos, uint32_t *out, size_t cap,
                   size_t *n)
{
    if (!v || !n || (n_eos && !eos) || (cap && !out) || kind > GS_TMPL_SIMPLE) return GS_ERR_INVALID;
    std::vector<uint32_t> stops(eos, eos + n_eos);
    static const char *const chatml[] = {"<|im_end|>", "<|endoftext|>", nullptr};
    static const char *const llama3[] = {"<|eot_id|>", "<|end_of_text|>", nullptr};
    static const char *const gemma[] = {"<end_of_turn>", nullptr};
    static const char *const phi3[] = {"<|end|>", nullptr};
    static const char *const none[] = {nullptr};
    const char *const *extras = kind == GS_TMPL_CHATML ? chatml
                                : kind == GS_TMPL_LLAMA3 ? llama3
                                : kind == GS_TMPL_GEMMA  ? gemma
                                : kind == GS_TMPL_PHI3   ? phi3
                                                         : none;
    for (; *extras; extras++) {
        auto it = v->to_id.find(*extras);
        if (it != v->to_id.end()) stops.push_back(it->second);
    }
    std::sort(stops.begin(), stops.end());
    stops.erase(std::unique(stops.begin(), stops.end()), stops.end());
    *n = stops.size();
    for (size_t i = 0; i < stops.size() && i < cap; i++) out[i] = stops[i];
    return GS_OK;
}

} // extern "C"
