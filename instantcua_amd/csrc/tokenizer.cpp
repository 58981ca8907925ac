// Qwen2 byte-level BPE tokenizer on the host (Sources/Tokenizer/Tokenizer.swift:36-462,
// Core.swift:1-559): NFC normalisation, the Qwen2 split pattern as a hand-written scanner, BPE by
// merge rank, added tokens matched on the raw text, lossy UTF-8 decoding, a streaming detokenizer,
// and the Qwen3-VL chat templates.  It reads the file written by instantcua_amd/tokenizer.py
// (`compile`), which holds the vocabulary as raw bytes, the merges with their result ids, the
// added tokens and the Unicode tables (property classes, canonical combining classes, full
// canonical decompositions and primary compositions).
//
// Split pattern (Tokenizer.swift qwen2SplitRegex), leftmost-first at every position:
//   A1 (?i:'s|'t|'re|'ve|'m|'ll|'d)   A2 [^\r\n\p{L}\p{N}]?\p{L}+   A3 \p{N}
//   A4 ' '?[^\s\p{L}\p{N}]+[\r\n]*     A5 \s*[\r\n]+   A6 \s+(?!\S)   A7 \s+
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "icua_tok.h"

namespace {

thread_local std::string g_tok_err;
int tok_fail(const std::string& m) {
    g_tok_err = m;
    return -1;
}

// Property word of a code point: class in bits 0-2, contraction flags, combining class in 8-15.
enum : uint16_t { C_L = 0, C_N = 1, C_O = 2, C_WS = 3, C_SP = 4, C_NL = 5 };
constexpr uint16_t F_C1 = 1 << 4;  // s t m d (case-insensitive): one-letter contractions
constexpr uint16_t F_RV = 1 << 5;  // r v: 're 've
constexpr uint16_t F_E = 1 << 6;   // e
constexpr uint16_t F_LL = 1 << 7;  // l: 'll

constexpr uint32_t MAGIC = 0x31544349u;  // "ICT1"

struct Header {
    uint32_t magic, version, n_total, n_merges, n_specials, n_blocks, n_decomp, n_comp;
    uint64_t off_tok_off, off_tok_bytes, off_byte_tok, off_merges, off_specials, off_spec_bytes, off_uni1, off_uni2,
        off_decomp_keys, off_decomp_vals, off_decomp_data, off_comp_keys, off_comp_vals, size;
};

uint32_t decode_cp(const uint8_t* p, size_t i, size_t n, int* len) {
    const uint8_t b = p[i];
    if (b < 0x80) {
        *len = 1;
        return b;
    }
    int l = b >= 0xF0 ? 4 : b >= 0xE0 ? 3 : 2;
    if (i + l > n) l = (int)(n - i);
    uint32_t c = b & (l == 2 ? 0x1F : l == 3 ? 0x0F : 0x07);
    for (int k = 1; k < l; ++k) c = (c << 6) | (p[i + k] & 0x3F);
    *len = l;
    return c;
}

void append_utf8(uint32_t c, std::string& out) {
    if (c < 0x80) {
        out += (char)c;
    } else if (c < 0x800) {
        out += (char)(0xC0 | (c >> 6));
        out += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
        out += (char)(0xE0 | (c >> 12));
        out += (char)(0x80 | ((c >> 6) & 0x3F));
        out += (char)(0x80 | (c & 0x3F));
    } else {
        out += (char)(0xF0 | (c >> 18));
        out += (char)(0x80 | ((c >> 12) & 0x3F));
        out += (char)(0x80 | ((c >> 6) & 0x3F));
        out += (char)(0x80 | (c & 0x3F));
    }
}

}  // namespace

struct icua_tok {
    std::vector<uint8_t> file;
    const Header* h = nullptr;
    const uint32_t* tok_off = nullptr;
    const uint8_t* tok_bytes = nullptr;
    const int32_t* byte_tok = nullptr;
    const uint32_t* specials = nullptr;  // (id, offset, len)
    const uint8_t* spec_bytes = nullptr;
    const uint16_t *uni1 = nullptr, *uni2 = nullptr;
    const uint32_t *decomp_keys = nullptr, *decomp_vals = nullptr, *decomp_data = nullptr;
    const uint64_t* comp_keys = nullptr;
    const uint32_t* comp_vals = nullptr;
    std::unordered_map<uint64_t, uint64_t> merge;  // (left << 32 | right) -> (rank << 32 | result id)
    int32_t im_start = -1, im_end = -1, end_of_text = -1;

    uint16_t prop(uint32_t c) const {
        if (c >= 0x110000) return C_O;
        return uni2[(size_t)uni1[c >> 8] * 256 + (c & 0xFF)];
    }
    int cls_at(const uint8_t* p, size_t i, size_t n, int* len) const { return prop(decode_cp(p, i, n, len)) & 7; }
    uint16_t ccc(uint32_t c) const { return prop(c) >> 8; }

    // --- NFC (UAX #15: full canonical decomposition, canonical ordering, composition) ---------
    void decompose(uint32_t c, std::vector<uint32_t>& out) const {
        const uint32_t* k = std::lower_bound(decomp_keys, decomp_keys + h->n_decomp, c);
        if (k != decomp_keys + h->n_decomp && *k == c) {
            const uint32_t v = decomp_vals[k - decomp_keys];
            for (uint32_t j = 0; j < (v & 31); ++j) out.push_back(decomp_data[(v >> 5) + j]);
        } else {
            out.push_back(c);
        }
    }
    uint32_t compose(uint32_t a, uint32_t b) const {
        const uint64_t key = (uint64_t)a << 21 | b;
        const uint64_t* k = std::lower_bound(comp_keys, comp_keys + h->n_comp, key);
        return (k != comp_keys + h->n_comp && *k == key) ? comp_vals[k - comp_keys] : 0;
    }
    void nfc(const uint8_t* p, size_t n, std::string& out) const {
        std::vector<uint32_t> d;
        d.reserve(n);
        for (size_t i = 0; i < n;) {
            int l;
            const uint32_t c = decode_cp(p, i, n, &l);
            decompose(c, d);
            i += l;
        }
        // Canonical ordering: stable sort of every run of non-starters by combining class.
        for (size_t i = 0; i < d.size();) {
            if (ccc(d[i]) == 0) {
                ++i;
                continue;
            }
            size_t j = i;
            while (j < d.size() && ccc(d[j]) != 0) ++j;
            std::stable_sort(d.begin() + i, d.begin() + j,
                             [&](uint32_t a, uint32_t b) { return ccc(a) < ccc(b); });
            i = j;
        }
        // Canonical composition: a character joins the last starter unless a character between
        // them has class 0 or a class not below its own.
        std::vector<uint32_t> r;
        r.reserve(d.size());
        int starter = -1, last = 0;
        for (uint32_t c : d) {
            const int cc = ccc(c);
            if (starter >= 0 && (last < cc || last == 0)) {
                const uint32_t comp = compose(r[starter], c);
                if (comp) {
                    r[starter] = comp;
                    continue;
                }
            }
            if (cc == 0) starter = (int)r.size();
            last = cc;
            r.push_back(c);
        }
        for (uint32_t c : r) append_utf8(c, out);
    }

    // --- pre-tokenizer --------------------------------------------------------------------
    size_t scan_class(const uint8_t* p, size_t j, size_t n, int cls) const {
        while (j < n) {
            int l;
            if (cls_at(p, j, n, &l) != cls) return j;
            j += l;
        }
        return j;
    }
    static size_t scan_nl(const uint8_t* p, size_t j, size_t n) {
        while (j < n && (p[j] == '\n' || p[j] == '\r')) ++j;
        return j;
    }
    // A5 / A6 / A7 on the whitespace run starting at i.
    size_t ws_run(const uint8_t* p, size_t i, size_t n) const {
        size_t j = i, last_start = i;
        long last_nl = -1;
        while (j < n) {
            int l;
            const int c = cls_at(p, j, n, &l);
            if (c < C_WS) break;
            if (c == C_NL) last_nl = (long)j;
            last_start = j;
            j += l;
        }
        if (last_nl >= 0) return (size_t)last_nl + 1;  // A5: through the last CR / LF
        if (j == n) return n;                          // A6: the run ends the text
        if (last_start > i) return last_start;         // A6: all but the run's last character
        return j;                                      // A7: one whitespace character
    }
    // A1 after an apostrophe at k - 1: end of the contraction, or 0.
    size_t contraction(const uint8_t* p, size_t k, size_t n) const {
        if (k >= n) return 0;
        int l1;
        const uint16_t p1 = prop(decode_cp(p, k, n, &l1));
        if (p1 & F_C1) return k + l1;
        if (p1 & (F_RV | F_LL)) {
            const size_t k2 = k + l1;
            if (k2 >= n) return 0;
            int l2;
            const uint16_t p2 = prop(decode_cp(p, k2, n, &l2));
            if (((p1 & F_RV) && (p2 & F_E)) || ((p1 & F_LL) && (p2 & F_LL))) return k2 + l2;
        }
        return 0;
    }
    size_t piece_end(const uint8_t* p, size_t i, size_t n) const {
        int l;
        const int c = cls_at(p, i, n, &l);
        const size_t nx = i + l;
        if (c == C_L) return scan_class(p, nx, n, C_L);  // A2, no prefix
        if (c == C_N) return nx;                          // A3
        if (c == C_O) {
            if (p[i] == '\'') {
                const size_t k = contraction(p, i + 1, n);
                if (k) return k;  // A1
            }
            if (nx >= n) return nx;
            int ln;
            const int cn = cls_at(p, nx, n, &ln);
            if (cn == C_L) return scan_class(p, nx + ln, n, C_L);  // A2: prefix + letters
            return scan_nl(p, scan_class(p, nx, n, C_O), n);       // A4
        }
        if (c == C_SP) {
            if (nx >= n) return n;
            int ln;
            const int cn = cls_at(p, nx, n, &ln);
            if (cn == C_L) return scan_class(p, nx + ln, n, C_L);                 // A2: " word"
            if (cn == C_O) return scan_nl(p, scan_class(p, nx + ln, n, C_O), n);  // A4: " +="
            return ws_run(p, i, n);
        }
        if (c == C_WS) {
            if (nx >= n) return n;
            int ln;
            if (cls_at(p, nx, n, &ln) == C_L) return scan_class(p, nx + ln, n, C_L);  // A2: "\tword"
            return ws_run(p, i, n);
        }
        return ws_run(p, i, n);  // CR / LF
    }

    // --- BPE --------------------------------------------------------------------------------
    // Merges the adjacent pair of lowest rank, leftmost first, until none applies.
    void bpe(const uint8_t* s, size_t n, std::vector<int32_t>& out) const {
        std::vector<int32_t> sym(n);
        for (size_t i = 0; i < n; ++i) sym[i] = byte_tok[s[i]];
        auto rank_of = [&](int32_t a, int32_t b, int32_t* res) -> uint32_t {
            auto it = merge.find((uint64_t)(uint32_t)a << 32 | (uint32_t)b);
            if (it == merge.end()) return UINT32_MAX;
            *res = (int32_t)(it->second & 0xFFFFFFFFu);
            return (uint32_t)(it->second >> 32);
        };
        while (sym.size() > 1) {
            uint32_t best = UINT32_MAX;
            size_t bi = 0;
            int32_t bres = -1;
            for (size_t i = 0; i + 1 < sym.size(); ++i) {
                int32_t res;
                const uint32_t r = rank_of(sym[i], sym[i + 1], &res);
                if (r < best) {
                    best = r;
                    bi = i;
                    bres = res;
                }
            }
            if (best == UINT32_MAX) break;
            sym[bi] = bres;
            sym.erase(sym.begin() + bi + 1);
        }
        out.insert(out.end(), sym.begin(), sym.end());
    }
    void encode_segment(const uint8_t* p, size_t n, std::vector<int32_t>& out) const {
        for (size_t i = 0; i < n;) {
            const size_t j = piece_end(p, i, n);
            bpe(p + i, j - i, out);
            i = j;
        }
    }
    void encode_text(const uint8_t* p, size_t n, std::vector<int32_t>& out) const {
        bool ascii = true;
        for (size_t i = 0; i < n && ascii; ++i) ascii = p[i] < 0x80;
        if (ascii) {
            encode_segment(p, n, out);
            return;
        }
        std::string s;
        nfc(p, n, s);
        encode_segment((const uint8_t*)s.data(), s.size(), out);
    }
    // Longest added token at p[q] (its index), or -1.
    int match_special(const uint8_t* p, size_t q, size_t n) const {
        int best = -1;
        uint32_t best_len = 0;
        for (uint32_t k = 0; k < h->n_specials; ++k) {
            const uint32_t len = specials[3 * k + 2];
            if (len <= best_len || len > n - q) continue;
            if (memcmp(spec_bytes + specials[3 * k + 1], p + q, len) == 0) {
                best = (int)k;
                best_len = len;
            }
        }
        return best;
    }
    void encode(const uint8_t* p, size_t n, bool with_specials, std::vector<int32_t>& out) const {
        if (!with_specials) {
            encode_text(p, n, out);
            return;
        }
        size_t seg = 0;
        for (size_t i = 0; i < n;) {
            const int k = match_special(p, i, n);
            if (k < 0) {
                ++i;
                continue;
            }
            if (i > seg) encode_text(p + seg, i - seg, out);
            out.push_back((int32_t)specials[3 * k]);
            i += specials[3 * k + 2];
            seg = i;
        }
        if (seg < n) encode_text(p + seg, n - seg, out);
    }
    int32_t special_id(const char* s) const {
        const size_t n = strlen(s);
        for (uint32_t k = 0; k < h->n_specials; ++k)
            if (specials[3 * k + 2] == n && memcmp(spec_bytes + specials[3 * k + 1], s, n) == 0)
                return (int32_t)specials[3 * k];
        return -1;
    }
};

namespace {

// Lossy UTF-8: each maximal invalid subpart becomes U+FFFD.  With `final` false, a valid but
// incomplete sequence at the end is left undecoded; returns the bytes consumed.
size_t lossy_utf8(const uint8_t* p, size_t n, std::string& out, bool final) {
    size_t i = 0;
    while (i < n) {
        const uint8_t b = p[i];
        if (b < 0x80) {
            out += (char)b;
            ++i;
            continue;
        }
        int need;
        uint8_t lo = 0x80, hi = 0xBF;
        if (b >= 0xC2 && b <= 0xDF) {
            need = 1;
        } else if (b >= 0xE0 && b <= 0xEF) {
            need = 2;
            lo = b == 0xE0 ? 0xA0 : 0x80;
            hi = b == 0xED ? 0x9F : 0xBF;
        } else if (b >= 0xF0 && b <= 0xF4) {
            need = 3;
            lo = b == 0xF0 ? 0x90 : 0x80;
            hi = b == 0xF4 ? 0x8F : 0xBF;
        } else {
            out += "\xEF\xBF\xBD";
            ++i;
            continue;
        }
        int k = 1;
        bool bad = false;
        for (; k <= need; ++k) {
            if (i + k >= n) break;
            const uint8_t c = p[i + k];
            const bool ok = k == 1 ? (c >= lo && c <= hi) : (c >= 0x80 && c <= 0xBF);
            if (!ok) {
                bad = true;
                break;
            }
        }
        if (!bad && k > need) {  // complete
            out.append((const char*)p + i, need + 1);
            i += need + 1;
        } else if (!bad) {  // ran out of bytes: incomplete but valid so far
            if (!final) return i;
            out += "\xEF\xBF\xBD";
            i = n;
        } else {  // the maximal valid prefix p[i .. i + k) is one replacement
            out += "\xEF\xBF\xBD";
            i += k;
        }
    }
    return n;
}

bool valid_utf8(const char* p, size_t n) {
    std::string tmp;
    tmp.reserve(n);
    lossy_utf8((const uint8_t*)p, n, tmp, true);
    return tmp.size() == n && memcmp(tmp.data(), p, n) == 0;
}

int copy_out(const std::vector<int32_t>& v, int32_t* out, size_t cap, size_t* n_out) {
    *n_out = v.size();
    if (v.size() > cap) return tok_fail("output buffer too small: " + std::to_string(v.size()) + " tokens");
    if (!v.empty()) memcpy(out, v.data(), v.size() * sizeof(int32_t));
    return 0;
}

}  // namespace

extern "C" {

const char* icua_tok_last_error(void) { return g_tok_err.c_str(); }

int icua_tok_open(const char* path, icua_tok** out) {
    if (!path || !out) return tok_fail("null argument");
    *out = nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) return tok_fail(std::string("cannot open ") + path);
    auto* t = new icua_tok();
    fseek(f, 0, SEEK_END);
    const long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    t->file.resize(len > 0 ? (size_t)len : 0);
    const size_t got = len > 0 ? fread(t->file.data(), 1, (size_t)len, f) : 0;
    fclose(f);
    if (len < (long)sizeof(Header) || got != (size_t)len) {
        delete t;
        return tok_fail("truncated tokenizer file");
    }
    const Header* h = (const Header*)t->file.data();
    if (h->magic != MAGIC || h->version != 1 || h->size != (uint64_t)len) {
        delete t;
        return tok_fail("not a compiled tokenizer file (magic, version or size)");
    }
    const uint64_t sec[][2] = {{h->off_tok_off, 4ull * (h->n_total + 1)},
                               {h->off_byte_tok, 4ull * 256},
                               {h->off_merges, 12ull * h->n_merges},
                               {h->off_specials, 12ull * h->n_specials},
                               {h->off_uni1, 2ull * 4352},
                               {h->off_uni2, 512ull * h->n_blocks},
                               {h->off_decomp_keys, 4ull * h->n_decomp},
                               {h->off_decomp_vals, 4ull * h->n_decomp},
                               {h->off_comp_keys, 8ull * h->n_comp},
                               {h->off_comp_vals, 4ull * h->n_comp}};
    for (const auto& s : sec)
        if (s[0] % 8 || s[0] + s[1] > (uint64_t)len) {
            delete t;
            return tok_fail("tokenizer file section out of range");
        }
    const uint8_t* b = t->file.data();
    t->h = h;
    t->tok_off = (const uint32_t*)(b + h->off_tok_off);
    t->tok_bytes = b + h->off_tok_bytes;
    t->byte_tok = (const int32_t*)(b + h->off_byte_tok);
    t->specials = (const uint32_t*)(b + h->off_specials);
    t->spec_bytes = b + h->off_spec_bytes;
    t->uni1 = (const uint16_t*)(b + h->off_uni1);
    t->uni2 = (const uint16_t*)(b + h->off_uni2);
    t->decomp_keys = (const uint32_t*)(b + h->off_decomp_keys);
    t->decomp_vals = (const uint32_t*)(b + h->off_decomp_vals);
    t->decomp_data = (const uint32_t*)(b + h->off_decomp_data);
    t->comp_keys = (const uint64_t*)(b + h->off_comp_keys);
    t->comp_vals = (const uint32_t*)(b + h->off_comp_vals);
    if (t->tok_off[h->n_total] > h->off_spec_bytes - h->off_tok_bytes) {
        delete t;
        return tok_fail("token bytes out of range");
    }
    for (uint32_t k = 0; k < 4352; ++k)
        if (t->uni1[k] >= h->n_blocks) {
            delete t;
            return tok_fail("bad Unicode table");
        }
    const uint32_t* m = (const uint32_t*)(b + h->off_merges);
    t->merge.reserve(h->n_merges * 2);
    for (uint32_t r = 0; r < h->n_merges; ++r)
        t->merge.emplace((uint64_t)m[3 * r] << 32 | m[3 * r + 1], (uint64_t)r << 32 | m[3 * r + 2]);
    t->im_start = t->special_id("<|im_start|>");
    t->im_end = t->special_id("<|im_end|>");
    t->end_of_text = t->special_id("<|endoftext|>");
    *out = t;
    return 0;
}

void icua_tok_close(icua_tok* t) { delete t; }

int icua_tok_vocab_size(const icua_tok* t) { return t ? (int)t->h->n_total : -1; }

int32_t icua_tok_special_id(const icua_tok* t, const char* content) {
    return (t && content) ? t->special_id(content) : -1;
}

int icua_tok_encode(const icua_tok* t, const char* text, size_t len, int with_specials, int32_t* out, size_t cap,
                    size_t* n_out) {
    if (!t || (!text && len) || !n_out || (!out && cap)) return tok_fail("null argument");
    if (!valid_utf8(text, len)) return tok_fail("text is not valid UTF-8");
    std::vector<int32_t> v;
    t->encode((const uint8_t*)text, len, with_specials != 0, v);
    return copy_out(v, out, cap, n_out);
}

int icua_tok_encode_chat(const icua_tok* t, const char* system, size_t slen, const char* user, size_t ulen, int32_t* out,
                         size_t cap, size_t* n_out) {
    if (!t || (!system && slen) || (!user && ulen) || !n_out) return tok_fail("null argument");
    if (!valid_utf8(system, slen) || !valid_utf8(user, ulen)) return tok_fail("text is not valid UTF-8");
    std::string s = "<|im_start|>system\n";
    s.append(system, slen);
    s += "<|im_end|>\n<|im_start|>user\n";
    s.append(user, ulen);
    s += "<|im_end|>\n<|im_start|>assistant\n";
    std::vector<int32_t> v;
    t->encode((const uint8_t*)s.data(), s.size(), true, v);
    return copy_out(v, out, cap, n_out);
}

int icua_tok_encode_vision_chat(const icua_tok* t, const char* system, size_t slen, const char* user, size_t ulen,
                                int num_image_tokens, int32_t* out, size_t cap, size_t* n_out, int* image_offset) {
    if (!t || (!system && slen) || (!user && ulen) || !n_out || !image_offset || num_image_tokens < 0)
        return tok_fail("bad argument");
    if (!valid_utf8(system, slen) || !valid_utf8(user, ulen)) return tok_fail("text is not valid UTF-8");
    std::string pre = "<|im_start|>system\n";
    pre.append(system, slen);
    pre += "<|im_end|>\n<|im_start|>user\n";
    std::string suf(user, ulen);
    suf += "<|im_end|>\n<|im_start|>assistant\n";
    std::vector<int32_t> v;
    t->encode((const uint8_t*)pre.data(), pre.size(), true, v);
    *image_offset = (int)v.size() + 1;
    v.push_back(ICUA_TOK_VISION_START);
    v.insert(v.end(), (size_t)num_image_tokens, ICUA_TOK_IMAGE_PAD);
    v.push_back(ICUA_TOK_VISION_END);
    t->encode((const uint8_t*)suf.data(), suf.size(), true, v);
    return copy_out(v, out, cap, n_out);
}

int icua_tok_token_bytes(const icua_tok* t, int32_t id, const uint8_t** bytes, size_t* len) {
    if (!t || !bytes || !len) return tok_fail("null argument");
    if (id < 0 || (uint32_t)id >= t->h->n_total) {
        *bytes = nullptr;
        *len = 0;
        return 0;
    }
    *bytes = t->tok_bytes + t->tok_off[id];
    *len = t->tok_off[id + 1] - t->tok_off[id];
    return 0;
}

int icua_tok_decode(const icua_tok* t, const int32_t* ids, size_t n, char* out, size_t cap, size_t* n_out) {
    if (!t || (!ids && n) || !n_out) return tok_fail("null argument");
    std::string raw, s;
    for (size_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || (uint32_t)ids[i] >= t->h->n_total) continue;
        raw.append((const char*)t->tok_bytes + t->tok_off[ids[i]], t->tok_off[ids[i] + 1] - t->tok_off[ids[i]]);
    }
    lossy_utf8((const uint8_t*)raw.data(), raw.size(), s, true);
    *n_out = s.size();
    if (s.size() > cap) return tok_fail("output buffer too small");
    if (!s.empty()) memcpy(out, s.data(), s.size());
    return 0;
}

// Streaming detokenizer: bytes of pushed tokens not yet shown (a valid but incomplete UTF-8
// sequence at the end is held back).
struct icua_tok_stream {
    std::string pending;
};

icua_tok_stream* icua_tok_stream_new(void) { return new icua_tok_stream(); }
void icua_tok_stream_free(icua_tok_stream* s) { delete s; }

int icua_tok_stream_push(const icua_tok* t, icua_tok_stream* s, int32_t id, int final, char* out, size_t cap,
                         size_t* n_out) {
    if (!t || !s || !n_out || (!out && cap)) return tok_fail("null argument");
    const size_t before = s->pending.size();
    if (id >= 0 && (uint32_t)id < t->h->n_total)
        s->pending.append((const char*)t->tok_bytes + t->tok_off[id], t->tok_off[id + 1] - t->tok_off[id]);
    std::string txt;
    const size_t used = lossy_utf8((const uint8_t*)s->pending.data(), s->pending.size(), txt, final != 0);
    *n_out = txt.size();
    if (txt.size() > cap) {  // the stream is left as it was: call again with a larger buffer
        s->pending.resize(before);
        return tok_fail("output buffer too small");
    }
    s->pending.erase(0, used);
    if (!txt.empty()) memcpy(out, txt.data(), txt.size());
    return 0;
}

}  // extern "C"
