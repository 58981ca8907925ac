// Qwen2 byte-level BPE tokenizer on the host (Sources/Tokenizer/Tokenizer.swift:36-462,
// Core.swift:1-559): NFC normalisation, the tokenizer.json Split pattern, BPE by merge rank,
// added tokens matched on the raw text, lossy UTF-8 decoding, a streaming detokenizer, and the
// Qwen3-VL chat templates.
//
// It reads the file written by instantcua_amd/tokenizer.py (`compile`): a directory of tagged
// sections (the vocabulary as raw bytes, the merges with their result ids, the added tokens, the
// split program and its character-class bitmaps, canonical combining classes, canonical
// decompositions and primary compositions).
//
// Pre-tokenizer: the Split pattern is not hand-coded here.  instantcua_amd/split_pattern.py
// lowers the regex of tokenizer.json to a program of six instructions (MATCH, CLASS, SPLIT, JMP,
// AHEAD, NOT_AHEAD; a SPLIT carries the class of the code points that can begin its preferred
// branch, so alternatives that cannot match are skipped without backtracking) with every character class as a two-stage bitmap over the code points;
// `Splitter` runs it by backtracking with a visited set over (instruction, position), which keeps
// Oniguruma's leftmost-first result and bounds the work of one match attempt by
// (program length x bytes explored).
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "icua_tok.h"

namespace {

thread_local std::string g_tok_err;
int tok_fail(const std::string& m) {
    g_tok_err = m;
    return -1;
}

constexpr uint32_t FILE_MAGIC = 0x32544349u;  // "ICT2"
constexpr uint32_t FILE_VERSION = 2;
constexpr uint32_t STAGE1 = 0x110000 >> 8;  // 256-code-point blocks in a two-stage table

struct FileHead {
    uint32_t magic, version, n_sections, reserved;
};
struct SectionEntry {
    char tag[4];
    uint32_t elem_size;
    uint64_t offset, count;
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

// The split program (instantcua_amd/split_pattern.py).
enum : int32_t { OP_MATCH = 0, OP_CLASS = 1, OP_SPLIT = 2, OP_JMP = 3, OP_AHEAD = 4, OP_NOT_AHEAD = 5 };
struct Insn {
    int32_t op, a, b, guard;
};

// Longest piece one match may return, in bytes.  The matcher reads at most this many bytes past a
// match's start, as if the text ended there, so its visited set (MAX_PIECE * n_code bits, n_code
// <= 4096) and its backtracking stack stay bounded, and so does the BPE of one piece.  Hugging
// Face's pre-tokenizer has no such limit: a run of more than 16 KiB that its split pattern takes
// as one piece (e.g. 16 Ki spaces or letters in a row) is cut into pieces of 16 KiB here.
constexpr size_t MAX_PIECE = 16384;

// Per-call state of the matcher: the visited set of one attempt (bit (p - start) * n_code + pc,
// cleared after the attempt up to the highest word it touched) and the backtracking stack.
struct MatchScratch {
    std::vector<uint64_t> seen;
    std::vector<std::pair<int32_t, size_t>> stack;
};

struct Splitter {
    const Insn* code = nullptr;
    uint32_t n_code = 0, n_classes = 0;
    const uint16_t* stage1 = nullptr;  // [n_classes][STAGE1] -> block
    const uint8_t* blocks = nullptr;   // 32 bytes (256 bits, LSB first) per block
    std::vector<uint64_t> ascii;       // [n_classes][2]: the classes on code points below 128

    bool member(int32_t k, uint32_t cp) const {
        if (cp < 128) return (ascii[2 * (size_t)k + (cp >> 6)] >> (cp & 63)) & 1;
        if (cp >= 0x110000) return false;
        const uint8_t* b = blocks + 32 * (size_t)stage1[(size_t)k * STAGE1 + (cp >> 8)];
        return (b[(cp & 255) >> 3] >> (cp & 7)) & 1;
    }

    // End of the leftmost-first match that starts at byte `start`, or `start` when there is none
    // (the compiler rejects patterns that match the empty string); the text is read up to
    // start + MAX_PIECE at most.
    size_t match(const uint8_t* s, size_t start, size_t n, MatchScratch& sc) const {
        n = std::min(n, start + MAX_PIECE);
        size_t top = 0, end = start;
        bool found = false;
        sc.stack.clear();
        sc.stack.emplace_back(0, start);
        while (!found && !sc.stack.empty()) {
            int32_t pc = sc.stack.back().first;
            size_t p = sc.stack.back().second;
            sc.stack.pop_back();
            for (;;) {
                const size_t bit = (p - start) * n_code + (size_t)pc, w = bit >> 6;
                if (w >= sc.seen.size()) sc.seen.resize(std::max(w + 1, 2 * sc.seen.size()), 0);
                const uint64_t m = 1ull << (bit & 63);
                if (sc.seen[w] & m) break;  // explored before from here, without a match
                sc.seen[w] |= m;
                top = std::max(top, w);
                const Insn& in = code[pc];
                if (in.op == OP_MATCH) {
                    end = p;
                    found = true;
                    break;
                }
                if (in.op == OP_SPLIT) {
                    int len;
                    if (in.guard >= 0 && (p >= n || !member(in.guard, decode_cp(s, p, n, &len)))) {
                        pc = in.b;  // no match can begin through a here
                    } else {
                        sc.stack.emplace_back(in.b, p);
                        pc = in.a;
                    }
                    continue;
                }
                if (in.op == OP_JMP) {
                    pc = in.a;
                    continue;
                }
                int len = 0;
                const bool inside = p < n && member(in.a, decode_cp(s, p, n, &len));
                if (in.op == OP_CLASS) {
                    if (!inside) break;
                    p += len;
                } else if (inside != (in.op == OP_AHEAD)) {
                    break;
                }
                ++pc;
            }
        }
        std::fill(sc.seen.begin(), sc.seen.begin() + (std::ptrdiff_t)top + 1, 0ull);
        return end;
    }
};

}  // namespace

struct icua_tok {
    std::vector<uint8_t> file;
    uint32_t n_total = 0, n_merges = 0, n_specials = 0, n_decomp = 0, n_comp = 0;
    size_t n_tok_bytes = 0, n_spec_bytes = 0;
    const uint32_t* tok_off = nullptr;
    const uint8_t* tok_bytes = nullptr;
    const int32_t* byte_tok = nullptr;
    const uint32_t* specials = nullptr;  // (id, offset, len)
    const uint8_t* spec_bytes = nullptr;
    const uint16_t* ccc_stage1 = nullptr;
    const uint8_t* ccc_blocks = nullptr;  // 256 classes per block
    const uint32_t *decomp_keys = nullptr, *decomp_vals = nullptr, *decomp_data = nullptr;
    const uint64_t* comp_keys = nullptr;
    const uint32_t* comp_vals = nullptr;
    Splitter split;
    std::unordered_map<uint64_t, uint64_t> merge;  // (left << 32 | right) -> (rank << 32 | result id)
    int32_t im_start = -1, im_end = -1, end_of_text = -1;

    uint16_t ccc(uint32_t c) const {
        if (c >= 0x110000) return 0;
        return ccc_blocks[(size_t)ccc_stage1[c >> 8] * 256 + (c & 255)];
    }

    // --- NFC (UAX #15: full canonical decomposition, canonical ordering, composition) ---------
    void decompose(uint32_t c, std::vector<uint32_t>& out) const {
        const uint32_t* k = std::lower_bound(decomp_keys, decomp_keys + n_decomp, c);
        if (k != decomp_keys + n_decomp && *k == c) {
            const uint32_t v = decomp_vals[k - decomp_keys];
            for (uint32_t j = 0; j < (v & 31); ++j) out.push_back(decomp_data[(v >> 5) + j]);
        } else {
            out.push_back(c);
        }
    }
    uint32_t compose(uint32_t a, uint32_t b) const {
        const uint64_t key = (uint64_t)a << 21 | b;
        const uint64_t* k = std::lower_bound(comp_keys, comp_keys + n_comp, key);
        return (k != comp_keys + n_comp && *k == key) ? comp_vals[k - comp_keys] : 0;
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


    // --- BPE --------------------------------------------------------------------------------
    // Merges the adjacent pair of lowest rank, leftmost first, until none applies.  The symbols
    // form a linked list and the candidate pairs a min-heap of (rank, left position): a popped
    // pair is still current when its left symbol is alive and the pair there still has that rank
    // (every merge rule has its own rank, so the rank names the pair).  O(n log n) per piece.
    void bpe(const uint8_t* s, size_t n, std::vector<int32_t>& out) const {
        if (n == 0) return;
        std::vector<int32_t> id(n);
        std::vector<int32_t> prv(n), nxt(n);  // -1: none
        for (size_t i = 0; i < n; ++i) {
            id[i] = byte_tok[s[i]];
            prv[i] = (int32_t)i - 1;
            nxt[i] = i + 1 < n ? (int32_t)i + 1 : -1;
        }
        auto rank_of = [&](int32_t a, int32_t b, int32_t* res) -> uint32_t {
            auto it = merge.find((uint64_t)(uint32_t)a << 32 | (uint32_t)b);
            if (it == merge.end()) return UINT32_MAX;
            if (res) *res = (int32_t)(it->second & 0xFFFFFFFFu);
            return (uint32_t)(it->second >> 32);
        };
        std::vector<uint64_t> heap;  // (rank << 32 | left position), smallest on top
        auto push = [&](int32_t i) {
            if (i < 0 || nxt[i] < 0) return;
            const uint32_t r = rank_of(id[i], id[nxt[i]], nullptr);
            if (r == UINT32_MAX) return;
            heap.push_back((uint64_t)r << 32 | (uint32_t)i);
            std::push_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
        };
        for (size_t i = 0; i + 1 < n; ++i) push((int32_t)i);
        std::vector<uint8_t> dead(n, 0);
        while (!heap.empty()) {
            std::pop_heap(heap.begin(), heap.end(), std::greater<uint64_t>());
            const uint64_t top = heap.back();
            heap.pop_back();
            const int32_t i = (int32_t)(uint32_t)top;
            if (dead[i] || nxt[i] < 0) continue;
            int32_t res;
            if (rank_of(id[i], id[nxt[i]], &res) != (uint32_t)(top >> 32)) continue;  // a stale pair
            const int32_t j = nxt[i];
            id[i] = res;
            dead[j] = 1;
            nxt[i] = nxt[j];
            if (nxt[j] >= 0) prv[nxt[j]] = i;
            push(prv[i]);
            push(i);
        }
        for (int32_t i = 0; i >= 0; i = nxt[i]) out.push_back(id[i]);
    }
    // Split's "isolated" behaviour: every match is a piece and so is every gap between matches.
    void encode_segment(const uint8_t* p, size_t n, std::vector<int32_t>& out) const {
        MatchScratch sc;
        size_t gap = 0;
        for (size_t i = 0; i < n;) {
            const size_t e = split.match(p, i, n, sc);
            if (e > i) {
                if (gap < i) bpe(p + gap, i - gap, out);
                bpe(p + i, e - i, out);
                i = gap = e;
            } else {
                int len;
                decode_cp(p, i, n, &len);
                i += len;
            }
        }
        if (gap < n) bpe(p + gap, n - gap, out);
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
        for (uint32_t k = 0; k < n_specials; ++k) {
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
        for (uint32_t k = 0; k < n_specials; ++k)
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
    std::vector<uint8_t> file;
    fseek(f, 0, SEEK_END);
    const long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    file.resize(len > 0 ? (size_t)len : 0);
    const size_t got = len > 0 ? fread(file.data(), 1, (size_t)len, f) : 0;
    fclose(f);
    if (len < (long)sizeof(FileHead) || got != (size_t)len) return tok_fail("truncated tokenizer file");
    const FileHead* head = (const FileHead*)file.data();
    if (head->magic != FILE_MAGIC || head->version != FILE_VERSION)
        return tok_fail("not a compiled tokenizer file of version 2 (magic or version)");
    const size_t size = file.size();
    if (head->n_sections > 64 || sizeof(FileHead) + head->n_sections * sizeof(SectionEntry) > size)
        return tok_fail("tokenizer file: bad section directory");
    const SectionEntry* dir = (const SectionEntry*)(file.data() + sizeof(FileHead));
    // Finds a section by tag and checks its element size and extent; count < 0 is any count.
    std::string err;
    auto section = [&](const char* tag, uint32_t elem, int64_t count, uint64_t* n) -> const uint8_t* {
        for (uint32_t k = 0; k < head->n_sections; ++k) {
            const SectionEntry& e = dir[k];
            if (memcmp(e.tag, tag, 4) != 0) continue;
            const bool fits = e.elem_size == elem && e.offset % 8 == 0 && e.offset <= size &&
                              e.count <= (size - e.offset) / elem && (count < 0 || e.count == (uint64_t)count);
            if (!fits) {
                if (err.empty()) err = std::string("tokenizer file: section ") + tag + " has a bad size";
                return nullptr;
            }
            if (n) *n = e.count;
            return file.data() + e.offset;
        }
        if (err.empty()) err = std::string("tokenizer file: section ") + tag + " is missing";
        return nullptr;
    };
    auto* t = new icua_tok();
    uint64_t n_off = 0, n_tok_bytes = 0, n_merges = 0, n_specials = 0, n_spec_bytes = 0, n_code = 0, n_stage1 = 0,
             n_blocks = 0, n_ccc_blocks = 0, n_dk = 0, n_dv = 0, n_dd = 0, n_ck = 0, n_cv = 0;
    t->tok_off = (const uint32_t*)section("TOFF", 4, -1, &n_off);
    t->tok_bytes = section("TBYT", 1, -1, &n_tok_bytes);
    t->byte_tok = (const int32_t*)section("BYTK", 4, 256, nullptr);
    const uint32_t* merges = (const uint32_t*)section("MRGE", 12, -1, &n_merges);
    t->specials = (const uint32_t*)section("SPEC", 12, -1, &n_specials);
    t->spec_bytes = section("SBYT", 1, -1, &n_spec_bytes);
    t->split.code = (const Insn*)section("PROG", 16, -1, &n_code);
    t->split.stage1 = (const uint16_t*)section("CIDX", 2, -1, &n_stage1);
    t->split.blocks = section("CBIT", 32, -1, &n_blocks);
    t->ccc_stage1 = (const uint16_t*)section("CCCI", 2, STAGE1, nullptr);
    t->ccc_blocks = section("CCCD", 256, -1, &n_ccc_blocks);
    t->decomp_keys = (const uint32_t*)section("DKEY", 4, -1, &n_dk);
    t->decomp_vals = (const uint32_t*)section("DVAL", 4, -1, &n_dv);
    t->decomp_data = (const uint32_t*)section("DDAT", 4, -1, &n_dd);
    t->comp_keys = (const uint64_t*)section("CKEY", 8, -1, &n_ck);
    t->comp_vals = (const uint32_t*)section("CVAL", 4, -1, &n_cv);
    auto bad = [&](const std::string& m) {
        delete t;
        return tok_fail(err.empty() ? "tokenizer file: " + m : err);
    };
    if (!err.empty()) return bad("");
    if (n_off < 1 || n_off - 1 > (uint64_t)INT32_MAX || n_dk != n_dv || n_ck != n_cv || n_code < 1 ||
        n_code > 4096 || n_stage1 % STAGE1 != 0 || n_blocks > 0x10000 || n_merges > UINT32_MAX ||
        n_specials > UINT32_MAX)
        return bad("inconsistent section counts");
    t->n_total = (uint32_t)(n_off - 1);
    t->n_merges = (uint32_t)n_merges;
    t->n_specials = (uint32_t)n_specials;
    t->n_decomp = (uint32_t)n_dk;
    t->n_comp = (uint32_t)n_ck;
    t->n_tok_bytes = n_tok_bytes;
    t->n_spec_bytes = n_spec_bytes;
    for (uint32_t i = 0; i < t->n_total; ++i)
        if (t->tok_off[i] > t->tok_off[i + 1]) return bad("token offsets out of order");
    if (t->tok_off[t->n_total] > n_tok_bytes) return bad("token bytes out of range");
    for (int b = 0; b < 256; ++b)
        if (t->byte_tok[b] < 0 || (uint32_t)t->byte_tok[b] >= t->n_total) return bad("byte token out of range");
    for (uint64_t r = 0; r < n_merges; ++r)
        for (int j = 0; j < 3; ++j)
            if (merges[3 * r + j] >= t->n_total) return bad("merge names a token outside the vocabulary");
    for (uint64_t k = 0; k < n_specials; ++k) {
        const uint32_t* s = t->specials + 3 * k;
        if (s[0] >= t->n_total || s[1] > n_spec_bytes || s[2] > n_spec_bytes - s[1])
            return bad("added token out of range");
    }
    // The program: every jump lands inside it, every class exists, and it ends in MATCH.
    Splitter& sp = t->split;
    sp.n_code = (uint32_t)n_code;
    sp.n_classes = (uint32_t)(n_stage1 / STAGE1);
    for (uint32_t pc = 0; pc < sp.n_code; ++pc) {
        const Insn& in = sp.code[pc];
        const bool jumps_ok = in.a >= 0 && (uint32_t)in.a < sp.n_code && in.b >= 0 && (uint32_t)in.b < sp.n_code;
        const bool class_ok = in.a >= 0 && (uint32_t)in.a < sp.n_classes;
        const bool guard_ok =
            in.guard == -1 || (in.op == OP_SPLIT && in.guard >= 0 && (uint32_t)in.guard < sp.n_classes);
        const bool op_ok = in.op == OP_MATCH || ((in.op == OP_SPLIT || in.op == OP_JMP) && jumps_ok) ||
                           ((in.op == OP_CLASS || in.op == OP_AHEAD || in.op == OP_NOT_AHEAD) && class_ok);
        const bool ok = guard_ok && op_ok;
        if (!ok) return bad("bad split program instruction " + std::to_string(pc));
    }
    if (sp.code[sp.n_code - 1].op != OP_MATCH) return bad("split program does not end in MATCH");
    for (uint64_t k = 0; k < n_stage1; ++k)
        if (sp.stage1[k] >= n_blocks) return bad("class bitmap index out of range");
    for (uint32_t k = 0; k < STAGE1; ++k)
        if (t->ccc_stage1[k] >= n_ccc_blocks) return bad("combining-class index out of range");
    for (uint64_t k = 0; k < n_dk; ++k)
        if ((t->decomp_vals[k] >> 5) + (t->decomp_vals[k] & 31) > n_dd) return bad("decomposition out of range");
    sp.ascii.assign(2 * (size_t)sp.n_classes, 0);
    for (uint32_t k = 0; k < sp.n_classes; ++k)
        for (uint32_t cp = 0; cp < 128; ++cp) {
            const uint8_t* b = sp.blocks + 32 * (size_t)sp.stage1[(size_t)k * STAGE1];
            if ((b[cp >> 3] >> (cp & 7)) & 1) sp.ascii[2 * k + (cp >> 6)] |= 1ull << (cp & 63);
        }
    t->merge.reserve(n_merges * 2);
    for (uint32_t r = 0; r < n_merges; ++r)
        t->merge.emplace((uint64_t)merges[3 * r] << 32 | merges[3 * r + 1], (uint64_t)r << 32 | merges[3 * r + 2]);
    t->file.swap(file);  // the pointers stay valid: swap keeps the buffer
    t->im_start = t->special_id("<|im_start|>");
    t->im_end = t->special_id("<|im_end|>");
    t->end_of_text = t->special_id("<|endoftext|>");
    *out = t;
    return 0;
}

void icua_tok_close(icua_tok* t) { delete t; }

int icua_tok_vocab_size(const icua_tok* t) { return t ? (int)t->n_total : -1; }

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
    if (id < 0 || (uint32_t)id >= t->n_total) {
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
        if (ids[i] < 0 || (uint32_t)ids[i] >= t->n_total) continue;
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
    if (id >= 0 && (uint32_t)id < t->n_total)
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
