// Byte-level BPE tokenizer (the reference's Tokenizer::encode / decode, tokenizer.rs:94-116, which
// call the HF `tokenizers` crate on aideen-backbone/tokenizer.json: GPT-2's byte-level BPE).
// Restated from the published algorithm of that configuration:
//   - added tokens (here <|endoftext|>) are cut out of the text first and map to their ids;
//   - the ByteLevel pre-tokenizer splits the rest with the GPT-2 pattern
//       's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
//     (first alternative that matches at the current position, each one greedy; \s is the Unicode
//     White_Space property), and maps every byte of a piece to a printable character
//     (bytes_to_unicode: 33..126, 161..172, 174..255 map to themselves, the other 68 bytes to
//     256 + n in byte order);
//   - BPE: starting from one symbol per byte, the adjacent pair with the lowest merge rank is
//     merged (leftmost first among equal pairs) until no pair has a rank;
//   - decode (skip_special_tokens = true) drops special ids, maps each token's characters back to
//     bytes (a token with a character outside the byte map contributes its own UTF-8) and
//     decodes the bytes as UTF-8 with every maximal invalid subsequence replaced by U+FFFD.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "aideen_hip.h"
#include "unicode_tables.h"

namespace adn {
void set_error(const std::string &msg);
}

namespace {

// ---------------------------------------------------------------------------------------------
// a small JSON reader (objects, arrays, strings with escapes, numbers, literals)
// ---------------------------------------------------------------------------------------------
struct JVal {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;
    const JVal *get(const char *key) const {
        if (kind != OBJ) return nullptr;
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

void put_utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xC0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        out += (char)(0xE0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    } else {
        out += (char)(0xF0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3F));
        out += (char)(0x80 | ((cp >> 6) & 0x3F));
        out += (char)(0x80 | (cp & 0x3F));
    }
}

struct JParser {
    const char *p, *e;
    std::string err;
    void ws() {
        while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool fail(const char *m) {
        if (err.empty()) err = m;
        return false;
    }
    bool hex4(uint32_t &v) {
        if (e - p < 4) return fail("bad \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return fail("bad \\u escape");
        }
        return true;
    }
    bool string(std::string &out) {
        if (p >= e || *p != '"') return fail("expected string");
        ++p;
        while (p < e && *p != '"') {
            if (*p != '\\') {
                out += *p++;
                continue;
            }
            if (++p >= e) return fail("bad escape");
            const char c = *p++;
            switch (c) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                        const char *save = p;
                        p += 2;
                        uint32_t lo;
                        if (hex4(lo) && lo >= 0xDC00 && lo < 0xE000)
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        else
                            p = save;
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: return fail("bad escape");
            }
        }
        if (p >= e) return fail("unterminated string");
        ++p;
        return true;
    }
    bool value(JVal &v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= e) return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            v.kind = JVal::OBJ;
            ++p;
            ws();
            if (p < e && *p == '}') {
                ++p;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= e || *p != ':') return fail("expected ':'");
                ++p;
                v.obj.emplace_back(std::move(k), JVal());
                if (!value(v.obj.back().second, depth + 1)) return false;
                ws();
                if (p < e && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < e && *p == '}') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            v.kind = JVal::ARR;
            ++p;
            ws();
            if (p < e && *p == ']') {
                ++p;
                return true;
            }
            for (;;) {
                v.arr.emplace_back();
                if (!value(v.arr.back(), depth + 1)) return false;
                ws();
                if (p < e && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < e && *p == ']') {
                    ++p;
                    return true;
                }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = JVal::STR;
            return string(v.str);
        }
        if (e - p >= 4 && !strncmp(p, "null", 4)) {
            p += 4;
            return true;
        }
        if (e - p >= 4 && !strncmp(p, "true", 4)) {
            v.kind = JVal::BOOL;
            v.b = true;
            p += 4;
            return true;
        }
        if (e - p >= 5 && !strncmp(p, "false", 5)) {
            v.kind = JVal::BOOL;
            p += 5;
            return true;
        }
        const char *s = p;
        while (p < e && ((*p && strchr("+-.eE", *p)) || (*p >= '0' && *p <= '9'))) ++p;
        if (p == s) return fail("unexpected character");
        v.kind = JVal::NUM;
        v.num = std::strtod(std::string(s, p).c_str(), nullptr);
        return true;
    }
};

// ---------------------------------------------------------------------------------------------
// character classes and UTF-8
// ---------------------------------------------------------------------------------------------
template <size_t N>
bool in_ranges(const uint32_t (&r)[N][2], uint32_t cp) {
    size_t lo = 0, hi = N;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        if (cp < r[mid][0]) hi = mid;
        else if (cp > r[mid][1]) lo = mid + 1;
        else return true;
    }
    return false;
}
bool is_letter(uint32_t c) {
    if (c < 0x80) return (c | 0x20) >= 'a' && (c | 0x20) <= 'z';
    return in_ranges(kLetterRanges, c);
}
bool is_number(uint32_t c) {
    if (c < 0x80) return c >= '0' && c <= '9';
    return in_ranges(kNumberRanges, c);
}
bool is_space(uint32_t c) {
    if (c < 0x80) return c == ' ' || (c >= 0x9 && c <= 0xD);
    return in_ranges(kSpaceRanges, c);
}

// strict decode of valid UTF-8 into code points and their byte offsets; false on invalid input
bool decode_utf8(const char *s, size_t n, std::vector<uint32_t> &cps, std::vector<uint32_t> &offs) {
    const unsigned char *u = (const unsigned char *)s;
    size_t i = 0;
    while (i < n) {
        const unsigned c = u[i];
        uint32_t cp;
        int len;
        if (c < 0x80) {
            cp = c;
            len = 1;
        } else if (c >= 0xC2 && c <= 0xDF) {
            cp = c & 0x1F;
            len = 2;
        } else if (c >= 0xE0 && c <= 0xEF) {
            cp = c & 0x0F;
            len = 3;
        } else if (c >= 0xF0 && c <= 0xF4) {
            cp = c & 0x07;
            len = 4;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (int k = 1; k < len; ++k) {
            if ((u[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (u[i + k] & 0x3F);
        }
        if ((len == 3 && (cp < 0x800 || (cp >= 0xD800 && cp < 0xE000))) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)))
            return false;
        cps.push_back(cp);
        offs.push_back((uint32_t)i);
        i += len;
    }
    offs.push_back((uint32_t)n);
    return true;
}

// bytes -> UTF-8 text with each maximal invalid subsequence replaced by U+FFFD (the WHATWG /
// Unicode "maximal subpart" practice of String::from_utf8_lossy)
void lossy_utf8(const std::string &b, std::string &out) {
    const unsigned char *u = (const unsigned char *)b.data();
    const size_t n = b.size();
    size_t i = 0;
    while (i < n) {
        const unsigned c = u[i];
        if (c < 0x80) {
            out += (char)c;
            ++i;
            continue;
        }
        int need;
        unsigned lo = 0x80, hi = 0xBF;
        if (c >= 0xC2 && c <= 0xDF) need = 1;
        else if (c == 0xE0) { need = 2; lo = 0xA0; }
        else if (c >= 0xE1 && c <= 0xEC) need = 2;
        else if (c == 0xED) { need = 2; hi = 0x9F; }
        else if (c >= 0xEE && c <= 0xEF) need = 2;
        else if (c == 0xF0) { need = 3; lo = 0x90; }
        else if (c >= 0xF1 && c <= 0xF3) need = 3;
        else if (c == 0xF4) { need = 3; hi = 0x8F; }
        else {
            out += "\xEF\xBF\xBD";
            ++i;
            continue;
        }
        size_t j = i + 1;
        int got = 0;
        while (got < need && j < n) {
            const unsigned t = u[j];
            const unsigned l = got == 0 ? lo : 0x80, h = got == 0 ? hi : 0xBF;
            if (t < l || t > h) break;
            ++j;
            ++got;
        }
        if (got == need) out.append(b, i, j - i);
        else out += "\xEF\xBF\xBD";
        i = j;
    }
}

}  // namespace

struct adn_tokenizer {
    std::vector<std::string> id_to_tok;
    std::unordered_map<std::string, int32_t> tok_to_id;
    std::unordered_map<uint64_t, std::pair<int32_t, int32_t>> merges;  // (a, b) -> (rank, merged id)
    int32_t byte_sym[256];     // symbol id of each byte's character
    int32_t char_byte[512];    // byte of each byte-map character (code point < 512), -1 otherwise
    struct Added {
        std::string content;
        int32_t id;
        bool special;
    };
    std::vector<Added> added;
    std::vector<char> is_special;  // by id
    std::mutex mu;
    std::unordered_map<std::string, std::vector<int32_t>> cache;

    void bpe(const std::string &piece, std::vector<int32_t> &out) {
        {
            std::lock_guard<std::mutex> g(mu);
            auto it = cache.find(piece);
            if (it != cache.end()) {
                out.insert(out.end(), it->second.begin(), it->second.end());
                return;
            }
        }
        std::vector<int32_t> w(piece.size());
        for (size_t i = 0; i < piece.size(); ++i) w[i] = byte_sym[(unsigned char)piece[i]];
        for (;;) {
            int32_t best_rank = INT32_MAX, best_id = -1;
            size_t at = 0;
            for (size_t i = 0; i + 1 < w.size(); ++i) {
                auto it = merges.find(((uint64_t)(uint32_t)w[i] << 32) | (uint32_t)w[i + 1]);
                if (it != merges.end() && it->second.first < best_rank) {
                    best_rank = it->second.first;
                    best_id = it->second.second;
                    at = i;
                }
            }
            if (best_id < 0) break;
            w[at] = best_id;
            w.erase(w.begin() + (long)at + 1);
        }
        out.insert(out.end(), w.begin(), w.end());
        std::lock_guard<std::mutex> g(mu);
        if (cache.size() < 100000) cache.emplace(piece, std::move(w));
    }

    // the ByteLevel pre-tokenizer's pattern over the code points of one added-token-free span
    void pretokenize_encode(const std::string &text, std::vector<int32_t> &ids) {
        std::vector<uint32_t> cp, off;
        cp.reserve(text.size());
        decode_utf8(text.data(), text.size(), cp, off);  // validated by the caller
        const size_t n = cp.size();
        size_t i = 0;
        while (i < n) {
            size_t j = i;
            const uint32_t c = cp[i];
            // 's 't 're 've 'm 'll 'd
            if (c == '\'' && i + 1 < n) {
                const uint32_t a = cp[i + 1], b = i + 2 < n ? cp[i + 2] : 0;
                if (a == 's' || a == 't' || a == 'm' || a == 'd') j = i + 2;
                else if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) j = i + 3;
            }
            if (j == i) {
                const size_t k = (c == ' ' && i + 1 < n) ? i + 1 : i;  // optional single space
                if (is_letter(cp[k])) {
                    j = k;
                    while (j < n && is_letter(cp[j])) ++j;
                } else if (is_number(cp[k])) {
                    j = k;
                    while (j < n && is_number(cp[j])) ++j;
                } else if (!is_space(cp[k])) {
                    j = k;
                    while (j < n && !is_space(cp[j]) && !is_letter(cp[j]) && !is_number(cp[j])) ++j;
                }
            }
            if (j == i) {
                // \s+(?!\S): the whitespace run, minus its last character when a non-space follows
                // (unless that leaves nothing: then \s+ takes the whole run)
                size_t r = i;
                while (r < n && is_space(cp[r])) ++r;
                j = (r < n && r - i > 1) ? r - 1 : r;
            }
            std::string piece = text.substr(off[i], off[j] - off[i]);
            bpe(piece, ids);
            i = j;
        }
    }
};

namespace {

int tok_fail(const std::string &msg) {
    adn::set_error(msg);
    return ADN_E_INVALID;
}

// bytes_to_unicode of the byte-level BPE
void byte_map(uint32_t (&b2c)[256]) {
    int n = 0;
    for (int b = 0; b < 256; ++b) {
        const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
        b2c[b] = printable ? (uint32_t)b : (uint32_t)(256 + n++);
    }
}

}  // namespace

extern "C" {

int adn_tokenizer_load(const char *path, adn_tokenizer **out) {
    if (!path || !out) return tok_fail("null argument");
    *out = nullptr;
    FILE *f = fopen(path, "rb");
    if (!f) return tok_fail(std::string("cannot open ") + path);
    std::string text;
    char buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, k);
    fclose(f);
    JVal root;
    JParser jp{text.data(), text.data() + text.size(), {}};
    if (!jp.value(root, 0)) return tok_fail("tokenizer.json: " + jp.err);
    const JVal *model = root.get("model");
    const JVal *type = model ? model->get("type") : nullptr;
    if (!model || (type && (type->kind != JVal::STR || type->str != "BPE")))
        return tok_fail("tokenizer.json: only a BPE model is supported");
    const JVal *pre = root.get("pre_tokenizer");
    const JVal *pt = pre ? pre->get("type") : nullptr;
    const JVal *aps = pre ? pre->get("add_prefix_space") : nullptr;
    const JVal *ure = pre ? pre->get("use_regex") : nullptr;
    const JVal *norm = root.get("normalizer");
    if (!pt || pt->str != "ByteLevel" || (aps && aps->b) || (ure && ure->kind == JVal::BOOL && !ure->b) ||
        (norm && norm->kind != JVal::NUL))
        return tok_fail("tokenizer.json: only the byte-level pre-tokenizer without prefix space or normalizer is supported");
    for (const char *key : {"continuing_subword_prefix", "end_of_word_suffix"}) {
        const JVal *v = model->get(key);
        if (v && v->kind == JVal::STR && !v->str.empty())
            return tok_fail(std::string("tokenizer.json: ") + key + " is not supported");
    }
    const JVal *im = model->get("ignore_merges");
    if (im && im->kind == JVal::BOOL && im->b) return tok_fail("tokenizer.json: ignore_merges is not supported");
    const JVal *vocab = model->get("vocab");
    const JVal *merges = model->get("merges");
    if (!vocab || vocab->kind != JVal::OBJ || !merges || merges->kind != JVal::ARR)
        return tok_fail("tokenizer.json: model.vocab / model.merges missing");

    adn_tokenizer *t = new adn_tokenizer();
    int32_t max_id = -1;
    for (const auto &kv : vocab->obj) max_id = std::max(max_id, (int32_t)kv.second.num);
    const JVal *added = root.get("added_tokens");
    if (added && added->kind == JVal::ARR)
        for (const auto &a : added->arr)
            if (const JVal *id = a.get("id")) max_id = std::max(max_id, (int32_t)id->num);
    t->id_to_tok.assign((size_t)max_id + 1, std::string());
    t->is_special.assign((size_t)max_id + 1, 0);
    for (const auto &kv : vocab->obj) {
        t->tok_to_id[kv.first] = (int32_t)kv.second.num;
        t->id_to_tok[(size_t)kv.second.num] = kv.first;
    }
    uint32_t b2c[256];
    byte_map(b2c);
    for (int i = 0; i < 512; ++i) t->char_byte[i] = -1;
    for (int b = 0; b < 256; ++b) {
        std::string s;
        put_utf8(s, b2c[b]);
        auto it = t->tok_to_id.find(s);
        if (it == t->tok_to_id.end()) {
            delete t;
            return tok_fail("tokenizer.json: the vocabulary lacks a byte symbol");
        }
        t->byte_sym[b] = it->second;
        t->char_byte[b2c[b]] = b;
    }
    int32_t rank = 0;
    for (const auto &m : merges->arr) {
        std::string a, b;
        if (m.kind == JVal::STR) {
            const size_t sp = m.str.find(' ');
            if (sp == std::string::npos) continue;
            a = m.str.substr(0, sp);
            b = m.str.substr(sp + 1);
        } else if (m.kind == JVal::ARR && m.arr.size() == 2) {
            a = m.arr[0].str;
            b = m.arr[1].str;
        } else {
            continue;
        }
        auto ia = t->tok_to_id.find(a), ib = t->tok_to_id.find(b), im2 = t->tok_to_id.find(a + b);
        if (ia == t->tok_to_id.end() || ib == t->tok_to_id.end() || im2 == t->tok_to_id.end()) {
            delete t;
            return tok_fail("tokenizer.json: a merge refers to tokens outside the vocabulary");
        }
        const uint64_t key = ((uint64_t)(uint32_t)ia->second << 32) | (uint32_t)ib->second;
        if (!t->merges.count(key)) t->merges[key] = {rank, im2->second};
        ++rank;
    }
    if (added && added->kind == JVal::ARR) {
        for (const auto &a : added->arr) {
            const JVal *id = a.get("id"), *content = a.get("content"), *special = a.get("special");
            if (!id || !content || content->str.empty()) continue;
            const int32_t iid = (int32_t)id->num;
            t->added.push_back({content->str, iid, special && special->b});
            t->id_to_tok[(size_t)iid] = content->str;
            t->is_special[(size_t)iid] = special && special->b;
        }
    }
    *out = t;
    return ADN_OK;
}

void adn_tokenizer_free(adn_tokenizer *t) { delete t; }

int32_t adn_tokenizer_vocab_size(const adn_tokenizer *t) { return t ? (int32_t)t->id_to_tok.size() : 0; }

int adn_tokenizer_encode(adn_tokenizer *t, const char *text, int64_t len, int32_t *ids, int64_t cap, int64_t *n) {
    if (!t || (!text && len > 0) || !n || (cap > 0 && !ids) || len < 0 || cap < 0)
        return tok_fail("invalid argument");
    std::vector<uint32_t> cps, offs;
    if (!decode_utf8(text, (size_t)len, cps, offs)) return tok_fail("text is not valid UTF-8");
    const std::string s(text, (size_t)len);
    std::vector<int32_t> out;
    out.reserve(s.size() / 3 + 4);
    size_t pos = 0;
    while (pos < s.size()) {
        // the earliest (then longest) added token at or after pos
        size_t best = std::string::npos, blen = 0;
        int32_t bid = -1;
        for (const auto &a : t->added) {
            const size_t f = s.find(a.content, pos);
            if (f != std::string::npos && (f < best || (f == best && a.content.size() > blen))) {
                best = f;
                blen = a.content.size();
                bid = a.id;
            }
        }
        const size_t stop = best == std::string::npos ? s.size() : best;
        if (stop > pos) t->pretokenize_encode(s.substr(pos, stop - pos), out);
        if (best == std::string::npos) break;
        out.push_back(bid);
        pos = best + blen;
    }
    *n = (int64_t)out.size();
    if ((int64_t)out.size() > cap) {
        adn::set_error("ids buffer too small (the required count is in *n)");
        return ADN_E_CAPACITY;
    }
    if (!out.empty()) std::memcpy(ids, out.data(), out.size() * sizeof(int32_t));
    return ADN_OK;
}

int adn_tokenizer_decode(const adn_tokenizer *t, const int32_t *ids, int64_t count, char *text, int64_t cap,
                         int64_t *len) {
    if (!t || (!ids && count > 0) || !len || count < 0 || cap < 0 || (cap > 0 && !text))
        return tok_fail("invalid argument");
    std::string bytes;
    for (int64_t k = 0; k < count; ++k) {
        const int32_t id = ids[k];
        // ids without a token are skipped, as the HF decode's filter_map does
        if (id < 0 || id >= (int32_t)t->id_to_tok.size() || t->id_to_tok[(size_t)id].empty()) continue;
        if (t->is_special[(size_t)id]) continue;  // skip_special_tokens = true
        const std::string &tok = t->id_to_tok[(size_t)id];
        std::vector<uint32_t> cp, off;
        std::string mapped;
        bool all = decode_utf8(tok.data(), tok.size(), cp, off);
        for (size_t i = 0; all && i < cp.size(); ++i) {
            if (cp[i] >= 512 || t->char_byte[cp[i]] < 0) all = false;
            else mapped += (char)t->char_byte[cp[i]];
        }
        bytes += all ? mapped : tok;
    }
    std::string out;
    lossy_utf8(bytes, out);
    *len = (int64_t)out.size();
    if ((int64_t)out.size() > cap) {
        adn::set_error("text buffer too small (the required length is in *len)");
        return ADN_E_CAPACITY;
    }
    if (!out.empty()) std::memcpy(text, out.data(), out.size());
    return ADN_OK;
}

}  // extern "C"
