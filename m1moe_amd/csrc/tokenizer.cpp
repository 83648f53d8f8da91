// tokenizer.cpp — the reference's BPE tokenizer on the host
// (Sources/M1MoE/Tokenizer.swift).
//
// Reads a HuggingFace tokenizer.json: model.vocab {piece: id}, model.merges
// ["a b", ...] (rank = position) and model.byte_fallback, which selects the
// mode (:36-62):
//   * byte-level BPE (GPT-2 / OLMoE, byte_fallback absent or false): input
//     bytes become the printable characters of the GPT-2 byte table; words
//     are cut at every space (U+0020), and every word after the first starts
//     with the space's character 'Ġ' (:86-115); decoding maps the token
//     characters back to bytes (:117-130).
//   * SentencePiece BPE (Mistral / Mixtral, byte_fallback true): the text is
//     cut at every space, empty pieces are dropped, each piece gets the '▁'
//     prefix (:134-160); a final symbol missing from the vocabulary is spelled
//     as its UTF-8 bytes <0xNN> (:148-155); decoding drops <s> </s> <unk>
//     <pad> and <|...|> unless asked to keep them, turns <0xNN> into the
//     byte and '▁' into a space (:172-198).
// Both modes merge symbols the same way (:212-228): repeatedly the adjacent
// pair with the lowest merge rank, the leftmost of equal ranks, one merge at
// a time.  Encoding drops a final symbol missing from the vocabulary
// (byte-level) exactly as the reference does; decoding skips unknown ids and
// returns the bytes as UTF-8 when they are valid UTF-8, else read as
// ISO-8859-1 (:128-130, :195-197).
//
// Strings are compared byte for byte.  Swift compares String keys (vocabulary
// and merge pairs) by canonical equivalence and splits merge lines at the
// first space character (a space followed by a combining mark is one
// character there); the two agree on NFC-normalised vocabularies and text
// and on any merge line whose second part does not begin with a combining
// mark.  Host only; no device is touched.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "internal.hpp"
#include "m1moe_hip.h"

using namespace m1moe;

struct m1moe_tokenizer {
    bool sentencepiece = false;
    std::unordered_map<std::string, uint32_t> vocab;
    std::unordered_map<uint32_t, std::string> piece_of;
    std::unordered_map<std::string, int32_t> rank;  // key: a + '\xff' + b
    // The same merges on interned symbols (every vocab piece, merge part and
    // merge result has an id): (a, b) -> (rank, id of a + b), so the BPE loop
    // compares integers; built once after loading.
    std::unordered_map<std::string, int32_t> sym;
    std::vector<std::string> sym_str;
    std::vector<int64_t> sym_vocab;                              // vocab id or -1
    std::unordered_map<uint64_t, std::pair<int32_t, int32_t>> pair;
    int32_t byte_sym[256];     // byte-level: the symbol of each byte's table piece
    int64_t fallback_id[256];  // SentencePiece: the vocab id of "<0xHH>" or -1
};

namespace {

void build_symbols(m1moe_tokenizer& t);

// ---- UTF-8 -----------------------------------------------------------------

void put_utf8(std::string& s, uint32_t c) {
    if (c < 0x80) {
        s.push_back((char)c);
    } else if (c < 0x800) {
        s.push_back((char)(0xC0 | (c >> 6)));
        s.push_back((char)(0x80 | (c & 0x3F)));
    } else if (c < 0x10000) {
        s.push_back((char)(0xE0 | (c >> 12)));
        s.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
        s.push_back((char)(0x80 | (c & 0x3F)));
    } else {
        s.push_back((char)(0xF0 | (c >> 18)));
        s.push_back((char)(0x80 | ((c >> 12) & 0x3F)));
        s.push_back((char)(0x80 | ((c >> 6) & 0x3F)));
        s.push_back((char)(0x80 | (c & 0x3F)));
    }
}

// Length of the well-formed UTF-8 sequence at p (RFC 3629: no overlongs, no
// surrogates, at most U+10FFFF), 0 if there is none; *cp gets the scalar.
size_t utf8_seq(const unsigned char* p, size_t n, uint32_t* cp) {
    if (!n) return 0;
    const unsigned c = p[0];
    if (c < 0x80) return *cp = c, 1;
    size_t len;
    uint32_t v, lo;
    if (c >= 0xC2 && c <= 0xDF) len = 2, v = c & 0x1F, lo = 0x80;
    else if (c >= 0xE0 && c <= 0xEF) len = 3, v = c & 0x0F, lo = 0x800;
    else if (c >= 0xF0 && c <= 0xF4) len = 4, v = c & 0x07, lo = 0x10000;
    else return 0;
    if (n < len) return 0;
    for (size_t i = 1; i < len; ++i) {
        if ((p[i] & 0xC0) != 0x80) return 0;
        v = (v << 6) | (p[i] & 0x3F);
    }
    if (v < lo || v > 0x10FFFF || (v >= 0xD800 && v <= 0xDFFF)) return 0;
    *cp = v;
    return len;
}

bool valid_utf8(const std::string& s) {
    const unsigned char* p = (const unsigned char*)s.data();
    size_t i = 0, n = s.size();
    uint32_t cp;
    while (i < n) {
        const size_t l = utf8_seq(p + i, n - i, &cp);
        if (!l) return false;
        i += l;
    }
    return true;
}

// The scalars of valid UTF-8 text, each as its own UTF-8 string.
std::vector<std::string> scalars(const std::string& s) {
    std::vector<std::string> out;
    const unsigned char* p = (const unsigned char*)s.data();
    size_t i = 0;
    uint32_t cp;
    while (i < s.size()) {
        const size_t l = utf8_seq(p + i, s.size() - i, &cp);
        out.emplace_back(s, i, l);
        i += l;
    }
    return out;
}

// ---- the GPT-2 byte table (Tokenizer.swift:232-248) -------------------------
// Bytes 33..126, 161..172 and 174..255 stand for themselves; the other 68
// bytes, in increasing order, get U+0100, U+0101, ... (space -> U+0120 'Ġ').

struct ByteTable {
    std::string enc[256];
    std::unordered_map<std::string, uint8_t> dec;
    ByteTable() {
        uint32_t next = 256;
        for (int b = 0; b < 256; ++b) {
            const bool self = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || b >= 174;
            put_utf8(enc[b], self ? (uint32_t)b : next++);
            dec[enc[b]] = (uint8_t)b;
        }
    }
};

const ByteTable& byte_table() {
    static const ByteTable t;
    return t;
}

const char* const kMeta = "\xE2\x96\x81";  // U+2581 '▁'

// ---- JSON ------------------------------------------------------------------

struct Reader {
    const char* p;
    const char* end;
    std::string err;

    bool bad(const char* what) {
        if (err.empty()) err = what;
        return false;
    }
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < end && *p == c) return ++p, true;
        return false;
    }
    bool hex4(uint32_t& v) {
        if (end - p < 4) return bad("short \\u escape");
        v = 0;
        for (int i = 0; i < 4; ++i, ++p) {
            const char c = *p;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return bad("bad \\u escape");
        }
        return true;
    }
    bool string(std::string& out) {
        out.clear();
        if (!eat('"')) return bad("expected a string");
        while (p < end && *p != '"') {
            if ((unsigned char)*p < 0x20) return bad("control character in a string");
            if (*p != '\\') {
                out.push_back(*p++);
                continue;
            }
            if (++p >= end) break;
            const char e = *p++;
            switch (e) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    uint32_t v;
                    if (!hex4(v)) return false;
                    if (v >= 0xD800 && v <= 0xDBFF) {
                        uint32_t w;
                        if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return bad("lone surrogate");
                        p += 2;
                        if (!hex4(w) || w < 0xDC00 || w > 0xDFFF) return bad("lone surrogate");
                        v = 0x10000 + ((v - 0xD800) << 10) + (w - 0xDC00);
                    } else if (v >= 0xDC00 && v <= 0xDFFF) {
                        return bad("lone surrogate");
                    }
                    put_utf8(out, v);
                    break;
                }
                default: return bad("bad escape");
            }
        }
        if (p >= end) return bad("unterminated string");
        ++p;
        return valid_utf8(out) || bad("string is not UTF-8");
    }
    bool number(double& v) {
        ws();
        const char* q = p;
        if (q < end && *q == '-') ++q;
        while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' ||
                           *q == '+' || *q == '-'))
            ++q;
        if (q == p) return bad("expected a number");
        const std::string t(p, q);
        char* e = nullptr;
        v = std::strtod(t.c_str(), &e);
        if (!e || *e) return bad("bad number");
        p = q;
        return true;
    }
    bool literal(const char* w) {
        const size_t n = std::strlen(w);
        if ((size_t)(end - p) >= n && !std::strncmp(p, w, n)) return p += n, true;
        return false;
    }
    // kind of the next value: '"', '{', '[', 'n' (number), 't', 'f', 'z' (null)
    char next() {
        ws();
        if (p >= end) return 0;
        const char c = *p;
        if (c == '"' || c == '{' || c == '[') return c;
        if (c == 't' || c == 'f') return c;
        if (c == 'n') return 'z';
        return 'n';
    }
    bool skip(int depth = 0) {
        if (depth > 512) return bad("nesting too deep");
        const char k = next();
        std::string s;
        double d;
        switch (k) {
            case '"': return string(s);
            case 't': return literal("true") || bad("bad literal");
            case 'f': return literal("false") || bad("bad literal");
            case 'z': return literal("null") || bad("bad literal");
            case 'n': return number(d);
            case '{':
            case '[': {
                const char close = k == '{' ? '}' : ']';
                ++p;
                if (eat(close)) return true;
                do {
                    if (k == '{' && !(string(s) && (eat(':') || bad("expected ':'")))) return false;
                    if (!skip(depth + 1)) return false;
                } while (eat(','));
                return eat(close) || bad("expected ',' or a closing bracket");
            }
            default: return bad("expected a value");
        }
    }
    // for each member of an object: f(key) reads or skips the value
    template <class F>
    bool members(F f) {
        if (!eat('{')) return bad("expected an object");
        if (eat('}')) return true;
        std::string key;
        do {
            if (!string(key) || !(eat(':') || bad("expected ':'"))) return false;
            if (!f(key)) return false;
        } while (eat(','));
        return eat('}') || bad("expected ',' or '}'");
    }
};

// merge line -> (a, b): split at the first space after the leading spaces,
// as Swift's split(separator: " ", maxSplits: 1) does (leading separators
// produce no part; the second part keeps any further spaces).  False when
// there are not two parts.
bool split_merge(const std::string& m, std::string& a, std::string& b) {
    size_t i = 0;
    while (i < m.size() && m[i] == ' ') ++i;
    const size_t sp = m.find(' ', i);
    if (sp == std::string::npos || sp + 1 >= m.size()) return false;
    a.assign(m, i, sp - i);
    b.assign(m, sp + 1, std::string::npos);
    return true;
}

int32_t parse(const std::string& text, m1moe_tokenizer* t) {
    Reader r{text.data(), text.data() + text.size(), {}};
    bool have_model = false, have_vocab = false, have_merges = false;
    bool bad_vocab = false;
    std::string key, piece, merge, a, b;
    const bool ok = r.members([&](const std::string& k) {
        if (k != "model" || r.next() != '{') return r.skip();
        have_model = true;
        // a repeated "model" key: the last one wins, as in a JSON object
        have_vocab = have_merges = false;
        t->vocab.clear();
        t->rank.clear();
        t->sentencepiece = false;
        return r.members([&](const std::string& mk) {
            if (mk == "vocab" && r.next() == '{') {
                have_vocab = true;
                t->vocab.clear();
                return r.members([&](const std::string& pk) {
                    if (r.next() != 'n') return r.skip();  // not a number: skipped (:50-52)
                    double v;
                    if (!r.number(v)) return false;
                    if (v != std::floor(v)) return true;  // not an Int: skipped
                    if (v < 0 || v > 4294967295.0) return bad_vocab = true, r.bad("id out of range");
                    t->vocab[pk] = (uint32_t)v;
                    return true;
                });
            }
            if (mk == "merges" && r.next() == '[') {
                t->rank.clear();
                ++r.p;
                have_merges = true;
                if (r.eat(']')) return true;
                int32_t rank = 0;
                do {
                    if (r.next() != '"') {  // not [String]: invalid format (:40)
                        have_merges = false;
                        if (!r.skip()) return false;
                        continue;
                    }
                    if (!r.string(merge)) return false;
                    if (split_merge(merge, a, b)) t->rank[a + '\xff' + b] = rank;
                    ++rank;
                } while (r.eat(','));
                if (!have_merges) t->rank.clear();
                return r.eat(']') || r.bad("expected ',' or ']'");
            }
            if (mk == "byte_fallback") {
                // `as? Bool ?? false`: true (or the number 1) selects SentencePiece
                const char kind = r.next();
                if (kind == 't') return t->sentencepiece = true, r.skip();
                if (kind == 'n') {
                    double v;
                    if (!r.number(v)) return false;
                    t->sentencepiece = v == 1.0;
                    return true;
                }
                t->sentencepiece = false;
                return r.skip();
            }
            if (mk == "vocab" || mk == "merges") {  // wrong type
                if (mk == "vocab") have_vocab = false;
                else have_merges = false;
            }
            return r.skip();
        });
    });
    if (!ok || (r.ws(), r.p != r.end)) {
        if (bad_vocab) return fail(M1MOE_ERR_INVALID, "tokenizer: vocab id out of the u32 range");
        return fail(M1MOE_ERR_INVALID, "tokenizer: invalid JSON at byte %ld: %s",
                    (long)(r.p - text.data()), r.err.empty() ? "trailing data" : r.err.c_str());
    }
    if (!have_model || !have_vocab || !have_merges)
        return fail(M1MOE_ERR_INVALID, "tokenizer: invalid format (needs model.vocab {piece: id} "
                                       "and model.merges [\"a b\", ...])");
    t->piece_of.clear();
    for (const auto& kv : t->vocab) {
        auto it = t->piece_of.find(kv.second);
        // two pieces with one id: the reference would trap (:54); keep the
        // byte-wise smaller piece so the choice does not depend on hashing
        if (it == t->piece_of.end() || kv.first < it->second) t->piece_of[kv.second] = kv.first;
    }
    build_symbols(*t);
    return M1MOE_OK;
}

// ---- BPE (Tokenizer.swift:212-228) ------------------------------------------

int32_t intern(m1moe_tokenizer& t, const std::string& p) {
    auto it = t.sym.find(p);
    if (it != t.sym.end()) return it->second;
    const int32_t id = (int32_t)t.sym_str.size();
    t.sym.emplace(p, id);
    t.sym_str.push_back(p);
    auto v = t.vocab.find(p);
    t.sym_vocab.push_back(v == t.vocab.end() ? -1 : (int64_t)v->second);
    return id;
}

inline uint64_t pair_key(int32_t a, int32_t b) { return (uint64_t)(uint32_t)a << 32 | (uint32_t)b; }

// The interned form of the loaded vocabulary and merges (see m1moe_tokenizer).
void build_symbols(m1moe_tokenizer& t) {
    t.sym.clear();
    t.sym_str.clear();
    t.sym_vocab.clear();
    t.pair.clear();
    for (const auto& kv : t.vocab) intern(t, kv.first);
    for (const auto& kv : t.rank) {
        const size_t cut = kv.first.find('\xff');  // never inside UTF-8
        const std::string a = kv.first.substr(0, cut), b = kv.first.substr(cut + 1);
        const int32_t ia = intern(t, a), ib = intern(t, b);
        t.pair[pair_key(ia, ib)] = {kv.second, intern(t, a + b)};
    }
    const ByteTable& bt = byte_table();
    char hex[8];
    for (int c = 0; c < 256; ++c) {
        t.byte_sym[c] = intern(t, bt.enc[c]);
        std::snprintf(hex, sizeof hex, "<0x%02X>", c);
        auto it = t.vocab.find(hex);
        t.fallback_id[c] = it == t.vocab.end() ? -1 : (int64_t)it->second;
    }
}

// Tokenizer.swift:212-228: while a pair has a merge, merge the one with the
// lowest rank (the leftmost of equal ranks) and look again.  Negative ids are
// scalars that no merge or vocab piece contains.
void apply_bpe(const m1moe_tokenizer& t, std::vector<int32_t>& syms) {
    while (syms.size() > 1) {
        int32_t best = INT32_MAX, merged = -1;
        size_t at = SIZE_MAX;
        for (size_t i = 0; i + 1 < syms.size(); ++i) {
            if (syms[i] < 0 || syms[i + 1] < 0) continue;
            auto it = t.pair.find(pair_key(syms[i], syms[i + 1]));
            if (it != t.pair.end() && it->second.first < best)
                best = it->second.first, merged = it->second.second, at = i;
        }
        if (at == SIZE_MAX) break;
        syms[at] = merged;
        syms.erase(syms.begin() + (ptrdiff_t)at + 1);
    }
}

// Encoding is a function of the word alone, so each call keeps the ids of the
// words it has seen (bounded; cleared when full).
struct WordCache {
    std::unordered_map<std::string, std::vector<uint32_t>> map;
    const std::vector<uint32_t>* find(const std::string& w) const {
        auto it = map.find(w);
        return it == map.end() ? nullptr : &it->second;
    }
    void put(const std::string& w, std::vector<uint32_t> ids) {
        if (map.size() >= (1u << 16)) map.clear();
        map.emplace(w, std::move(ids));
    }
};

// Words start at each space (the space is the word's first symbol, as
// U+0120); a word's symbols are its bytes' table pieces.  The text is valid
// UTF-8, so a space byte is always the scalar ' '.
void encode_byte_level(const m1moe_tokenizer& t, const std::string& text, std::vector<uint32_t>& ids) {
    WordCache cache;
    std::vector<int32_t> syms;
    std::vector<uint32_t> out;
    auto word = [&](size_t b, size_t e) {
        const std::string w = text.substr(b, e - b);
        if (const std::vector<uint32_t>* hit = cache.find(w)) {
            ids.insert(ids.end(), hit->begin(), hit->end());
            return;
        }
        syms.clear();
        for (size_t i = b; i < e; ++i) syms.push_back(t.byte_sym[(unsigned char)text[i]]);
        apply_bpe(t, syms);
        out.clear();
        for (int32_t id : syms)
            if (t.sym_vocab[(size_t)id] >= 0) out.push_back((uint32_t)t.sym_vocab[(size_t)id]);
        ids.insert(ids.end(), out.begin(), out.end());
        cache.put(w, out);
    };
    size_t start = 0;
    for (size_t i = 1; i < text.size(); ++i)
        if (text[i] == ' ' && i > start) {
            word(start, i);
            start = i;
        }
    if (start < text.size()) word(start, text.size());
}

// Words split at spaces (empty ones skipped), each prefixed with U+2581 and
// split into scalars; a final symbol outside the vocab becomes its bytes'
// "<0xHH>" pieces (those present).
void encode_sentencepiece(const m1moe_tokenizer& t, const std::string& text, std::vector<uint32_t>& ids) {
    WordCache cache;
    std::vector<int32_t> syms;
    std::vector<std::string> unknown;  // the scalars behind negative ids
    std::vector<uint32_t> out;
    size_t start = 0;
    for (;;) {
        const size_t sp = text.find(' ', start);
        const size_t end = sp == std::string::npos ? text.size() : sp;
        if (end > start) {
            const std::string w = text.substr(start, end - start);
            if (const std::vector<uint32_t>* hit = cache.find(w)) {
                ids.insert(ids.end(), hit->begin(), hit->end());
            } else {
                syms.clear();
                unknown.clear();
                for (std::string& ch : scalars(kMeta + w)) {
                    auto it = t.sym.find(ch);
                    if (it != t.sym.end()) {
                        syms.push_back(it->second);
                    } else {
                        unknown.push_back(std::move(ch));
                        syms.push_back(-(int32_t)unknown.size());
                    }
                }
                apply_bpe(t, syms);
                out.clear();
                for (int32_t id : syms) {
                    if (id >= 0 && t.sym_vocab[(size_t)id] >= 0) {
                        out.push_back((uint32_t)t.sym_vocab[(size_t)id]);
                        continue;
                    }
                    const std::string& p = id >= 0 ? t.sym_str[(size_t)id] : unknown[(size_t)(-id - 1)];
                    for (unsigned char c : p)  // byte fallback
                        if (t.fallback_id[c] >= 0) out.push_back((uint32_t)t.fallback_id[c]);
                }
                ids.insert(ids.end(), out.begin(), out.end());
                cache.put(w, out);
            }
        }
        if (sp == std::string::npos) break;
        start = sp + 1;
    }
}

bool sp_special(const std::string& p) {
    if (p == "<s>" || p == "</s>" || p == "<unk>" || p == "<pad>") return true;
    return p.size() >= 2 && p.compare(0, 2, "<|") == 0 && p.compare(p.size() - 2, 2, "|>") == 0;
}

int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

// "<0xNN>" -> byte, as `tok.count == 6` and UInt8(hex, radix: 16) accept it
// (two hex digits, or a sign and one digit: "+F" is 15, "-0" is 0).
int byte_piece(const std::string& p) {
    if (p.size() != 6 || p.compare(0, 3, "<0x") != 0 || p[5] != '>') return -1;
    const char c0 = p[3], c1 = p[4];
    const int h1 = hexval(c1);
    if (h1 < 0) return -1;
    if (c0 == '+') return h1;
    if (c0 == '-') return h1 == 0 ? 0 : -1;
    const int h0 = hexval(c0);
    return h0 < 0 ? -1 : h0 * 16 + h1;
}

std::string decode_bytes(const m1moe_tokenizer& t, const uint32_t* ids, uint64_t n, bool skip_special) {
    std::string bytes;
    if (!t.sentencepiece) {
        const ByteTable& bt = byte_table();
        for (uint64_t i = 0; i < n; ++i) {
            auto it = t.piece_of.find(ids[i]);
            if (it == t.piece_of.end()) continue;
            for (const std::string& ch : scalars(it->second)) {
                auto jt = bt.dec.find(ch);
                if (jt != bt.dec.end()) bytes.push_back((char)jt->second);
            }
        }
        return bytes;
    }
    for (uint64_t i = 0; i < n; ++i) {
        auto it = t.piece_of.find(ids[i]);
        if (it == t.piece_of.end()) continue;
        const std::string& p = it->second;
        if (sp_special(p)) {
            if (!skip_special) bytes += p;
            continue;
        }
        const int b = byte_piece(p);
        if (b >= 0) {
            bytes.push_back((char)b);
            continue;
        }
        size_t s = 0;
        for (size_t m; (m = p.find(kMeta, s)) != std::string::npos; s = m + 3) {
            bytes.append(p, s, m - s);
            bytes.push_back(' ');
        }
        bytes.append(p, s, std::string::npos);
    }
    return bytes;
}

}  // namespace

extern "C" {

int32_t m1moe_tokenizer_load(const char* path, m1moe_tokenizer_t* out) {
    if (!path || !out) return fail(M1MOE_ERR_INVALID, "tokenizer_load: null argument");
    *out = nullptr;
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(M1MOE_ERR_INVALID, "tokenizer_load: cannot read %s", path);
    std::stringstream ss;
    ss << f.rdbuf();
    auto* t = new m1moe_tokenizer();
    const int32_t rc = parse(ss.str(), t);
    if (rc) {
        delete t;
        return rc;
    }
    *out = t;
    return M1MOE_OK;
}

void m1moe_tokenizer_free(m1moe_tokenizer_t tok) { delete tok; }

int32_t m1moe_tokenizer_info(m1moe_tokenizer_t tok, int32_t* sentencepiece, uint64_t* vocab_size,
                             uint64_t* merges) {
    if (!tok) return fail(M1MOE_ERR_INVALID, "tokenizer_info: null tokenizer");
    if (sentencepiece) *sentencepiece = tok->sentencepiece ? 1 : 0;
    if (vocab_size) *vocab_size = tok->vocab.size();
    if (merges) *merges = tok->rank.size();
    return M1MOE_OK;
}

int32_t m1moe_tokenizer_encode(m1moe_tokenizer_t tok, const char* text, uint64_t text_len,
                               int32_t add_bos, uint32_t bos, uint32_t* ids, uint64_t cap,
                               uint64_t* n_ids) {
    if (!tok || !n_ids || (text_len && !text))
        return fail(M1MOE_ERR_INVALID, "tokenizer_encode: null argument");
    const std::string s(text ? text : "", text_len);
    if (!valid_utf8(s)) return fail(M1MOE_ERR_INVALID, "tokenizer_encode: text is not UTF-8");
    std::vector<uint32_t> v;
    if (add_bos) v.push_back(bos);
    if (!s.empty()) {
        if (tok->sentencepiece) encode_sentencepiece(*tok, s, v);
        else encode_byte_level(*tok, s, v);
    }
    *n_ids = v.size();
    if (!ids) return M1MOE_OK;  // size query
    if (cap < v.size())
        return fail(M1MOE_ERR_INVALID, "tokenizer_encode: %llu ids do not fit in %llu",
                    (unsigned long long)v.size(), (unsigned long long)cap);
    if (!v.empty()) std::memcpy(ids, v.data(), v.size() * 4);
    return M1MOE_OK;
}

int32_t m1moe_tokenizer_decode(m1moe_tokenizer_t tok, const uint32_t* ids, uint64_t n,
                               int32_t skip_special, char* out, uint64_t cap, uint64_t* out_len) {
    if (!tok || !out_len || (n && !ids))
        return fail(M1MOE_ERR_INVALID, "tokenizer_decode: null argument");
    std::string bytes = decode_bytes(*tok, ids, n, skip_special != 0);
    if (!valid_utf8(bytes)) {  // read as ISO-8859-1: byte b is U+00bb
        std::string latin;
        for (unsigned char c : bytes) put_utf8(latin, c);
        bytes.swap(latin);
    }
    *out_len = bytes.size();
    if (!out) return M1MOE_OK;  // size query
    if (cap < bytes.size())
        return fail(M1MOE_ERR_INVALID, "tokenizer_decode: %llu bytes do not fit in %llu",
                    (unsigned long long)bytes.size(), (unsigned long long)cap);
    std::memcpy(out, bytes.data(), bytes.size());
    if (cap > bytes.size()) out[bytes.size()] = 0;
    return M1MOE_OK;
}

}  // extern "C"
