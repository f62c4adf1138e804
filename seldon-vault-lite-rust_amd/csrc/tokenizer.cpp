// Exact BPE tokenizer of the frozen model (src/model/tokenizer.rs) and the
// text embedder's string entry point (TextEmbedder::embed, src/model/text.rs:
// 610-626), host code of libsvl_hip.so.
//
// Pipeline (tokenizer.rs:1-14): added tokens are matched in the raw text
// (longest first, then the smaller id); the text between them is one BPE
// word whose characters become their single-character vocabulary ids (space
// replaced by U+2581) or, failing that, the ids of their UTF-8 bytes; merges
// then apply by rank. The reference merges every occurrence of the
// lowest-ranked adjacent pair in one left-to-right pass and repeats
// (tokenizer.rs:497-552); here the same passes run over a linked list of
// symbols with a min-heap of (rank, position) candidates, so a word of n
// symbols costs O(n log n) instead of O(n^2), with identical output: each
// pass drains every live candidate of the lowest rank in position order and
// skips those whose symbols an earlier merge of the pass consumed.
//
// Batches of texts are encoded on several host threads; each text's result
// is the reference's encode of that text.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <string_view>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/svl_hip.h"
#include "host_common.hpp"
#include "json.hpp"

namespace {

using namespace svl;
using json::Doc;
using json::Type;

// tokenizer.rs:25-46
constexpr uint64_t MAX_TOKENIZER_FILE_BYTES = 64ull * 1024 * 1024;
constexpr size_t MAX_VOCAB_ENTRIES = 1000000;
constexpr size_t MAX_MERGES = 1000000;
constexpr size_t MAX_ADDED_TOKENS = 10000;
constexpr size_t MAX_INPUT_BYTES = 1024 * 1024;
constexpr size_t MAX_TOKENS = 262144;
constexpr uint32_t SPACE_MARKER = 0x2581;  // U+2581
constexpr uint32_t MAX_CODEPOINT = 0x110000;
// config.rs MAX_TEXT_TOKENS
constexpr size_t MAX_TEXT_TOKENS = 8192;

// prompt.rs:13-35, in Prompt order (prompt.rs:38-55).
const char *const PROMPT_PREFIX[] = {
    "task: search result | query: ",   "title: none | text: ",
    "task: classification | query: ",  "task: clustering | query: ",
    "task: code retrieval | query: ",   "task: fact checking | query: ",
    "task: sentence similarity | query: ", "task: question answering | query: ",
};

// Open-addressing map from a (left, right) id pair to its merge.
class MergeTable {
public:
    void build(size_t n) {
        size_t cap = 16;
        while (cap < 2 * n + 16) cap <<= 1;
        mask_ = cap - 1;
        keys_.assign(cap, 0);
        rank_.assign(cap, 0);
        merged_.assign(cap, 0);
        used_.assign(cap, 0);
    }
    // false when the pair is already present
    bool insert(uint32_t l, uint32_t r, uint32_t rank, uint32_t merged) {
        const uint64_t k = key(l, r);
        for (size_t i = hash(k);; i = (i + 1) & mask_) {
            if (!used_[i]) {
                used_[i] = 1;
                keys_[i] = k;
                rank_[i] = rank;
                merged_[i] = merged;
                return true;
            }
            if (keys_[i] == k) return false;
        }
    }
    bool find(uint32_t l, uint32_t r, uint32_t &rank, uint32_t &merged) const {
        const uint64_t k = key(l, r);
        for (size_t i = hash(k);; i = (i + 1) & mask_) {
            if (!used_[i]) return false;
            if (keys_[i] == k) {
                rank = rank_[i];
                merged = merged_[i];
                return true;
            }
        }
    }

private:
    static uint64_t key(uint32_t l, uint32_t r) { return ((uint64_t)l << 32) | r; }
    size_t hash(uint64_t k) const {
        k ^= k >> 33;
        k *= 0xff51afd7ed558ccdull;
        k ^= k >> 33;
        k *= 0xc4ceb9fe1a85ec53ull;
        k ^= k >> 33;
        return (size_t)k & mask_;
    }
    size_t mask_ = 0;
    std::vector<uint64_t> keys_;
    std::vector<uint32_t> rank_, merged_;
    std::vector<uint8_t> used_;
};

// Byte trie of the added tokens: the longest token that is a prefix of the
// text, the smallest id among equal contents (tokenizer.rs:336-343, 489-494).
class AddedTrie {
public:
    void add(const std::string &s, uint32_t id) {
        uint32_t node = 0;
        for (unsigned char c : s) {
            const uint64_t k = ((uint64_t)node << 8) | c;
            auto it = edges_.find(k);
            if (it == edges_.end()) {
                terminal_.push_back(-1);
                it = edges_.emplace(k, (uint32_t)(terminal_.size() - 1)).first;
            }
            node = it->second;
        }
        if (terminal_[node] < 0 || (int64_t)id < terminal_[node]) terminal_[node] = id;
        first_[(unsigned char)s[0]] = 1;
    }
    // (id, byte length) of the match at s[0..n); length 0 when none matches.
    std::pair<uint32_t, size_t> match(const char *s, size_t n) const {
        if (!n || !first_[(unsigned char)s[0]]) return {0, 0};
        uint32_t node = 0, best = 0;
        size_t best_len = 0;
        for (size_t i = 0; i < n; ++i) {
            auto it = edges_.find(((uint64_t)node << 8) | (unsigned char)s[i]);
            if (it == edges_.end()) break;
            node = it->second;
            if (terminal_[node] >= 0) {
                best = (uint32_t)terminal_[node];
                best_len = i + 1;
            }
        }
        return {best, best_len};
    }

private:
    std::unordered_map<uint64_t, uint32_t> edges_;
    std::vector<int64_t> terminal_{-1};  // node 0 = root; -1 = no token ends here
    uint8_t first_[256] = {};
};

uint32_t decode_cp(const unsigned char *s, size_t &i) {
    const unsigned char c = s[i];
    if (c < 0x80) {
        i += 1;
        return c;
    }
    if ((c & 0xE0) == 0xC0) {
        const uint32_t cp = ((uint32_t)(c & 0x1F) << 6) | (s[i + 1] & 0x3F);
        i += 2;
        return cp;
    }
    if ((c & 0xF0) == 0xE0) {
        const uint32_t cp =
            ((uint32_t)(c & 0x0F) << 12) | ((uint32_t)(s[i + 1] & 0x3F) << 6) | (s[i + 2] & 0x3F);
        i += 3;
        return cp;
    }
    const uint32_t cp = ((uint32_t)(c & 0x07) << 18) | ((uint32_t)(s[i + 1] & 0x3F) << 12) |
                        ((uint32_t)(s[i + 2] & 0x3F) << 6) | (s[i + 3] & 0x3F);
    i += 4;
    return cp;
}

int encode_cp(uint32_t cp, unsigned char *out) {
    if (cp < 0x80) {
        out[0] = (unsigned char)cp;
        return 1;
    }
    if (cp < 0x800) {
        out[0] = (unsigned char)(0xC0 | (cp >> 6));
        out[1] = (unsigned char)(0x80 | (cp & 0x3F));
        return 2;
    }
    if (cp < 0x10000) {
        out[0] = (unsigned char)(0xE0 | (cp >> 12));
        out[1] = (unsigned char)(0x80 | ((cp >> 6) & 0x3F));
        out[2] = (unsigned char)(0x80 | (cp & 0x3F));
        return 3;
    }
    out[0] = (unsigned char)(0xF0 | (cp >> 18));
    out[1] = (unsigned char)(0x80 | ((cp >> 12) & 0x3F));
    out[2] = (unsigned char)(0x80 | ((cp >> 6) & 0x3F));
    out[3] = (unsigned char)(0x80 | (cp & 0x3F));
    return 4;
}

// parse_byte_token (tokenizer.rs:825-832): "<0xHH>" with u8::from_str_radix
// semantics on the two characters (an optional '+' then hex digits).
bool parse_byte_token(const std::string &t, uint8_t &byte) {
    if (t.size() != 6 || t.compare(0, 3, "<0x") != 0 || t[5] != '>') return false;
    auto hex = [](char c, int &d) {
        if (c >= '0' && c <= '9') d = c - '0';
        else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
        else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
        else return false;
        return true;
    };
    int a, b;
    if (t[3] == '+') {
        if (!hex(t[4], b)) return false;
        byte = (uint8_t)b;
        return true;
    }
    if (!hex(t[3], a) || !hex(t[4], b)) return false;
    byte = (uint8_t)(a * 16 + b);
    return true;
}

struct Scratch {
    std::vector<uint32_t> sym;
    std::vector<uint8_t> alive;
    std::vector<int32_t> prev, next;
    std::vector<std::pair<uint64_t, int32_t>> heap;  // (rank << 32 | pos) min-heap, pos
    std::vector<int32_t> pass;
};

}  // namespace

struct svl_tokenizer {
    std::unordered_map<std::string, uint32_t> vocab;
    std::unordered_map<uint32_t, std::string> id_to_token;
    std::vector<uint32_t> char_ids;  // codepoint -> id where has_char
    std::vector<uint8_t> has_char;
    uint32_t byte_ids[256] = {};
    MergeTable merges;
    AddedTrie added;
    std::unordered_set<uint32_t> special_ids;
    uint32_t unk_id = 0, bos_id = 0, eos_id = 0, max_token_id = 0;
    int64_t pad_id = -1;

    svl_status encode_word(const unsigned char *s, size_t n, std::vector<uint32_t> &ids,
                           Scratch &w) const;
    svl_status encode(const char *text, size_t len, bool add_special,
                      std::vector<uint32_t> &ids, Scratch &w) const;
};

namespace {

// ---- document validation (tokenizer.rs:102-334, 581-824) -----------------------

struct Reader {
    const Doc &d;
    svl_status err(svl_status st, const char *fmt, const std::string &a = "") {
        return fail(st, fmt, a.c_str());
    }
    // Member `key` of object node `obj`; CORRUPT "<missing>" when absent.
    svl_status member(uint32_t obj, const char *key, const char *missing, uint32_t &out) {
        out = d.get(obj, key);
        if (out == UINT32_MAX) return fail(SVL_CORRUPT, "%s", missing);
        return SVL_OK;
    }
    svl_status object(uint32_t i, const char *ctx) {
        if (d.type(i) != Type::Object) return fail(SVL_CORRUPT, "tokenizer %s must be a JSON object", ctx);
        return SVL_OK;
    }
    svl_status array(uint32_t i, const char *ctx) {
        if (d.type(i) != Type::Array) return fail(SVL_CORRUPT, "tokenizer %s must be a JSON array", ctx);
        return SVL_OK;
    }
    svl_status string(uint32_t i, const char *ctx, std::string_view &out) {
        if (d.type(i) != Type::String) return fail(SVL_CORRUPT, "tokenizer %s must be a string", ctx);
        out = d.str(i);
        return SVL_OK;
    }
    svl_status boolean(uint32_t i, const char *ctx, bool &out) {
        if (d.type(i) != Type::Bool) return fail(SVL_CORRUPT, "tokenizer %s must be a boolean", ctx);
        out = d.at(i).b;
        return SVL_OK;
    }
    svl_status unsigned_(uint32_t i, const char *ctx, uint64_t &out) {
        if (!d.as_u64(i, out))
            return fail(SVL_CORRUPT, "tokenizer %s must be an unsigned integer", ctx);
        return SVL_OK;
    }
    svl_status null(uint32_t i, const char *ctx) {
        if (d.type(i) != Type::Null) return fail(SVL_UNSUPPORTED, "tokenizer %s is not null", ctx);
        return SVL_OK;
    }
    // A string field that must equal `want` (UNSUPPORTED `msg` otherwise).
    svl_status expect(uint32_t obj, const char *key, const char *missing, const char *ctx,
                      const char *want, const char *msg) {
        uint32_t v;
        ST_TRY(member(obj, key, missing, v));
        std::string_view s;
        ST_TRY(string(v, ctx, s));
        if (s != want) return fail(SVL_UNSUPPORTED, "%s", msg);
        return SVL_OK;
    }
};

svl_status validate_normalizer(Reader &r, uint32_t v) {
    ST_TRY(r.object(v, "normalizer"));
    ST_TRY(r.expect(v, "type", "normalizer is missing type", "normalizer.type", "Replace",
                    "tokenizer normalizer is not a Replace normalizer"));
    uint32_t p;
    ST_TRY(r.member(v, "pattern", "normalizer is missing pattern", p));
    ST_TRY(r.object(p, "normalizer.pattern"));
    ST_TRY(r.expect(p, "String", "normalizer pattern is missing String", "normalizer.pattern.String",
                    " ", "tokenizer normalizer does not replace a space"));
    return r.expect(v, "content", "normalizer is missing content", "normalizer.content",
                    "\xE2\x96\x81", "tokenizer normalizer does not use the expected space marker");
}

svl_status validate_pre_tokenizer(Reader &r, uint32_t v) {
    ST_TRY(r.object(v, "pre_tokenizer"));
    ST_TRY(r.expect(v, "type", "pre_tokenizer is missing type", "pre_tokenizer.type", "Split",
                    "tokenizer pre_tokenizer is not a Split pre-tokenizer"));
    uint32_t p;
    ST_TRY(r.member(v, "pattern", "pre_tokenizer is missing pattern", p));
    ST_TRY(r.object(p, "pre_tokenizer.pattern"));
    ST_TRY(r.expect(p, "String", "pre_tokenizer pattern is missing String",
                    "pre_tokenizer.pattern.String", " ",
                    "tokenizer pre_tokenizer does not split on a space"));
    ST_TRY(r.expect(v, "behavior", "pre_tokenizer is missing behavior", "pre_tokenizer.behavior",
                    "MergedWithPrevious", "tokenizer pre_tokenizer does not use MergedWithPrevious"));
    uint32_t inv;
    ST_TRY(r.member(v, "invert", "pre_tokenizer is missing invert", inv));
    bool b = false;
    ST_TRY(r.boolean(inv, "pre_tokenizer.invert", b));
    if (b) return fail(SVL_UNSUPPORTED, "tokenizer pre_tokenizer is inverted");
    return SVL_OK;
}

svl_status special_token_name(Reader &r, uint32_t part, const char *ctx, std::string_view &out) {
    ST_TRY(r.object(part, ctx));
    uint32_t sp = r.d.get(part, "SpecialToken");
    if (sp == UINT32_MAX) return fail(SVL_CORRUPT, "%s is missing SpecialToken", ctx);
    ST_TRY(r.object(sp, ctx));
    uint32_t id = r.d.get(sp, "id");
    if (id == UINT32_MAX) return fail(SVL_CORRUPT, "%s is missing id", ctx);
    return r.string(id, ctx, out);
}

svl_status validate_post_processor(Reader &r, uint32_t v, const svl_tokenizer &t, uint32_t &bos,
                                   uint32_t &eos) {
    ST_TRY(r.object(v, "post_processor"));
    ST_TRY(r.expect(v, "type", "post_processor is missing type", "post_processor.type",
                    "TemplateProcessing", "tokenizer post_processor is not TemplateProcessing"));
    uint32_t single;
    ST_TRY(r.member(v, "single", "post_processor is missing single", single));
    ST_TRY(r.array(single, "post_processor.single"));
    if (r.d.at(single).count != 3)
        return fail(SVL_UNSUPPORTED, "tokenizer post_processor single template must have three parts");
    uint32_t parts[3], k = 0;
    r.d.each(single, [&](uint32_t, uint32_t val) { parts[k++] = val; });
    std::string_view name;
    ST_TRY(special_token_name(r, parts[0], "post_processor.single[0]", name));
    if (name != "<bos>") return fail(SVL_UNSUPPORTED, "tokenizer post_processor does not prepend <bos>");
    ST_TRY(r.object(parts[1], "post_processor.single[1]"));
    if (r.d.get(parts[1], "Sequence") == UINT32_MAX)
        return fail(SVL_UNSUPPORTED, "tokenizer post_processor middle part is not a Sequence");
    ST_TRY(special_token_name(r, parts[2], "post_processor.single[2]", name));
    if (name != "<eos>") return fail(SVL_UNSUPPORTED, "tokenizer post_processor does not append <eos>");
    auto b = t.vocab.find("<bos>");
    if (b == t.vocab.end()) return fail(SVL_CORRUPT, "tokenizer vocabulary is missing <bos>");
    auto e = t.vocab.find("<eos>");
    if (e == t.vocab.end()) return fail(SVL_CORRUPT, "tokenizer vocabulary is missing <eos>");
    bos = b->second;
    eos = e->second;
    return SVL_OK;
}

svl_status validate_decoder(Reader &r, uint32_t v) {
    ST_TRY(r.object(v, "decoder"));
    ST_TRY(r.expect(v, "type", "decoder is missing type", "decoder.type", "Sequence",
                    "tokenizer decoder is not a Sequence decoder"));
    uint32_t decs;
    ST_TRY(r.member(v, "decoders", "decoder is missing decoders", decs));
    ST_TRY(r.array(decs, "decoder.decoders"));
    if (r.d.at(decs).count != 3)
        return fail(SVL_UNSUPPORTED, "tokenizer decoder chain must have three stages");
    uint32_t st[3], k = 0;
    r.d.each(decs, [&](uint32_t, uint32_t val) { st[k++] = val; });
    ST_TRY(r.object(st[0], "decoder.decoders[0]"));
    ST_TRY(r.expect(st[0], "type", "decoder stage is missing type", "decoder.decoders[0].type",
                    "Replace", "tokenizer decoder first stage is not Replace"));
    uint32_t p;
    ST_TRY(r.member(st[0], "pattern", "decoder Replace is missing pattern", p));
    ST_TRY(r.object(p, "decoder.decoders[0].pattern"));
    ST_TRY(r.expect(p, "String", "decoder Replace pattern is missing String",
                    "decoder.decoders[0].pattern.String", "\xE2\x96\x81",
                    "tokenizer decoder does not replace the space marker"));
    ST_TRY(r.expect(st[0], "content", "decoder Replace is missing content",
                    "decoder.decoders[0].content", " ",
                    "tokenizer decoder does not replace the marker with a space"));
    ST_TRY(r.object(st[1], "decoder.decoders[1]"));
    ST_TRY(r.expect(st[1], "type", "decoder stage is missing type", "decoder.decoders[1].type",
                    "ByteFallback", "tokenizer decoder second stage is not ByteFallback"));
    ST_TRY(r.object(st[2], "decoder.decoders[2]"));
    return r.expect(st[2], "type", "decoder stage is missing type", "decoder.decoders[2].type",
                    "Fuse", "tokenizer decoder third stage is not Fuse");
}

// Tokenizer::from_json (tokenizer.rs:102-334), in its validation order.
svl_status build(const Doc &d, svl_tokenizer &t) {
    Reader r{d};
    const uint32_t root = 0;
    if (d.type(root) != Type::Object) return fail(SVL_CORRUPT, "tokenizer is missing model");
    uint32_t model;
    ST_TRY(r.member(root, "model", "tokenizer is missing model", model));
    ST_TRY(r.object(model, "model"));
    uint32_t v;
    std::string_view s;
    ST_TRY(r.member(model, "type", "tokenizer model is missing type", v));
    ST_TRY(r.string(v, "model.type", s));
    if (s != "BPE")
        return fail(SVL_UNSUPPORTED, "tokenizer model %s; only BPE is implemented",
                    std::string(s).c_str());
    bool b = false;
    ST_TRY(r.member(model, "byte_fallback", "tokenizer model is missing byte_fallback", v));
    ST_TRY(r.boolean(v, "model.byte_fallback", b));
    if (!b) return fail(SVL_UNSUPPORTED, "tokenizer without byte fallback is not supported");
    ST_TRY(r.member(model, "fuse_unk", "tokenizer model is missing fuse_unk", v));
    ST_TRY(r.boolean(v, "model.fuse_unk", b));
    if (!b) return fail(SVL_UNSUPPORTED, "tokenizer with fuse_unk disabled is not supported");
    ST_TRY(r.member(model, "ignore_merges", "tokenizer model is missing ignore_merges", v));
    ST_TRY(r.boolean(v, "model.ignore_merges", b));
    if (b) return fail(SVL_UNSUPPORTED, "tokenizer with ignore_merges enabled is not supported");
    ST_TRY(r.member(model, "continuing_subword_prefix",
                    "tokenizer model is missing continuing_subword_prefix", v));
    ST_TRY(r.null(v, "model.continuing_subword_prefix"));
    ST_TRY(r.member(model, "end_of_word_suffix", "tokenizer model is missing end_of_word_suffix", v));
    ST_TRY(r.null(v, "model.end_of_word_suffix"));
    ST_TRY(r.member(model, "dropout", "tokenizer model is missing dropout", v));
    ST_TRY(r.null(v, "model.dropout"));

    uint32_t vocab;
    ST_TRY(r.member(model, "vocab", "tokenizer model is missing vocab", vocab));
    ST_TRY(r.object(vocab, "model.vocab"));
    const size_t nv = d.at(vocab).count;
    if (nv > MAX_VOCAB_ENTRIES)
        return fail(SVL_LIMIT, "tokenizer vocabulary has %zu entries, above the %zu-entry cap", nv,
                    MAX_VOCAB_ENTRIES);
    t.vocab.reserve(nv * 2);
    t.id_to_token.reserve(nv * 2);
    svl_status st = SVL_OK;
    d.each(vocab, [&](uint32_t key, uint32_t val) {
        if (st != SVL_OK) return;
        uint64_t id;
        if ((st = r.unsigned_(val, "model.vocab id", id)) != SVL_OK) return;
        if (id > UINT32_MAX) {
            st = fail(SVL_LIMIT, "tokenizer vocabulary id does not fit u32");
            return;
        }
        std::string tok(d.str(key));
        if (!t.vocab.emplace(tok, (uint32_t)id).second) {
            st = fail(SVL_CORRUPT, "duplicate tokenizer vocabulary token");
            return;
        }
        if (!t.id_to_token.emplace((uint32_t)id, std::move(tok)).second)
            st = fail(SVL_CORRUPT, "duplicate tokenizer vocabulary id");
    });
    ST_TRY(st);

    t.char_ids.assign(MAX_CODEPOINT, 0);
    t.has_char.assign(MAX_CODEPOINT, 0);
    for (auto &kv : t.vocab) {
        const std::string &tok = kv.first;
        if (tok.empty()) continue;
        size_t i = 0;
        const uint32_t cp = decode_cp((const unsigned char *)tok.data(), i);
        if (i == tok.size()) {
            t.char_ids[cp] = kv.second;
            t.has_char[cp] = 1;
        }
    }
    if (!t.has_char[SPACE_MARKER])
        return fail(SVL_CORRUPT, "tokenizer vocabulary is missing the space marker token");
    for (int byte = 0; byte < 256; ++byte) {
        char name[8];
        snprintf(name, sizeof name, "<0x%02X>", byte);
        auto it = t.vocab.find(name);
        if (it == t.vocab.end())
            return fail(SVL_CORRUPT, "tokenizer vocabulary is missing byte token %s", name);
        t.byte_ids[byte] = it->second;
    }

    uint32_t merges;
    ST_TRY(r.member(model, "merges", "tokenizer model is missing merges", merges));
    ST_TRY(r.array(merges, "model.merges"));
    const size_t nm = d.at(merges).count;
    if (nm > MAX_MERGES)
        return fail(SVL_LIMIT, "tokenizer has %zu merges, above the %zu-merge cap", nm, MAX_MERGES);
    t.merges.build(nm);
    uint32_t rank = 0;
    std::string joined;
    d.each(merges, [&](uint32_t, uint32_t val) {
        if (st != SVL_OK) return;
        if ((st = r.array(val, "model.merges entry")) != SVL_OK) return;
        if (d.at(val).count != 2) {
            st = fail(SVL_CORRUPT, "tokenizer merge must contain exactly two strings");
            return;
        }
        std::string_view left, right;
        if ((st = r.string(val + 1, "merge left", left)) != SVL_OK) return;
        if ((st = r.string(d.at(val + 1).next, "merge right", right)) != SVL_OK) return;
        auto l = t.vocab.find(std::string(left));
        if (l == t.vocab.end()) {
            st = fail(SVL_CORRUPT, "merge left \"%s\" is not in the vocabulary", std::string(left).c_str());
            return;
        }
        auto rr = t.vocab.find(std::string(right));
        if (rr == t.vocab.end()) {
            st = fail(SVL_CORRUPT, "merge right \"%s\" is not in the vocabulary", std::string(right).c_str());
            return;
        }
        joined.assign(left);
        joined.append(right);
        auto m = t.vocab.find(joined);
        if (m == t.vocab.end()) {
            st = fail(SVL_CORRUPT, "merge result \"%s\" is not in the vocabulary", joined.c_str());
            return;
        }
        if (!t.merges.insert(l->second, rr->second, rank, m->second))
            st = fail(SVL_CORRUPT, "duplicate tokenizer merge pair");
        ++rank;
    });
    ST_TRY(st);

    ST_TRY(r.member(model, "unk_token", "tokenizer model is missing unk_token", v));
    ST_TRY(r.string(v, "model.unk_token", s));
    auto unk = t.vocab.find(std::string(s));
    if (unk == t.vocab.end())
        return fail(SVL_CORRUPT, "unknown token \"%s\" is not in the vocabulary", std::string(s).c_str());
    t.unk_id = unk->second;

    uint32_t added;
    ST_TRY(r.member(root, "added_tokens", "tokenizer is missing added_tokens", added));
    ST_TRY(r.array(added, "added_tokens"));
    const size_t na = d.at(added).count;
    if (na > MAX_ADDED_TOKENS)
        return fail(SVL_LIMIT, "tokenizer has %zu added tokens, above the %zu-token cap", na,
                    MAX_ADDED_TOKENS);
    std::unordered_set<uint32_t> seen;
    d.each(added, [&](uint32_t, uint32_t val) {
        if (st != SVL_OK) return;
        if ((st = r.object(val, "added token")) != SVL_OK) return;
        uint32_t f;
        std::string_view content;
        if ((st = r.member(val, "content", "added token is missing content", f)) != SVL_OK) return;
        if ((st = r.string(f, "added token content", content)) != SVL_OK) return;
        if (content.empty()) {
            st = fail(SVL_CORRUPT, "added token content must not be empty");
            return;
        }
        uint64_t id;
        if ((st = r.member(val, "id", "added token is missing id", f)) != SVL_OK) return;
        if ((st = r.unsigned_(f, "added token id", id)) != SVL_OK) return;
        if (id > UINT32_MAX) {
            st = fail(SVL_LIMIT, "added token id does not fit u32");
            return;
        }
        if (!seen.insert((uint32_t)id).second) {
            st = fail(SVL_CORRUPT, "duplicate added token id");
            return;
        }
        if (!t.id_to_token.count((uint32_t)id)) {
            st = fail(SVL_CORRUPT, "added token \"%s\" has id %u outside the vocabulary",
                      std::string(content).c_str(), (unsigned)id);
            return;
        }
        bool special = false;
        if ((st = r.member(val, "special", "added token is missing special", f)) != SVL_OK) return;
        if ((st = r.boolean(f, "added token special", special)) != SVL_OK) return;
        if (special) t.special_ids.insert((uint32_t)id);
        t.added.add(std::string(content), (uint32_t)id);
    });
    ST_TRY(st);

    uint32_t part;
    ST_TRY(r.member(root, "normalizer", "tokenizer is missing normalizer", part));
    ST_TRY(validate_normalizer(r, part));
    ST_TRY(r.member(root, "pre_tokenizer", "tokenizer is missing pre_tokenizer", part));
    ST_TRY(validate_pre_tokenizer(r, part));
    ST_TRY(r.member(root, "post_processor", "tokenizer is missing post_processor", part));
    ST_TRY(validate_post_processor(r, part, t, t.bos_id, t.eos_id));
    ST_TRY(r.member(root, "decoder", "tokenizer is missing decoder", part));
    ST_TRY(validate_decoder(r, part));

    auto pad = t.vocab.find("<pad>");
    t.pad_id = pad == t.vocab.end() ? -1 : (int64_t)pad->second;
    for (auto &kv : t.id_to_token) t.max_token_id = std::max(t.max_token_id, kv.first);
    return SVL_OK;
}

svl_status token_limit(size_t count) {
    if (count > MAX_TOKENS)
        return fail(SVL_LIMIT, "tokenization exceeds the %zu-token cap", MAX_TOKENS);
    return SVL_OK;
}

}  // namespace

// encode_segment (tokenizer.rs:497-538) with the pass-wise heap merge.
svl_status svl_tokenizer::encode_word(const unsigned char *s, size_t n, std::vector<uint32_t> &ids,
                                      Scratch &w) const {
    w.sym.clear();
    for (size_t i = 0; i < n;) {
        uint32_t cp = decode_cp(s, i);
        if (cp == ' ') cp = SPACE_MARKER;
        if (has_char[cp]) {
            w.sym.push_back(char_ids[cp]);
        } else {
            unsigned char buf[4];
            const int k = encode_cp(cp, buf);
            for (int j = 0; j < k; ++j) w.sym.push_back(byte_ids[buf[j]]);
        }
    }
    ST_TRY(token_limit(w.sym.size()));
    const int32_t m = (int32_t)w.sym.size();
    w.prev.resize((size_t)m);
    w.next.resize((size_t)m);
    w.alive.assign((size_t)m, 1);
    for (int32_t i = 0; i < m; ++i) {
        w.prev[(size_t)i] = i - 1;
        w.next[(size_t)i] = i + 1 < m ? i + 1 : -1;
    }
    auto cmp = [](const std::pair<uint64_t, int32_t> &a, const std::pair<uint64_t, int32_t> &b) {
        return a.first > b.first;  // min-heap on (rank << 32 | position)
    };
    w.heap.clear();
    auto consider = [&](int32_t p) {
        if (p < 0) return;
        const int32_t q = w.next[(size_t)p];
        if (q < 0) return;
        uint32_t rank, merged;
        if (merges.find(w.sym[(size_t)p], w.sym[(size_t)q], rank, merged)) {
            w.heap.emplace_back(((uint64_t)rank << 32) | (uint32_t)p, p);
            std::push_heap(w.heap.begin(), w.heap.end(), cmp);
        }
    };
    for (int32_t i = 0; i + 1 < m; ++i) consider(i);
    // a candidate is live when p still starts a pair with that rank
    auto live = [&](int32_t p, uint32_t rank, uint32_t &l, uint32_t &r, uint32_t &merged) {
        if (!w.alive[(size_t)p]) return false;
        const int32_t q = w.next[(size_t)p];
        if (q < 0) return false;
        uint32_t rk;
        if (!merges.find(w.sym[(size_t)p], w.sym[(size_t)q], rk, merged) || rk != rank) return false;
        l = w.sym[(size_t)p];
        r = w.sym[(size_t)q];
        return true;
    };
    while (!w.heap.empty()) {
        std::pop_heap(w.heap.begin(), w.heap.end(), cmp);
        const uint64_t key = w.heap.back().first;
        const int32_t p0 = w.heap.back().second;
        w.heap.pop_back();
        const uint32_t rank = (uint32_t)(key >> 32);
        uint32_t L, R, merged;
        if (!live(p0, rank, L, R, merged)) continue;
        // one pass: every candidate of this rank, in position order
        w.pass.clear();
        w.pass.push_back(p0);
        while (!w.heap.empty() && (uint32_t)(w.heap.front().first >> 32) == rank) {
            std::pop_heap(w.heap.begin(), w.heap.end(), cmp);
            w.pass.push_back(w.heap.back().second);
            w.heap.pop_back();
        }
        size_t done = 0;
        for (int32_t p : w.pass) {
            const int32_t q = w.next[(size_t)p];
            if (!w.alive[(size_t)p] || w.sym[(size_t)p] != L || q < 0 || w.sym[(size_t)q] != R)
                continue;
            w.sym[(size_t)p] = merged;
            w.alive[(size_t)q] = 0;  // consumed
            const int32_t nq = w.next[(size_t)q];
            w.next[(size_t)p] = nq;
            if (nq >= 0) w.prev[(size_t)nq] = p;
            w.pass[done++] = p;
        }
        for (size_t k = 0; k < done; ++k) {
            const int32_t p = w.pass[k];
            if (!w.alive[(size_t)p]) continue;
            consider(w.prev[(size_t)p]);
            consider(p);
        }
    }
    for (int32_t p = 0; p >= 0 && m > 0; p = w.next[(size_t)p]) ids.push_back(w.sym[(size_t)p]);
    return token_limit(ids.size());
}

// Tokenizer::encode (tokenizer.rs:339-389); `text` is valid UTF-8.
svl_status svl_tokenizer::encode(const char *text, size_t len, bool add_special,
                                 std::vector<uint32_t> &ids, Scratch &w) const {
    if (len > MAX_INPUT_BYTES)
        return fail(SVL_LIMIT, "tokenizer input is %zu bytes, above the %zu-byte cap", len,
                    MAX_INPUT_BYTES);
    ids.clear();
    if (add_special) ids.push_back(bos_id);
    const unsigned char *s = (const unsigned char *)text;
    size_t seg = 0, i = 0;
    while (i < len) {
        const auto m = added.match(text + i, len - i);
        if (m.second) {
            if (i > seg) ST_TRY(encode_word(s + seg, i - seg, ids, w));
            ids.push_back(m.first);
            ST_TRY(token_limit(ids.size()));
            i += m.second;
            seg = i;
        } else {
            size_t j = i;
            decode_cp(s, j);
            i = j;
        }
    }
    if (len > seg) ST_TRY(encode_word(s + seg, len - seg, ids, w));
    if (add_special) ids.push_back(eos_id);
    return token_limit(ids.size());
}

namespace {

// Encodes texts[0..n) on up to `threads` host threads; results[i] and
// status[i] per text (the thread-local message copied into messages[i]).
void encode_many(const svl_tokenizer *t, const char *const *texts, const size_t *lens, size_t n,
                 bool add_special, const char *prefix, std::vector<std::vector<uint32_t>> &results,
                 std::vector<svl_status> &status, std::vector<std::string> &messages) {
    results.assign(n, {});
    status.assign(n, SVL_OK);
    messages.assign(n, {});
    const size_t hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t threads = std::min<size_t>({n, hw, 16});
    auto work = [&](size_t begin) {
        Scratch w;
        std::string full;
        for (size_t i = begin; i < n; i += threads) {
            const char *src = texts[i] ? texts[i] : "";
            size_t len = texts[i] ? lens[i] : 0;
            if (lens[i] && !texts[i]) {
                status[i] = fail(SVL_USAGE, "text %zu is null", i);
            } else if (!json::valid_utf8(src, len)) {
                status[i] = fail(SVL_CORRUPT, "text %zu is not valid UTF-8", i);
            } else {
                if (prefix) {
                    full.assign(prefix);
                    full.append(src, len);
                    src = full.data();
                    len = full.size();
                }
                status[i] = t->encode(src, len, add_special, results[i], w);
            }
            if (status[i] != SVL_OK) messages[i] = g_err;
        }
    };
    if (threads <= 1) {
        work(0);
        return;
    }
    std::vector<std::thread> pool;
    for (size_t k = 0; k < threads; ++k) pool.emplace_back(work, k);
    for (auto &th : pool) th.join();
}

}  // namespace

extern "C" {

svl_status svl_tokenizer_create(const char *json_text, size_t len, svl_tokenizer **out) {
    if (!out || (!json_text && len)) return fail(SVL_USAGE, "document and output handle are required");
    *out = nullptr;
    if (len > MAX_TOKENIZER_FILE_BYTES)
        return fail(SVL_LIMIT, "tokenizer file is %zu bytes, above the %llu-byte cap", len,
                    (unsigned long long)MAX_TOKENIZER_FILE_BYTES);
    if (!json::valid_utf8(json_text ? json_text : "", len))
        return fail(SVL_CORRUPT, "tokenizer file is not valid UTF-8");
    // json_limits (tokenizer.rs:569-578)
    const json::Limits lim{(size_t)MAX_TOKENIZER_FILE_BYTES, 64, 1024 * 1024, 600000, 3000000};
    Doc doc;
    std::string err;
    const svl_status st = json::parse(json_text ? json_text : "", len, lim, doc, err);
    if (st != SVL_OK) return fail(st, "%s", err.c_str());
    std::unique_ptr<svl_tokenizer> t(new svl_tokenizer());
    ST_TRY(build(doc, *t));
    *out = t.release();
    return SVL_OK;
}

svl_status svl_tokenizer_destroy(svl_tokenizer *t) {
    delete t;
    return SVL_OK;
}

svl_status svl_tokenizer_encode(const svl_tokenizer *t, const char *text, size_t len,
                                int add_special_tokens, uint32_t *ids, size_t capacity,
                                size_t *count) {
    if (!t || !count || (len && !text)) return fail(SVL_USAGE, "tokenizer, text and count are required");
    std::vector<std::vector<uint32_t>> res;
    std::vector<svl_status> st;
    std::vector<std::string> msg;
    const char *texts[1] = {text};
    const size_t lens[1] = {len};
    encode_many(t, texts, lens, 1, add_special_tokens != 0, nullptr, res, st, msg);
    if (st[0] != SVL_OK) return fail(st[0], "%s", msg[0].c_str());
    *count = res[0].size();
    if (res[0].size() > capacity || (!ids && !res[0].empty()))
        return fail(SVL_USAGE, "output holds %zu ids, %zu needed", capacity, res[0].size());
    std::copy(res[0].begin(), res[0].end(), ids);
    return SVL_OK;
}

svl_status svl_tokenizer_encode_batch(const svl_tokenizer *t, const char *const *texts,
                                      const size_t *lens, int32_t n, int add_special_tokens,
                                      uint32_t *ids, size_t capacity, int64_t *offsets) {
    if (!t || n < 0 || (n > 0 && (!texts || !lens || !offsets)))
        return fail(SVL_USAGE, "tokenizer, texts, lengths and offsets are required");
    std::vector<std::vector<uint32_t>> res;
    std::vector<svl_status> st;
    std::vector<std::string> msg;
    encode_many(t, texts, lens, (size_t)n, add_special_tokens != 0, nullptr, res, st, msg);
    offsets[0] = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (st[(size_t)i] != SVL_OK) return fail(st[(size_t)i], "text %d: %s", i, msg[(size_t)i].c_str());
        offsets[i + 1] = offsets[i] + (int64_t)res[(size_t)i].size();
    }
    if ((size_t)offsets[n] > capacity || (!ids && offsets[n] > 0))
        return fail(SVL_USAGE, "output holds %zu ids, %lld needed", capacity, (long long)offsets[n]);
    for (int32_t i = 0; i < n; ++i)
        std::copy(res[(size_t)i].begin(), res[(size_t)i].end(), ids + offsets[i]);
    return SVL_OK;
}

// Tokenizer::decode (tokenizer.rs:391-425).
svl_status svl_tokenizer_decode(const svl_tokenizer *t, const uint32_t *ids, size_t n,
                                int skip_special_tokens, char *out, size_t capacity,
                                size_t *len) {
    if (!t || !len || (n && !ids)) return fail(SVL_USAGE, "tokenizer, ids and length are required");
    std::string bytes;
    for (size_t i = 0; i < n; ++i) {
        auto it = t->id_to_token.find(ids[i]);
        if (it == t->id_to_token.end())
            return fail(SVL_CORRUPT, "cannot decode unknown token id %u", (unsigned)ids[i]);
        if (skip_special_tokens && t->special_ids.count(ids[i])) continue;
        uint8_t byte;
        if (parse_byte_token(it->second, byte)) {
            bytes.push_back((char)byte);
        } else {
            const std::string &tok = it->second;
            for (size_t k = 0; k < tok.size();) {
                size_t j = k;
                const uint32_t cp = decode_cp((const unsigned char *)tok.data(), j);
                if (cp == SPACE_MARKER) bytes.push_back(' ');
                else bytes.append(tok, k, j - k);
                k = j;
            }
        }
    }
    if (!json::valid_utf8(bytes.data(), bytes.size()))
        return fail(SVL_CORRUPT, "decoded token sequence is not valid UTF-8");
    *len = bytes.size();
    if (bytes.size() > capacity || (!out && !bytes.empty()))
        return fail(SVL_USAGE, "output holds %zu bytes, %zu needed", capacity, bytes.size());
    if (!bytes.empty()) std::memcpy(out, bytes.data(), bytes.size());
    return SVL_OK;
}

int64_t svl_tokenizer_token_id(const svl_tokenizer *t, const char *token, size_t len) {
    if (!t || (!token && len)) return -1;
    auto it = t->vocab.find(std::string(token ? token : "", len));
    return it == t->vocab.end() ? -1 : (int64_t)it->second;
}

const char *svl_tokenizer_token(const svl_tokenizer *t, uint32_t id, size_t *len) {
    if (!t) return nullptr;
    auto it = t->id_to_token.find(id);
    if (it == t->id_to_token.end()) return nullptr;
    if (len) *len = it->second.size();
    return it->second.c_str();
}

int64_t svl_tokenizer_vocab_size(const svl_tokenizer *t) { return t ? (int64_t)t->vocab.size() : -1; }
int64_t svl_tokenizer_max_token_id(const svl_tokenizer *t) { return t ? (int64_t)t->max_token_id : -1; }
int64_t svl_tokenizer_bos_id(const svl_tokenizer *t) { return t ? (int64_t)t->bos_id : -1; }
int64_t svl_tokenizer_eos_id(const svl_tokenizer *t) { return t ? (int64_t)t->eos_id : -1; }
int64_t svl_tokenizer_unk_id(const svl_tokenizer *t) { return t ? (int64_t)t->unk_id : -1; }
int64_t svl_tokenizer_pad_id(const svl_tokenizer *t) { return t ? t->pad_id : -1; }
int svl_tokenizer_is_special_id(const svl_tokenizer *t, uint32_t id) {
    return t && t->special_ids.count(id) ? 1 : 0;
}

// TextEmbedder::embed (text.rs:610-626) for a batch: prompt prefix, encode
// with <bos>/<eos>, the 8192-token context check, then the forward pass of
// every row at once and ForwardOutput::embedding(dimension).
svl_status svl_text_embed_texts(svl_text_model *model, const svl_tokenizer *t,
                                const char *const *texts, const size_t *lens, int32_t n,
                                int32_t prompt, int64_t dimension, float *out) {
    if (!model || !t || n < 0 || (n > 0 && (!texts || !lens || !out)))
        return fail(SVL_USAGE, "model, tokenizer, texts and output are required");
    if (prompt < 0 || prompt >= (int32_t)(sizeof PROMPT_PREFIX / sizeof *PROMPT_PREFIX))
        return fail(SVL_USAGE, "unknown prompt role %d", prompt);
    std::vector<std::vector<uint32_t>> res;
    std::vector<svl_status> st;
    std::vector<std::string> msg;
    encode_many(t, texts, lens, (size_t)n, true, PROMPT_PREFIX[prompt], res, st, msg);
    const int64_t E = text_embedding_dim(model);
    std::vector<int64_t> offsets(1, 0);
    for (int32_t i = 0; i < n; ++i) {
        if (st[(size_t)i] != SVL_OK) return fail(st[(size_t)i], "text %d: %s", i, msg[(size_t)i].c_str());
        if (res[(size_t)i].size() > MAX_TEXT_TOKENS)
            return fail(SVL_LIMIT, "text %d: tokenized input has %zu tokens, above the %zu-token context",
                        i, res[(size_t)i].size(), MAX_TEXT_TOKENS);
        if (dimension <= 0 || dimension > E)
            return fail(SVL_INTERNAL, "embedding dimension %lld is outside 1..=%lld",
                        (long long)dimension, (long long)E);
        offsets.push_back(offsets.back() + (int64_t)res[(size_t)i].size());
    }
    if (n == 0) return SVL_OK;
    std::vector<uint32_t> ids;
    ids.reserve((size_t)offsets.back());
    for (auto &r : res) ids.insert(ids.end(), r.begin(), r.end());
    std::vector<float> normalized((size_t)(n * E));
    ST_TRY(svl_text_forward_batch(model, ids.data(), offsets.data(), n, nullptr, normalized.data(),
                                  nullptr, nullptr, nullptr));
    for (int32_t i = 0; i < n; ++i)
        ST_TRY(svl_truncate_and_normalize(normalized.data() + (size_t)i * E, (size_t)E,
                                          (size_t)dimension, out + (size_t)i * dimension));
    return SVL_OK;
}

}  // extern "C"
