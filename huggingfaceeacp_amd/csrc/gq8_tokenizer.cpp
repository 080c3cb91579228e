// gq8_tokenizer.cpp -- Gemma's SentencePiece BPE read from tokenizer.json, on
// the host (Tokenizer/Tokenizer.h:35-124, Tokenizer.cpp:206-683), and its C
// ABI (include/gemma_q8.h).
//
// The pieces, merges and added tokens come from the fast-tokenizer file.  A
// space becomes the metaspace replacement (U+2581 in Gemma's file) before
// BPE, every character reaches BPE as its own piece or as its bytes' pieces
// (byte fallback), and the merges apply lowest rank first, leftmost first on
// a tie.  Added tokens are matched verbatim before any of that, longest
// first; decoding turns runs of byte pieces back into text (U+FFFD for each
// byte of a run that is not UTF-8) and leaves special tokens out unless asked.
#include "gemma_q8.h"
#include "gq8_checkpoint.hpp"
#include "gq8_json.hpp"

#include <algorithm>
#include <array>
#include <cstdio>
#include <fstream>
#include <iterator>
#include <queue>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace {

constexpr int32_t kNoToken = -1;
const std::string kReplacementCharacter = "\xef\xbf\xbd";

// The length of the UTF-8 sequence starting at text[at], or 0 when the bytes
// there start no valid sequence (overlong forms, surrogates and code points
// above U+10FFFF included).
size_t utf8_length(std::string_view text, size_t at)
{
    const auto byte = [&](size_t i) { return (unsigned char) text[i]; };
    const unsigned char b0 = byte(at);
    if (b0 < 0x80)
        return 1;
    size_t n;
    unsigned char lo = 0x80, hi = 0xBF; // the second byte's range
    if (b0 >= 0xC2 && b0 <= 0xDF) {
        n = 2;
    } else if (b0 >= 0xE0 && b0 <= 0xEF) {
        n = 3;
        if (b0 == 0xE0) lo = 0xA0;
        if (b0 == 0xED) hi = 0x9F;
    } else if (b0 >= 0xF0 && b0 <= 0xF4) {
        n = 4;
        if (b0 == 0xF0) lo = 0x90;
        if (b0 == 0xF4) hi = 0x8F;
    } else {
        return 0;
    }
    if (at + n > text.size())
        return 0;
    if (byte(at + 1) < lo || byte(at + 1) > hi)
        return 0;
    for (size_t i = 2; i < n; ++i)
        if (byte(at + i) < 0x80 || byte(at + i) > 0xBF)
            return 0;
    return n;
}

bool valid_utf8(std::string_view text)
{
    for (size_t at = 0; at < text.size();) {
        const size_t n = utf8_length(text, at);
        if (n == 0)
            return false;
        at += n;
    }
    return true;
}

int hex_value(char c)
{
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    return -1;
}

// `<0xNN>` (either case of hex digit) names byte NN (ByteFallback.cpp).
int byte_of_piece(std::string_view piece)
{
    if (piece.size() != 6 || piece.substr(0, 3) != "<0x" || piece[5] != '>')
        return -1;
    const int h = hex_value(piece[3]), l = hex_value(piece[4]);
    return h < 0 || l < 0 ? -1 : h * 16 + l;
}

const gq8::Json *member(const gq8::Json &o, const char *key)
{
    return o.kind == gq8::Json::Object ? o.find(key) : nullptr;
}

std::string string_or(const gq8::Json &o, const char *key, const std::string &fallback)
{
    const gq8::Json *v = member(o, key);
    return v && v->kind == gq8::Json::String ? v->text : fallback;
}

bool flag_or(const gq8::Json &o, const char *key, bool fallback)
{
    const gq8::Json *v = member(o, key);
    return v && v->kind == gq8::Json::Bool ? v->boolean : fallback;
}

struct Refusal {
    std::string message;
};

int32_t token_id(const gq8::Json *v)
{
    if (!v || v->kind != gq8::Json::Number)
        throw Refusal{"expected a token id"};
    return (int32_t) v->number;
}

} // namespace

// The metaspace layer (Tokenizer/Metaspace.h:14-45).
struct Metaspace {
    std::string replacement = "\xe2\x96\x81";
    bool prepend = false; // the dummy prefix
    bool split = false;   // BPE per replacement-led word

    std::string normalize(std::string_view text) const
    {
        std::string out;
        out.reserve(text.size() + replacement.size());
        if (prepend)
            out += replacement;
        for (char c : text) {
            if (c == ' ')
                out += replacement;
            else
                out += c;
        }
        return out;
    }

    // The words of normalized text: each replacement after the first byte
    // starts a new word.
    std::vector<std::string_view> words(std::string_view text) const
    {
        std::vector<std::string_view> out;
        if (text.empty())
            return out;
        if (!split || replacement.empty()) {
            out.push_back(text);
            return out;
        }
        size_t begin = 0;
        for (size_t at = text.find(replacement, 1); at != std::string_view::npos;
             at = text.find(replacement, at + replacement.size())) {
            out.push_back(text.substr(begin, at - begin));
            begin = at;
        }
        out.push_back(text.substr(begin));
        return out;
    }

    void restore(std::string_view piece, std::string &out) const
    {
        if (replacement.empty()) {
            out += piece;
            return;
        }
        size_t at = 0;
        for (size_t found; (found = piece.find(replacement, at)) != std::string_view::npos;
             at = found + replacement.size()) {
            out += piece.substr(at, found - at);
            out += ' ';
        }
        out += piece.substr(at);
    }

    // One normalizer or pre-tokenizer component (Tokenizer.cpp:135-192).
    void read_component(const gq8::Json &c)
    {
        const std::string type = string_or(c, "type", "");
        if (type == "Prepend") {
            prepend = true;
            const std::string p = string_or(c, "prepend", "");
            if (!p.empty())
                replacement = p;
        } else if (type == "Replace") {
            const gq8::Json *pattern = member(c, "pattern");
            if (!pattern || string_or(*pattern, "String", "") != " ")
                return;
            const std::string content = string_or(c, "content", "");
            if (!content.empty())
                replacement = content;
        } else if (type == "Metaspace") {
            const std::string r = string_or(c, "replacement", "");
            if (!r.empty())
                replacement = r;
            const std::string scheme = string_or(c, "prepend_scheme", "");
            prepend = !scheme.empty() ? scheme != "never" : flag_or(c, "add_prefix_space", true);
            split = flag_or(c, "split", true);
        }
    }

    // A component, or a Sequence's components in order.
    void read(const gq8::Json *node)
    {
        if (!node || node->kind != gq8::Json::Object)
            return;
        for (const char *key : {"normalizers", "pretokenizers"}) {
            const gq8::Json *children = member(*node, key);
            if (!children || children->kind != gq8::Json::Array)
                continue;
            for (const gq8::Json &child : children->items)
                read(&child);
            return;
        }
        read_component(*node);
    }
};

struct gq8_tokenizer {
    std::vector<std::string> pieces;
    std::vector<uint8_t> special;
    std::unordered_map<std::string, int32_t> ids;
    struct Merge {
        int rank;
        int32_t merged;
    };
    std::unordered_map<uint64_t, Merge> merges;
    std::array<int32_t, 256> bytePiece{};
    struct Added {
        std::string content;
        int32_t token;
    };
    std::vector<Added> added;                     // longest first
    std::array<std::vector<int>, 256> addedByByte; // indices into added, longest first
    gq8_special_tokens specials{kNoToken, kNoToken, kNoToken, kNoToken, kNoToken, kNoToken};
    Metaspace metaspace;
    bool byteFallback = false;
    bool fuseUnknown = false;

    static uint64_t pair_key(int32_t l, int32_t r)
    {
        return ((uint64_t) (uint32_t) l << 32) | (uint32_t) r;
    }

    int32_t lookup(std::string_view text) const
    {
        const auto it = ids.find(std::string(text));
        return it == ids.end() ? kNoToken : it->second;
    }

    std::string_view piece(int32_t token) const
    {
        return token >= 0 && token < (int32_t) pieces.size() ? std::string_view(pieces[token])
                                                              : std::string_view();
    }

    bool is_special(int32_t token) const
    {
        return token >= 0 && token < (int32_t) special.size() && special[token];
    }

    void add_piece(const std::string &text, int32_t token, bool isSpecial)
    {
        if (token < 0 || text.empty())
            return;
        if (token >= (int32_t) pieces.size()) {
            pieces.resize(token + 1);
            special.resize(token + 1);
        }
        pieces[token] = text;
        special[token] = isSpecial ? 1 : 0;
        ids[text] = token;
    }

    void unknown(std::vector<int32_t> &out) const
    {
        if (specials.unk == kNoToken)
            return;
        if (fuseUnknown && !out.empty() && out.back() == specials.unk)
            return;
        out.push_back(specials.unk);
    }

    // One character: its own piece, else all of its bytes' pieces, else
    // unknown (Tokenizer.cpp:413-442).
    void character(std::string_view c, std::vector<int32_t> &out) const
    {
        const int32_t id = lookup(c);
        if (id != kNoToken) {
            out.push_back(id);
            return;
        }
        if (!byteFallback) {
            unknown(out);
            return;
        }
        for (char b : c)
            if (bytePiece[(unsigned char) b] == kNoToken) {
                unknown(out);
                return;
            }
        for (char b : c)
            out.push_back(bytePiece[(unsigned char) b]);
    }

    // BPE over one word: the symbols form a linked list; a heap holds the
    // mergeable neighbours by (rank, left index), and an entry whose symbols
    // have changed since it was pushed is dropped when it comes up.
    void word(std::string_view w, std::vector<int32_t> &out) const
    {
        std::vector<int32_t> token;
        for (size_t at = 0; at < w.size();) {
            const size_t n = std::max<size_t>(utf8_length(w, at), 1); // a stray byte is its own
            character(w.substr(at, n), token);
            at += n;
        }
        const int n = (int) token.size();
        if (n == 0)
            return;
        std::vector<int> prev(n), next(n);
        std::vector<char> live(n, 1);
        for (int i = 0; i < n; ++i) {
            prev[i] = i - 1;
            next[i] = i + 1 < n ? i + 1 : -1;
        }
        struct Entry {
            int rank, left;
            int32_t l, r;
            bool operator<(const Entry &o) const // the heap's top: lowest rank, then leftmost
            {
                return rank != o.rank ? rank > o.rank : left > o.left;
            }
        };
        std::priority_queue<Entry> heap;
        auto offer = [&](int left) {
            if (left < 0 || next[left] < 0)
                return;
            const auto it = merges.find(pair_key(token[left], token[next[left]]));
            if (it != merges.end())
                heap.push(Entry{it->second.rank, left, token[left], token[next[left]]});
        };
        for (int i = 0; i < n; ++i)
            offer(i);
        while (!heap.empty()) {
            const Entry e = heap.top();
            heap.pop();
            const int l = e.left, r = next[l];
            if (!live[l] || r < 0 || token[l] != e.l || token[r] != e.r)
                continue;
            token[l] = merges.at(pair_key(e.l, e.r)).merged;
            live[r] = 0;
            next[l] = next[r];
            if (next[l] >= 0)
                prev[next[l]] = l;
            offer(l);
            offer(prev[l]);
        }
        for (int i = 0; i >= 0; i = next[i])
            if (token[i] != kNoToken)
                out.push_back(token[i]);
    }

    void segment(std::string_view text, std::vector<int32_t> &out) const
    {
        const std::string normalized = metaspace.normalize(text);
        for (std::string_view w : metaspace.words(normalized))
            word(w, out);
    }

    int32_t added_at(std::string_view text, size_t at) const
    {
        for (int index : addedByByte[(unsigned char) text[at]]) {
            const Added &a = added[index];
            if (text.compare(at, a.content.size(), a.content) == 0)
                return a.token;
        }
        return kNoToken;
    }

    std::vector<int32_t> encode(std::string_view text) const
    {
        std::vector<int32_t> out;
        size_t begin = 0, at = 0;
        while (at < text.size()) {
            const int32_t a = added_at(text, at);
            if (a == kNoToken) {
                ++at;
                continue;
            }
            if (at > begin)
                segment(text.substr(begin, at - begin), out);
            out.push_back(a);
            at += piece(a).size();
            begin = at;
        }
        if (begin < text.size())
            segment(text.substr(begin), out);
        return out;
    }

    std::string decode(const int32_t *tokens, int count, bool keepSpecial) const
    {
        std::string text, run;
        auto flush = [&] {
            if (run.empty())
                return;
            if (valid_utf8(run)) {
                text += run;
            } else {
                for (size_t i = 0; i < run.size(); ++i)
                    text += kReplacementCharacter;
            }
            run.clear();
        };
        for (int i = 0; i < count; ++i) {
            const std::string_view p = piece(tokens[i]);
            if (p.empty())
                continue;
            const int b = byte_of_piece(p);
            if (b >= 0) {
                run += (char) b;
                continue;
            }
            flush();
            if (is_special(tokens[i])) {
                if (keepSpecial)
                    text += p;
                continue;
            }
            metaspace.restore(p, text);
        }
        flush();
        if (metaspace.prepend && !text.empty() && text[0] == ' ')
            text.erase(0, 1);
        return text;
    }

    // Tokenizer::fromJsonText (Tokenizer.cpp:211-301).
    void load(const gq8::Json &root)
    {
        const gq8::Json *model = member(root, "model");
        if (!model)
            throw Refusal{"tokenizer.json has no model"};
        const gq8::Json *vocab = member(*model, "vocab"), *mergeList = member(*model, "merges");
        if (!vocab)
            throw Refusal{"model.vocab is missing"};
        if (!mergeList)
            throw Refusal{"model.merges is missing"};
        if (vocab->kind != gq8::Json::Object)
            throw Refusal{"model.vocab is not an object"};
        if (mergeList->kind != gq8::Json::Array)
            throw Refusal{"model.merges is not an array"};
        const gq8::Json *addedList = member(root, "added_tokens");
        const bool hasAdded = addedList && addedList->kind == gq8::Json::Array;

        int32_t highest = -1;
        for (const auto &m : vocab->members)
            highest = std::max(highest, token_id(&m.second));
        if (hasAdded)
            for (const gq8::Json &e : addedList->items)
                highest = std::max(highest, token_id(member(e, "id")));
        bytePiece.fill(kNoToken);
        pieces.assign(highest + 1, std::string());
        special.assign(highest + 1, 0);
        ids.reserve((size_t) highest + 1);
        byteFallback = flag_or(*model, "byte_fallback", false);
        fuseUnknown = flag_or(*model, "fuse_unk", false);
        metaspace.read(member(root, "normalizer"));
        metaspace.read(member(root, "pre_tokenizer"));

        for (const auto &m : vocab->members)
            add_piece(m.first, token_id(&m.second), false);
        if (hasAdded) {
            for (const gq8::Json &e : addedList->items) {
                const int32_t id = token_id(member(e, "id"));
                const gq8::Json *content = member(e, "content");
                if (!content || content->kind != gq8::Json::String)
                    throw Refusal{"an added token has no content"};
                add_piece(content->text, id, flag_or(e, "special", true));
                added.push_back(Added{content->text, id});
                const std::string &c = content->text;
                if (c == "<pad>") specials.pad = id;
                else if (c == "<eos>") specials.eos = id;
                else if (c == "<bos>") specials.bos = id;
                else if (c == "<unk>") specials.unk = id;
                else if (c == "<start_of_turn>") specials.start_of_turn = id;
                else if (c == "<end_of_turn>") specials.end_of_turn = id;
            }
        }
        for (int i = 0; i < (int) added.size(); ++i)
            if (!added[i].content.empty())
                addedByByte[(unsigned char) added[i].content[0]].push_back(i);
        for (auto &bucket : addedByByte)
            std::stable_sort(bucket.begin(), bucket.end(), [&](int a, int b) {
                return added[a].content.size() > added[b].content.size();
            });
        for (int32_t id = 0; id < (int32_t) pieces.size(); ++id) {
            const int b = byte_of_piece(pieces[id]);
            if (b >= 0)
                bytePiece[b] = id;
        }
        const std::string unk = string_or(*model, "unk_token", "");
        if (!unk.empty()) {
            const int32_t id = lookup(unk);
            if (id != kNoToken)
                specials.unk = id;
        }
        merges.reserve(mergeList->items.size());
        for (int rank = 0; rank < (int) mergeList->items.size(); ++rank) {
            const gq8::Json &rule = mergeList->items[rank];
            std::string left, right;
            if (rule.kind == gq8::Json::Array) {
                if (rule.items.size() != 2 || rule.items[0].kind != gq8::Json::String
                    || rule.items[1].kind != gq8::Json::String)
                    throw Refusal{"a merge rule is not a pair of strings"};
                left = rule.items[0].text;
                right = rule.items[1].text;
            } else if (rule.kind == gq8::Json::String) {
                const size_t space = rule.text.find(' ');
                if (space == std::string::npos)
                    throw Refusal{"merge rule '" + rule.text + "' has no space"};
                left = rule.text.substr(0, space);
                right = rule.text.substr(space + 1);
            } else {
                throw Refusal{"a merge rule is neither a string nor a pair"};
            }
            const int32_t l = lookup(left), r = lookup(right), m = lookup(left + right);
            if (l == kNoToken || r == kNoToken || m == kNoToken)
                continue;
            merges.emplace(pair_key(l, r), Merge{rank, m});
        }
    }
};

namespace {

int from_text(const char *text, size_t length, gq8_tokenizer **out)
{
    gq8::Json root;
    gq8::JsonReader reader(text, length);
    if (!reader.read(root))
        return gq8::report(GQ8_ERR_FORMAT, "tokenizer.json is not valid JSON");
    auto *t = new gq8_tokenizer();
    try {
        t->load(root);
    } catch (const Refusal &r) {
        delete t;
        return gq8::report(GQ8_ERR_FORMAT, r.message);
    }
    *out = t;
    return GQ8_OK;
}

// Copies as much of `text` as fits (no terminator) and reports its length.
void copy_out(const std::string &text, char *out, size_t capacity, size_t *length)
{
    if (out && capacity)
        std::memcpy(out, text.data(), std::min(capacity, text.size()));
    if (length)
        *length = text.size();
}

} // namespace

extern "C" int gq8_tokenizer_from_json(const char *text, size_t length, gq8_tokenizer **out)
{
    if (!text || !out)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_from_json: null argument");
    *out = nullptr;
    return from_text(text, length, out);
}

extern "C" int gq8_tokenizer_open(const char *path, gq8_tokenizer **out)
{
    if (!path || !out)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_open: null argument");
    *out = nullptr;
    std::ifstream in(path, std::ios::binary);
    if (!in)
        return gq8::report(GQ8_ERR_FORMAT, std::string("cannot open '") + path + "'");
    const std::string text{std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>()};
    return from_text(text.data(), text.size(), out);
}

extern "C" void gq8_tokenizer_destroy(gq8_tokenizer *t)
{
    delete t;
}

extern "C" int gq8_tokenizer_encode(const gq8_tokenizer *t, const char *text, size_t length,
                                    int with_bos, int32_t *out, int capacity)
{
    if (!t || (!text && length) || (!out && capacity > 0) || capacity < 0)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_encode: bad argument");
    std::vector<int32_t> ids;
    if (with_bos && t->specials.bos != kNoToken)
        ids.push_back(t->specials.bos);
    const std::vector<int32_t> body = t->encode(std::string_view(text ? text : "", length));
    ids.insert(ids.end(), body.begin(), body.end());
    std::copy_n(ids.begin(), std::min<size_t>(ids.size(), (size_t) capacity), out);
    return (int) ids.size();
}

extern "C" int gq8_tokenizer_decode(const gq8_tokenizer *t, const int32_t *tokens, int count,
                                    int keep_special, char *out, size_t capacity, size_t *length)
{
    if (!t || (!tokens && count) || count < 0 || !length)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_decode: bad argument");
    copy_out(t->decode(tokens, count, keep_special != 0), out, capacity, length);
    return GQ8_OK;
}

extern "C" int gq8_tokenizer_vocabulary_size(const gq8_tokenizer *t)
{
    return t ? (int) t->pieces.size() : gq8::report(GQ8_ERR_ARGUMENT, "null tokenizer");
}

extern "C" int gq8_tokenizer_specials(const gq8_tokenizer *t, gq8_special_tokens *out)
{
    if (!t || !out)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_specials: null argument");
    *out = t->specials;
    return GQ8_OK;
}

extern "C" int gq8_tokenizer_is_special(const gq8_tokenizer *t, int32_t token)
{
    return t && t->is_special(token) ? 1 : 0;
}

extern "C" int gq8_tokenizer_token_text(const gq8_tokenizer *t, int32_t token, char *out,
                                        size_t capacity, size_t *length)
{
    if (!t || !length)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_token_text: null argument");
    copy_out(std::string(t->piece(token)), out, capacity, length);
    return GQ8_OK;
}

extern "C" int32_t gq8_tokenizer_token_for_text(const gq8_tokenizer *t, const char *text,
                                                size_t length)
{
    if (!t || (!text && length))
        return kNoToken;
    return t->lookup(std::string_view(text ? text : "", length));
}

extern "C" int gq8_tokenizer_metaspace(const gq8_tokenizer *t, char *replacement, size_t capacity,
                                       size_t *length, int *prepends, int *splits)
{
    if (!t || !length || !prepends || !splits)
        return gq8::report(GQ8_ERR_ARGUMENT, "tokenizer_metaspace: null argument");
    copy_out(t->metaspace.replacement, replacement, capacity, length);
    *prepends = t->metaspace.prepend ? 1 : 0;
    *splits = t->metaspace.split ? 1 : 0;
    return GQ8_OK;
}
