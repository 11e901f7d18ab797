// Byte-level BPE tokenizer of a Qwen2 GGUF vocabulary (see jfh_tokenizer.hpp).
#include "jfh_tokenizer.hpp"

#include <algorithm>
#include <filesystem>
#include <fstream>
#include <iterator>
#include <queue>
#include <stdexcept>

#include "jfh_format.hpp"

namespace jfh::runtime::tokenization {
namespace {

struct CodeRange {
    uint32_t lo, hi;
};
#include "jfh_unicode_ranges.inc"

template <size_t N>
bool in_ranges(const CodeRange (&r)[N], uint32_t cp) {
    const CodeRange* end = r + N;
    const CodeRange* it = std::upper_bound(r, end, cp, [](uint32_t v, const CodeRange& x) { return v < x.lo; });
    return it != r && cp <= (it - 1)->hi;
}

bool is_letter(uint32_t cp) { return cp < 0x80 ? ((cp | 0x20) >= 'a' && (cp | 0x20) <= 'z') : in_ranges(kLetterRanges, cp); }
bool is_number(uint32_t cp) { return cp < 0x80 ? (cp >= '0' && cp <= '9') : in_ranges(kNumberRanges, cp); }
// The regex's \s: the Unicode White_Space property.
bool is_space(uint32_t cp) {
    return (cp >= 0x09 && cp <= 0x0D) || cp == 0x20 || cp == 0x85 || cp == 0xA0 || cp == 0x1680 ||
           (cp >= 0x2000 && cp <= 0x200A) || cp == 0x2028 || cp == 0x2029 || cp == 0x202F || cp == 0x205F ||
           cp == 0x3000;
}
bool is_crlf(uint32_t cp) { return cp == '\r' || cp == '\n'; }
// [^\s\p{L}\p{N}]
bool is_other(uint32_t cp) { return !is_space(cp) && !is_letter(cp) && !is_number(cp); }

// UTF-8 -> code points; an invalid byte becomes U+FFFD and is skipped alone.
std::vector<uint32_t> code_points(std::string_view s) {
    std::vector<uint32_t> out;
    out.reserve(s.size());
    size_t i = 0;
    auto cont = [&](size_t k) { return i + k < s.size() && (static_cast<uint8_t>(s[i + k]) & 0xC0) == 0x80; };
    while (i < s.size()) {
        const uint8_t b = static_cast<uint8_t>(s[i]);
        if (b < 0x80) {
            out.push_back(b);
            i += 1;
        } else if ((b & 0xE0) == 0xC0 && cont(1)) {
            out.push_back(((b & 0x1Fu) << 6) | (static_cast<uint8_t>(s[i + 1]) & 0x3Fu));
            i += 2;
        } else if ((b & 0xF0) == 0xE0 && cont(1) && cont(2)) {
            out.push_back(((b & 0x0Fu) << 12) | ((static_cast<uint8_t>(s[i + 1]) & 0x3Fu) << 6) |
                          (static_cast<uint8_t>(s[i + 2]) & 0x3Fu));
            i += 3;
        } else if ((b & 0xF8) == 0xF0 && cont(1) && cont(2) && cont(3)) {
            out.push_back(((b & 0x07u) << 18) | ((static_cast<uint8_t>(s[i + 1]) & 0x3Fu) << 12) |
                          ((static_cast<uint8_t>(s[i + 2]) & 0x3Fu) << 6) | (static_cast<uint8_t>(s[i + 3]) & 0x3Fu));
            i += 4;
        } else {
            out.push_back(0xFFFD);
            i += 1;
        }
    }
    return out;
}

void append_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
        s += static_cast<char>(cp);
    } else if (cp < 0x800) {
        s += static_cast<char>(0xC0 | (cp >> 6));
        s += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        s += static_cast<char>(0xE0 | (cp >> 12));
        s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        s += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
        s += static_cast<char>(0xF0 | (cp >> 18));
        s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
        s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
        s += static_cast<char>(0x80 | (cp & 0x3F));
    }
}

// GPT-2's byte <-> character map: printable Latin-1 bytes stand for
// themselves, the other 68 bytes for U+0100.. in byte order.
struct ByteMap {
    uint32_t to_cp[256];
    std::unordered_map<uint32_t, uint8_t> to_byte;
    ByteMap() {
        uint32_t extra = 0;
        for (uint32_t b = 0; b < 256; ++b) {
            const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
            to_cp[b] = printable ? b : 0x100 + extra++;
            to_byte[to_cp[b]] = static_cast<uint8_t>(b);
        }
    }
};
const ByteMap& byte_map() {
    static const ByteMap m;
    return m;
}

// Length in code points of the Qwen2 pre-tokenizer's match at i:
// (?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])
// | [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} | ' '?[^\s\p{L}\p{N}]+[\r\n]*
// | \s*[\r\n]+ | \s+(?!\S) | \s+
// (alternatives in order, the first that matches wins; quantifiers greedy).
size_t qwen2_match(const std::vector<uint32_t>& c, size_t i) {
    const size_t n = c.size();
    auto lower = [](uint32_t x) { return (x >= 'A' && x <= 'Z') ? x + 32 : x; };
    if (c[i] == '\'' && i + 1 < n) {
        const uint32_t a = lower(c[i + 1]);
        if (a == 's' || a == 't' || a == 'm' || a == 'd') return 2;
        if (i + 2 < n) {
            const uint32_t b = lower(c[i + 2]);
            if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return 3;
        }
    }
    {
        size_t j = i;
        if (!is_letter(c[i]) && !is_number(c[i]) && !is_crlf(c[i]) && i + 1 < n && is_letter(c[i + 1])) j = i + 1;
        if (is_letter(c[j])) {
            while (j < n && is_letter(c[j])) ++j;
            return j - i;
        }
    }
    if (is_number(c[i])) return 1;
    {
        size_t j = i;
        if (c[i] == ' ' && i + 1 < n && is_other(c[i + 1])) j = i + 1;
        if (is_other(c[j])) {
            while (j < n && is_other(c[j])) ++j;
            while (j < n && is_crlf(c[j])) ++j;
            return j - i;
        }
    }
    // c[i] is white space: the run [i, j)
    size_t j = i, last_crlf = n;
    while (j < n && is_space(c[j])) {
        if (is_crlf(c[j])) last_crlf = j;
        ++j;
    }
    if (last_crlf != n) return last_crlf + 1 - i;  // \s*[\r\n]+ ends after the run's last CR/LF
    if (j == n || j - i == 1) return j - i;       // \s+(?!\S) at the end, or \s+
    return j - 1 - i;                             // \s+(?!\S): leave the last blank to the next word
}

// The end texts llama.cpp's vocabulary loader marks as end of generation.
constexpr const char* kEndTexts[] = {
    "<|eot_id|>", "<|im_end|>", "<|end|>", "<|return|>", "<|call|>", "<end_of_turn>", "<|endoftext|>",
    "<|eom_id|>", "<EOT>", "_<EOT>", "<|end_of_text|>", "<end_of_utterance>",
    // fill-in-the-middle pad / repository / file separator tokens
    "<|fim_pad|>", "<fim-pad>", "<fim_pad>", "<|fim_repo|>", "<|repo_name|>", "<fim-repo>", "<reponame>",
    "<|file_sep|>", "<file_sep>",
};

std::vector<uint8_t> read_file(const std::string& path, size_t limit) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw Error(Status::IoError, "cannot open tokenizer metadata " + path);
    std::vector<uint8_t> bytes;
    char buf[1 << 16];
    while (in && bytes.size() < limit) {
        in.read(buf, sizeof(buf));
        bytes.insert(bytes.end(), buf, buf + in.gcount());
    }
    return bytes;
}

}  // namespace

std::shared_ptr<const BpeTokenizer> BpeTokenizer::open(const std::string& path) {
    namespace fs = std::filesystem;
    const bool dir = fs::is_directory(path);
    const std::string file = dir ? (fs::path(path) / "metadata.gguf").string() : path;
    if (dir && !fs::exists(file)) throw Error(Status::NotFound, "native model package is missing metadata.gguf");
    // the KV section of a GGUF file precedes its tensor data; 256 MiB bounds a vocabulary
    const std::vector<uint8_t> bytes = read_file(file, size_t{256} << 20);
    if (bytes.empty()) throw Error(Status::FormatError, "native model metadata is empty");
    return from_gguf(bytes.data(), bytes.size());
}

std::shared_ptr<const BpeTokenizer> BpeTokenizer::from_gguf(const uint8_t* data, size_t size) {
    const std::map<std::string, GgufValue> kv = parse_gguf_kv(data, size, true);
    auto find = [&](const char* key) -> const GgufValue* {
        const auto it = kv.find(key);
        return it == kv.end() ? nullptr : &it->second;
    };
    const GgufValue* model = find("tokenizer.ggml.model");
    if (model == nullptr || model->kind != GgufValue::Str || model->str != "gpt2") {
        throw Error(Status::FormatError, "metadata holds no byte-level BPE vocabulary (tokenizer.ggml.model gpt2)");
    }
    const GgufValue* tokens = find("tokenizer.ggml.tokens");
    const GgufValue* merges = find("tokenizer.ggml.merges");
    if (tokens == nullptr || tokens->kind != GgufValue::StrArr || tokens->strs.empty()) {
        throw Error(Status::FormatError, "tokenizer.ggml.tokens is missing");
    }
    if (merges == nullptr || merges->kind != GgufValue::StrArr) {
        throw Error(Status::FormatError, "tokenizer.ggml.merges is missing");
    }
    std::shared_ptr<BpeTokenizer> t(new BpeTokenizer());
    t->tokens_ = tokens->strs;
    const size_t n = t->tokens_.size();
    t->types_.assign(n, kNormal);
    if (const GgufValue* types = find("tokenizer.ggml.token_type"); types && types->kind == GgufValue::I32Arr) {
        if (types->ints.size() != n) throw Error(Status::FormatError, "tokenizer.ggml.token_type does not match the vocabulary");
        t->types_ = types->ints;
    }
    // llama.cpp's vocabulary load: an empty text is spelled "[EMPTY_<id>]", and
    // a text listed twice maps to its last id
    t->text_to_id_.reserve(n);
    for (size_t id = 0; id < n; ++id) {
        if (t->tokens_[id].empty()) t->tokens_[id] = "[EMPTY_" + std::to_string(id) + "]";
        t->text_to_id_[t->tokens_[id]] = static_cast<int32_t>(id);
    }
    t->merge_rank_.reserve(merges->strs.size());
    for (size_t r = 0; r < merges->strs.size(); ++r) {
        const std::string& m = merges->strs[r];
        const size_t sp = m.find(' ', 1);
        if (sp == std::string::npos) throw Error(Status::FormatError, "tokenizer merge without a separator");
        t->merge_rank_.emplace(m, static_cast<int32_t>(r));
    }
    for (size_t id = 0; id < n; ++id) {
        const int32_t ty = t->types_[id];
        if (ty == kControl || ty == kUserDefined || ty == kUnknown) t->specials_.push_back(static_cast<int32_t>(id));
    }
    std::stable_sort(t->specials_.begin(), t->specials_.end(), [&](int32_t a, int32_t b) {
        return t->tokens_[a].size() > t->tokens_[b].size();
    });
    auto id_of = [&](const char* key) -> int32_t {
        const GgufValue* v = find(key);
        if (v == nullptr || (v->kind != GgufValue::U32 && v->kind != GgufValue::I32)) return -1;
        const int32_t id = static_cast<int32_t>(v->u32);
        return id >= 0 && static_cast<size_t>(id) < n ? id : -1;
    };
    auto flag = [&](const char* key) {
        const GgufValue* v = find(key);
        return v != nullptr && v->kind == GgufValue::Bool && v->u32 != 0;
    };
    t->bos_ = id_of("tokenizer.ggml.bos_token_id");
    t->eos_ = id_of("tokenizer.ggml.eos_token_id");
    t->add_bos_ = flag("tokenizer.ggml.add_bos_token");
    t->add_eos_ = flag("tokenizer.ggml.add_eos_token");
    for (const char* key : {"tokenizer.ggml.eos_token_id", "tokenizer.ggml.eot_token_id", "tokenizer.ggml.eom_token_id"}) {
        if (const int32_t id = id_of(key); id >= 0) t->end_.insert(id);
    }
    for (const char* text : kEndTexts) {
        if (const auto it = t->text_to_id_.find(text); it != t->text_to_id_.end()) t->end_.insert(it->second);
    }
    return t;
}

int32_t BpeTokenizer::rank(const std::string& left, const std::string& right) const {
    std::string key;
    key.reserve(left.size() + right.size() + 1);
    key += left;
    key += ' ';
    key += right;
    const auto it = merge_rank_.find(key);
    return it == merge_rank_.end() ? -1 : it->second;
}

// One pre-tokenizer piece: its bytes as GPT-2 byte characters, merged pair
// by pair (lowest rank first, the leftmost of equal ranks), then each final
// symbol's id; a symbol outside the vocabulary falls back to the ids of its
// single bytes that are tokens.
void BpeTokenizer::bpe(const std::string& piece, std::vector<std::int32_t>& out) const {
    const ByteMap& bm = byte_map();
    struct Sym {
        std::string text;
        int prev, next;
    };
    std::vector<Sym> sym;
    sym.reserve(piece.size());
    for (size_t k = 0; k < piece.size(); ++k) {
        Sym s;
        append_utf8(s.text, bm.to_cp[static_cast<uint8_t>(piece[k])]);
        s.prev = static_cast<int>(k) - 1;
        s.next = k + 1 < piece.size() ? static_cast<int>(k) + 1 : -1;
        sym.push_back(std::move(s));
    }
    struct Cand {
        int32_t rank;
        int left, right;
        size_t size;  // merged text length: a stale candidate no longer matches
    };
    auto worse = [](const Cand& a, const Cand& b) { return a.rank != b.rank ? a.rank > b.rank : a.left > b.left; };
    std::priority_queue<Cand, std::vector<Cand>, decltype(worse)> queue(worse);
    auto consider = [&](int l, int r) {
        if (l < 0 || r < 0) return;
        const int32_t rk = rank(sym[l].text, sym[r].text);
        if (rk >= 0) queue.push({rk, l, r, sym[l].text.size() + sym[r].text.size()});
    };
    for (int k = 0; k + 1 < static_cast<int>(sym.size()); ++k) consider(k, k + 1);
    while (!queue.empty()) {
        const Cand c = queue.top();
        queue.pop();
        Sym& l = sym[c.left];
        Sym& r = sym[c.right];
        if (l.text.empty() || r.text.empty() || l.next != c.right || l.text.size() + r.text.size() != c.size) continue;
        l.text += r.text;
        r.text.clear();
        l.next = r.next;
        if (r.next >= 0) sym[r.next].prev = c.left;
        consider(l.prev, c.left);
        consider(c.left, l.next);
    }
    for (int k = sym.empty() ? -1 : 0; k >= 0; k = sym[k].next) {
        const std::string& s = sym[k].text;
        if (const auto it = text_to_id_.find(s); it != text_to_id_.end()) {
            out.push_back(it->second);
            continue;
        }
        for (const char ch : s) {
            if (const auto jt = text_to_id_.find(std::string(1, ch)); jt != text_to_id_.end()) out.push_back(jt->second);
        }
    }
}

std::vector<std::string> BpeTokenizer::pre_tokenize(std::string_view text) const {
    const std::vector<uint32_t> cps = code_points(text);
    std::vector<std::string> pieces;
    for (size_t i = 0; i < cps.size();) {
        const size_t len = qwen2_match(cps, i);
        std::string piece;
        for (size_t k = i; k < i + len; ++k) append_utf8(piece, cps[k]);
        pieces.push_back(std::move(piece));
        i += len;
    }
    return pieces;
}

std::vector<std::int32_t> BpeTokenizer::encode(std::string_view text, bool add_special, bool parse_special) const {
    // fragments: raw text, or a special token id (text_id >= 0)
    struct Frag {
        int32_t id;
        std::string_view text;
    };
    std::vector<Frag> frags{{-1, text}};
    if (parse_special) {
        for (const int32_t sid : specials_) {
            const std::string& st = tokens_[sid];
            if (st.empty()) continue;
            std::vector<Frag> next;
            for (const Frag& f : frags) {
                if (f.id >= 0) {
                    next.push_back(f);
                    continue;
                }
                std::string_view rest = f.text;
                for (size_t at; (at = rest.find(st)) != std::string_view::npos;) {
                    if (at > 0) next.push_back({-1, rest.substr(0, at)});
                    next.push_back({sid, {}});
                    rest = rest.substr(at + st.size());
                }
                if (!rest.empty()) next.push_back({-1, rest});
            }
            frags.swap(next);
        }
    }
    std::vector<std::int32_t> out;
    if (add_special && add_bos_ && bos_ >= 0) out.push_back(bos_);
    for (const Frag& f : frags) {
        if (f.id >= 0) {
            out.push_back(f.id);
            continue;
        }
        for (const std::string& piece : pre_tokenize(f.text)) bpe(piece, out);
    }
    if (add_special && add_eos_ && eos_ >= 0) out.push_back(eos_);
    return out;
}

std::vector<std::int32_t> BpeTokenizer::tokenize(std::string_view text) const {
    std::vector<std::int32_t> ids = encode(text, true, true);
    if (ids.empty()) throw Error(Status::InvalidArgument, "native prompt tokenization produced no tokens");
    return ids;
}

std::string BpeTokenizer::token_piece(std::int32_t token) const {
    if (token < 0 || static_cast<size_t>(token) >= tokens_.size()) {
        throw Error(Status::InvalidArgument, "token id is outside the vocabulary");
    }
    const std::string& text = tokens_[token];
    const int32_t ty = types_[token];
    if (ty == kControl || ty == kUserDefined || ty == kUnknown) return text;
    if (ty != kNormal) return {};
    // byte characters back to bytes; a character outside the byte map is
    // spelled [UNK_BYTE_0x<its UTF-8 bytes in hex><the token text>]
    const ByteMap& bm = byte_map();
    std::string out;
    const std::vector<uint32_t> cps = code_points(text);
    for (const uint32_t cp : cps) {
        const auto it = bm.to_byte.find(cp);
        if (it != bm.to_byte.end()) {
            out += static_cast<char>(it->second);
            continue;
        }
        std::string u;
        append_utf8(u, cp);
        out += "[UNK_BYTE_0x";
        static const char hexd[] = "0123456789abcdef";
        for (const char ch : u) {
            out += hexd[static_cast<uint8_t>(ch) >> 4];
            out += hexd[static_cast<uint8_t>(ch) & 15];
        }
        out += text + "]";
    }
    return out;
}

bool BpeTokenizer::is_end_token(std::int32_t token) const { return token == -1 || end_.count(token) != 0; }

std::vector<std::int32_t> BpeTokenizer::end_tokens() const {
    std::vector<std::int32_t> ids(end_.begin(), end_.end());
    std::sort(ids.begin(), ids.end());
    return ids;
}

}  // namespace jfh::runtime::tokenization
