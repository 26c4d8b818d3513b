// Byte-level BPE (the Hugging Face tokenizer.json form SmolLM2 uses); see tokenizer.h.
//
// Encode, as AccelEP's Bpe::Encode does it (src/bpe.cc:999-1026, pieces :970-997):
//  1. added tokens are cut out of the text first: at each position the longest added token
//     that matches (the earliest listed on a tie) becomes its id;
//  2. between them, the text is decoded as UTF-8 and split so that every Unicode number
//     (general category N) stands alone (the Digits pre-tokenizer, individual digits);
//  3. each part is cut by the GPT-2 pattern
//        's|'t|'re|'ve|'m|'ll|'d| ?\p{L}+| ?\p{N}+| ?[^\s\p{L}\p{N}]+|\s+(?!\S)|\s+
//     with the lookahead confined to the part;
//  4. each match's UTF-8 bytes become the one-byte tokens of GPT-2's byte alphabet (a byte
//     whose token is not in the vocabulary is dropped), and the merges are applied, lowest
//     rank first, leftmost on a tie, until none applies.
// Decode maps each token's characters back to bytes through the same alphabet (a token with
// a character outside it, such as an added token, is copied as written), joins them and
// replaces every byte that does not start a valid UTF-8 sequence with U+FFFD
// (src/bpe.cc:1028-1066).
#include "tokenizer.h"

#include <algorithm>
#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iterator>
#include <limits>
#include <stdexcept>
#include <utility>

namespace accel_hip {
namespace {

[[noreturn]] void Bad(const std::string& what) { throw std::invalid_argument(what); }

// ---- UTF-8 --------------------------------------------------------------------------------

// The code point starting at s[i] and its length, or false when s[i] does not start a valid
// (shortest-form, non-surrogate, <= U+10FFFF) UTF-8 sequence.
bool NextCodePoint(std::string_view s, size_t i, char32_t* cp, size_t* len) {
  if (i >= s.size()) return false;
  const auto b0 = static_cast<unsigned char>(s[i]);
  if (b0 < 0x80) {
    *cp = b0;
    *len = 1;
    return true;
  }
  size_t n;
  char32_t v;
  char32_t min;
  if (b0 >= 0xC0 && b0 < 0xE0) {
    n = 2, v = b0 & 0x1F, min = 0x80;
  } else if (b0 >= 0xE0 && b0 < 0xF0) {
    n = 3, v = b0 & 0x0F, min = 0x800;
  } else if (b0 >= 0xF0 && b0 < 0xF8) {
    n = 4, v = b0 & 0x07, min = 0x10000;
  } else {
    return false;
  }
  if (s.size() - i < n) return false;
  for (size_t k = 1; k < n; ++k) {
    const auto b = static_cast<unsigned char>(s[i + k]);
    if ((b & 0xC0) != 0x80) return false;
    v = (v << 6) | (b & 0x3F);
  }
  if (v < min || v > 0x10FFFF || (v >= 0xD800 && v <= 0xDFFF)) return false;
  *cp = v;
  *len = n;
  return true;
}

void PutUtf8(std::string& out, char32_t cp) {
  if (cp < 0x80) {
    out += static_cast<char>(cp);
  } else if (cp < 0x800) {
    out += static_cast<char>(0xC0 | (cp >> 6));
    out += static_cast<char>(0x80 | (cp & 0x3F));
  } else if (cp < 0x10000) {
    out += static_cast<char>(0xE0 | (cp >> 12));
    out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
    out += static_cast<char>(0x80 | (cp & 0x3F));
  } else {
    out += static_cast<char>(0xF0 | (cp >> 18));
    out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
    out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
    out += static_cast<char>(0x80 | (cp & 0x3F));
  }
}

// ---- character classes ----------------------------------------------------------------------

struct CodeRange {
  char32_t first, last;
};
#include "unicode_ranges.inc"

template <size_t N>
bool InTable(const CodeRange (&table)[N], char32_t cp) {
  const CodeRange* end = table + N;
  const CodeRange* it = std::upper_bound(table, end, cp, [](char32_t c, const CodeRange& r) { return c < r.first; });
  return it != table && cp <= (it - 1)->last;
}

bool IsLetter(char32_t cp) { return InTable(kLetterRanges, cp); }
bool IsNumber(char32_t cp) { return InTable(kNumberRanges, cp); }
// The Unicode White_Space property (\s of the pattern).
bool IsSpace(char32_t cp) {
  return (cp >= 0x09 && cp <= 0x0D) || cp == 0x20 || cp == 0x85 || cp == 0xA0 || cp == 0x1680 ||
         (cp >= 0x2000 && cp <= 0x200A) || cp == 0x2028 || cp == 0x2029 || cp == 0x202F || cp == 0x205F ||
         cp == 0x3000;
}
bool IsOther(char32_t cp) { return !IsSpace(cp) && !IsLetter(cp) && !IsNumber(cp); }

// ---- the GPT-2 pattern over one part [begin, end) of the code points ------------------------

// End of the match at `at` (> at), trying the alternatives in the pattern's order.
size_t PatternMatch(const std::vector<char32_t>& cp, size_t at, size_t end) {
  // 's 't 're 've 'm 'll 'd
  if (cp[at] == U'\'' && at + 1 < end) {
    const char32_t c1 = cp[at + 1];
    if (c1 == U's' || c1 == U't' || c1 == U'm' || c1 == U'd') return at + 2;
    if (at + 2 < end) {
      const char32_t c2 = cp[at + 2];
      if ((c1 == U'r' && c2 == U'e') || (c1 == U'v' && c2 == U'e') || (c1 == U'l' && c2 == U'l')) return at + 3;
    }
  }
  // " ?" then one or more of a class, for letters, numbers and everything else but spaces.
  for (bool (*cls)(char32_t) : {IsLetter, IsNumber, IsOther}) {
    size_t j = at;
    if (cp[j] == U' ' && j + 1 < end && cls(cp[j + 1])) ++j;
    if (!cls(cp[j])) continue;
    while (j < end && cls(cp[j])) ++j;
    return j;
  }
  // \s+(?!\S): a run of spaces reaching the part's end is taken whole; otherwise all but its
  // last space, when that leaves at least one. Then \s+ takes the run.
  size_t j = at;
  while (j < end && IsSpace(cp[j])) ++j;
  if (j == at) return at + 1;  // unreachable: every code point is a letter, number, other or space
  if (j == end || j - at == 1) return j;
  return j - 1;
}

// ---- a minimal JSON reader -------------------------------------------------------------------

struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject };
  Kind kind = kNull;
  bool boolean = false;
  double number = 0.0;
  std::string text;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  const Json* Find(const char* key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class JsonReader {
 public:
  explicit JsonReader(const std::string& s) : s_(s) {}

  Json Document() {
    Json v = Value();
    Space();
    if (i_ != s_.size()) Error("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void Error(const char* what) {
    Bad("tokenizer json: " + std::string(what) + " at byte " + std::to_string(i_));
  }
  void Space() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  bool Take(char c) {
    Space();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  void Need(char c) {
    if (!Take(c)) Error("unexpected character");
  }
  bool Word(const char* w) {
    const size_t n = std::strlen(w);
    if (s_.compare(i_, n, w) != 0) return false;
    i_ += n;
    return true;
  }
  uint32_t Hex4() {
    if (s_.size() - i_ < 4) Error("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else Error("bad \\u escape");
    }
    return v;
  }
  std::string String() {
    Space();
    if (i_ >= s_.size() || s_[i_] != '"') Error("expected a string");
    ++i_;
    std::string out;
    while (true) {
      if (i_ >= s_.size()) Error("unterminated string");
      const char c = s_[i_++];
      if (c == '"') return out;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) Error("unterminated escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          char32_t cp = Hex4();
          if (cp >= 0xD800 && cp <= 0xDBFF && s_.compare(i_, 2, "\\u") == 0) {
            const size_t save = i_;
            i_ += 2;
            const uint32_t lo = Hex4();
            if (lo >= 0xDC00 && lo <= 0xDFFF) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            else i_ = save;
          }
          PutUtf8(out, cp);
          break;
        }
        default: Error("bad escape");
      }
    }
  }
  Json Value() {
    Space();
    if (i_ >= s_.size()) Error("unexpected end");
    Json v;
    const char c = s_[i_];
    if ((c == '{' || c == '[') && ++depth_ > kMaxDepth) Error("nesting too deep");
    if (c == '{') {
      ++i_;
      v.kind = Json::kObject;
      if (Take('}')) {
        --depth_;
        return v;
      }
      do {
        std::string key = String();
        Need(':');
        v.members.emplace_back(std::move(key), Value());
      } while (Take(','));
      Need('}');
      --depth_;
    } else if (c == '[') {
      ++i_;
      v.kind = Json::kArray;
      if (Take(']')) {
        --depth_;
        return v;
      }
      do {
        v.items.push_back(Value());
      } while (Take(','));
      Need(']');
      --depth_;
    } else if (c == '"') {
      v.kind = Json::kString;
      v.text = String();
    } else if (Word("true")) {
      v.kind = Json::kBool;
      v.boolean = true;
    } else if (Word("false")) {
      v.kind = Json::kBool;
    } else if (Word("null")) {
      v.kind = Json::kNull;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const char* begin = s_.c_str() + i_;
      char* stop = nullptr;
      errno = 0;
      v.number = std::strtod(begin, &stop);
      if (stop == begin || errno == ERANGE) Error("bad number");
      v.kind = Json::kNumber;
      i_ += static_cast<size_t>(stop - begin);
    } else {
      Error("unexpected character");
    }
    return v;
  }

  static constexpr int kMaxDepth = 64;  // tokenizer.json nests a few levels; bounds the recursion
  const std::string& s_;
  size_t i_ = 0;
  int depth_ = 0;
};

// A non-negative integer id from a JSON number.
int32_t IdOf(const Json& v, const char* what) {
  if (v.kind != Json::kNumber || v.number < 0 || v.number > 2000000.0 || v.number != static_cast<int64_t>(v.number))
    Bad(std::string("tokenizer ") + what + " id is not an integer in range");
  return static_cast<int32_t>(v.number);
}

bool IsNullOrMissing(const Json* v) { return v == nullptr || v->kind == Json::kNull; }

const std::string& TypeOf(const Json& v) {
  static const std::string none;
  const Json* t = v.Find("type");
  return t != nullptr && t->kind == Json::kString ? t->text : none;
}

}  // namespace

ByteBpe::ByteBpe() {
  // GPT-2's byte alphabet: the printable bytes stand for themselves, the other 68 take code
  // points 256, 257, ... in byte order.
  char32_t next = 256;
  for (int b = 0; b < 256; ++b) {
    const bool printable = (b >= 0x21 && b <= 0x7E) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
    alphabet_[b] = printable ? static_cast<char32_t>(b) : next++;
    reverse_[alphabet_[b]] = static_cast<uint8_t>(b);
    byte_token_[b] = -1;
  }
}

void ByteBpe::Load(const std::string& path) {
  loaded_ = false;
  tokens_.clear();
  special_.clear();
  added_.clear();
  merges_.clear();
  for (int b = 0; b < 256; ++b) byte_token_[b] = -1;

  std::ifstream in(path, std::ios::binary);
  if (!in) Bad("cannot open tokenizer file " + path);
  const std::string file((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  const Json doc = JsonReader(file).Document();
  if (doc.kind != Json::kObject) Bad("tokenizer json is not an object");

  // The pipeline this tokenizer implements, and nothing else.
  // normalizer and post_processor must be present, as null.
  const Json* normalizer = doc.Find("normalizer");
  const Json* post = doc.Find("post_processor");
  if (normalizer == nullptr || post == nullptr) Bad("tokenizer json is missing bpe data");
  if (normalizer->kind != Json::kNull) Bad("tokenizer normalizer is not supported");
  if (post->kind != Json::kNull) Bad("tokenizer post-processor is not supported");
  const Json* pre = doc.Find("pre_tokenizer");
  bool pre_ok = pre != nullptr && TypeOf(*pre) == "Sequence";
  const Json* steps = pre_ok ? pre->Find("pretokenizers") : nullptr;
  pre_ok = pre_ok && steps != nullptr && steps->kind == Json::kArray && steps->items.size() == 2;
  if (pre_ok) {
    const Json& digits = steps->items[0];
    const Json& bytes = steps->items[1];
    const Json* individual = digits.Find("individual_digits");
    const Json* prefix = bytes.Find("add_prefix_space");
    const Json* regex = bytes.Find("use_regex");
    pre_ok = TypeOf(digits) == "Digits" && individual != nullptr && individual->kind == Json::kBool &&
             individual->boolean && TypeOf(bytes) == "ByteLevel" &&
             (prefix == nullptr || (prefix->kind == Json::kBool && !prefix->boolean)) &&
             (regex == nullptr || (regex->kind == Json::kBool && regex->boolean));
  }
  if (!pre_ok) Bad("tokenizer pre-tokenizer is not Digits(individual) then ByteLevel(no prefix space, regex)");
  const Json* decoder = doc.Find("decoder");
  if (decoder == nullptr || TypeOf(*decoder) != "ByteLevel") Bad("tokenizer decoder is not ByteLevel");
  const Json* model = doc.Find("model");
  if (model == nullptr || TypeOf(*model) != "BPE") Bad("tokenizer model is not BPE");
  for (const char* key : {"dropout", "unk_token", "continuing_subword_prefix", "end_of_word_suffix"})
    if (!IsNullOrMissing(model->Find(key))) Bad(std::string("tokenizer model ") + key + " is not supported");
  for (const char* key : {"fuse_unk", "byte_fallback", "ignore_merges"}) {
    const Json* flag = model->Find(key);
    if (flag != nullptr && flag->kind == Json::kBool && flag->boolean)
      Bad(std::string("tokenizer model ") + key + " is not supported");
  }

  // Vocabulary: ids 0 .. n-1, each once.
  const Json* vocab = model->Find("vocab");
  if (vocab == nullptr || vocab->kind != Json::kObject || vocab->members.empty()) Bad("tokenizer vocab is missing");
  std::unordered_map<std::string, int32_t> ids;
  ids.reserve(vocab->members.size() * 2);
  std::vector<std::string> tokens(vocab->members.size());
  std::vector<uint8_t> seen(vocab->members.size(), 0);
  for (const auto& [token, idv] : vocab->members) {
    const int32_t id = IdOf(idv, "vocab");
    if (static_cast<size_t>(id) >= tokens.size()) Bad("tokenizer vocab ids are not 0 .. n-1");
    if (seen[static_cast<size_t>(id)] || !ids.emplace(token, id).second) Bad("tokenizer vocab repeats a token or id");
    seen[static_cast<size_t>(id)] = 1;
    tokens[static_cast<size_t>(id)] = token;
  }

  // Merges, in rank order: "left right" strings or [left, right] pairs.
  const Json* merges = model->Find("merges");
  if (merges == nullptr || merges->kind != Json::kArray || merges->items.empty()) Bad("tokenizer merges are missing");
  std::unordered_map<uint64_t, MergeRule> rules;
  rules.reserve(merges->items.size() * 2);
  uint32_t rank = 0;
  for (const Json& m : merges->items) {
    std::string left, right;
    if (m.kind == Json::kString) {
      const size_t sp = m.text.find(' ');
      if (sp == std::string::npos || m.text.find(' ', sp + 1) != std::string::npos) Bad("tokenizer merge is not a pair");
      left = m.text.substr(0, sp);
      right = m.text.substr(sp + 1);
    } else if (m.kind == Json::kArray && m.items.size() == 2 && m.items[0].kind == Json::kString &&
               m.items[1].kind == Json::kString) {
      left = m.items[0].text;
      right = m.items[1].text;
    } else {
      Bad("tokenizer merge is not a pair");
    }
    const auto l = ids.find(left);
    const auto r = ids.find(right);
    const auto j = ids.find(left + right);
    if (l == ids.end() || r == ids.end() || j == ids.end()) Bad("tokenizer merge names a token outside the vocab");
    const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(l->second)) << 32) |
                         static_cast<uint32_t>(r->second);
    rules.emplace(key, MergeRule{rank, j->second});  // a repeated pair keeps its first (lowest) rank
    ++rank;
  }

  // Added tokens: in the vocabulary under the same id; `special` ones may be skipped on decode.
  std::vector<uint8_t> special(tokens.size(), 0);
  std::vector<AddedToken> added;
  if (const Json* list = doc.Find("added_tokens"); list != nullptr && list->kind != Json::kNull) {
    if (list->kind != Json::kArray) Bad("tokenizer added_tokens is not a list");
    for (const Json& a : list->items) {
      const Json* content = a.Find("content");
      const Json* idv = a.Find("id");
      if (content == nullptr || content->kind != Json::kString || idv == nullptr) Bad("tokenizer added token is invalid");
      const int32_t id = IdOf(*idv, "added token");
      const auto it = ids.find(content->text);
      if (it == ids.end() || it->second != id) Bad("tokenizer added token is not in the vocab under its id");
      const Json* sp = a.Find("special");
      if (sp != nullptr && sp->kind == Json::kBool && sp->boolean) special[static_cast<size_t>(id)] = 1;
      if (!content->text.empty()) added.push_back(AddedToken{content->text, id});
    }
  }

  for (int b = 0; b < 256; ++b) {
    std::string one;
    PutUtf8(one, alphabet_[b]);
    const auto it = ids.find(one);
    byte_token_[b] = it == ids.end() ? -1 : it->second;
  }
  tokens_ = std::move(tokens);
  special_ = std::move(special);
  added_ = std::move(added);
  merges_ = std::move(rules);
  loaded_ = true;
}

size_t ByteBpe::LongestAdded(std::string_view text, size_t pos, int32_t* id) const {
  size_t best = 0;
  for (const AddedToken& a : added_) {
    if (a.text.size() > best && text.size() - pos >= a.text.size() &&
        text.compare(pos, a.text.size(), a.text) == 0) {
      best = a.text.size();
      *id = a.id;
    }
  }
  return best;
}

void ByteBpe::EncodeWord(const std::vector<int32_t>& symbols, std::vector<int32_t>& out) const {
  std::vector<int32_t> w = symbols;
  while (w.size() > 1) {
    uint32_t best_rank = std::numeric_limits<uint32_t>::max();
    size_t best = 0;
    int32_t result = -1;
    for (size_t k = 0; k + 1 < w.size(); ++k) {
      const uint64_t key = (static_cast<uint64_t>(static_cast<uint32_t>(w[k])) << 32) | static_cast<uint32_t>(w[k + 1]);
      const auto it = merges_.find(key);
      if (it != merges_.end() && it->second.rank < best_rank) {
        best_rank = it->second.rank;
        best = k;
        result = it->second.result;
      }
    }
    if (result < 0) break;
    w[best] = result;
    w.erase(w.begin() + static_cast<std::ptrdiff_t>(best) + 1);
  }
  out.insert(out.end(), w.begin(), w.end());
}

void ByteBpe::EncodeSegment(std::string_view segment, std::vector<int32_t>& out) const {
  std::vector<char32_t> cps;
  std::vector<size_t> offset;  // byte offset of each code point, plus the end
  for (size_t i = 0; i < segment.size();) {
    char32_t cp;
    size_t len;
    if (!NextCodePoint(segment, i, &cp, &len)) Bad("prompt is not utf-8");
    cps.push_back(cp);
    offset.push_back(i);
    i += len;
  }
  offset.push_back(segment.size());
  std::vector<int32_t> symbols;
  size_t part = 0;
  while (part < cps.size()) {
    // The digit split: a number stands alone, everything else runs to the next number.
    size_t part_end = part + 1;
    if (!IsNumber(cps[part]))
      while (part_end < cps.size() && !IsNumber(cps[part_end])) ++part_end;
    for (size_t at = part; at < part_end;) {
      const size_t end = PatternMatch(cps, at, part_end);
      symbols.clear();
      for (size_t b = offset[at]; b < offset[end]; ++b) {
        const int32_t id = byte_token_[static_cast<unsigned char>(segment[b])];
        if (id >= 0) symbols.push_back(id);
      }
      if (!symbols.empty()) EncodeWord(symbols, out);
      at = end;
    }
    part = part_end;
  }
}

std::vector<int32_t> ByteBpe::Encode(std::string_view text) const {
  if (!loaded_) Bad("tokenizer is not loaded");
  std::vector<int32_t> out;
  size_t pos = 0;
  while (pos < text.size()) {
    int32_t id = -1;
    const size_t n = LongestAdded(text, pos, &id);
    if (n > 0) {
      out.push_back(id);
      pos += n;
      continue;
    }
    size_t next = pos + 1;
    for (int32_t unused; next < text.size() && LongestAdded(text, next, &unused) == 0;) ++next;
    EncodeSegment(text.substr(pos, next - pos), out);
    pos = next;
  }
  return out;
}

std::string ByteBpe::Decode(const int32_t* ids, int32_t count, bool skip_special) const {
  if (!loaded_) Bad("tokenizer is not loaded");
  if (count < 0 || (count > 0 && ids == nullptr)) Bad("invalid decode");
  std::string bytes;
  for (int32_t k = 0; k < count; ++k) {
    const int32_t id = ids[k];
    if (id < 0 || id >= vocab_size()) Bad("token id is outside the vocabulary");
    if (skip_special && special_[static_cast<size_t>(id)]) continue;
    const std::string& token = tokens_[static_cast<size_t>(id)];
    std::string mapped;
    bool all_mapped = true;
    for (size_t i = 0; i < token.size();) {
      char32_t cp;
      size_t len;
      const auto it = NextCodePoint(token, i, &cp, &len) ? reverse_.find(cp) : reverse_.end();
      if (it == reverse_.end()) {
        all_mapped = false;
        break;
      }
      mapped += static_cast<char>(it->second);
      i += len;
    }
    bytes += all_mapped ? mapped : token;
  }
  std::string text;
  text.reserve(bytes.size());
  for (size_t i = 0; i < bytes.size();) {
    char32_t cp;
    size_t len;
    if (NextCodePoint(bytes, i, &cp, &len)) {
      text.append(bytes, i, len);
      i += len;
    } else {
      PutUtf8(text, 0xFFFD);
      ++i;
    }
  }
  return text;
}

}  // namespace accel_hip
