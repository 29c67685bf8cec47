// Tokenizers (kuiper/source/op/encode.cpp:14-182): SentencePiece BPE models
// and byte-level BPE tokenizer.json files, self-contained (see
// kuiper/encode.h for what each class reads and how it encodes).
#include "kuiper/encode.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <limits>
#include <queue>
#include <sstream>

namespace op {
namespace {

#include "unicode_ranges.inc"

// ---------------------------------------------------------------- UTF-8 ---
// Decodes the code point at s[i] and advances i; a byte that does not start a
// valid sequence (a stray continuation byte, a truncated or overlong form, a
// surrogate or a value above U+10FFFF) decodes as itself, one "character" of
// one byte.
uint32_t utf8_next(const std::string& s, size_t& i) {
  const unsigned char c = static_cast<unsigned char>(s[i]);
  int len = c < 0x80 ? 1 : (c >> 5) == 0x6 ? 2 : (c >> 4) == 0xE ? 3 : (c >> 3) == 0x1E ? 4 : 0;
  if (len == 0 || i + len > s.size()) {
    ++i;
    return c;
  }
  uint32_t cp = len == 1 ? c : len == 2 ? (c & 0x1F) : len == 3 ? (c & 0x0F) : (c & 0x07);
  for (int k = 1; k < len; ++k) {
    const unsigned char d = static_cast<unsigned char>(s[i + k]);
    if ((d >> 6) != 0x2) {
      ++i;
      return c;
    }
    cp = (cp << 6) | (d & 0x3F);
  }
  static const uint32_t kMin[5] = {0, 0, 0x80, 0x800, 0x10000};
  if (cp < kMin[len] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) {
    ++i;
    return c;
  }
  i += len;
  return cp;
}

void utf8_append(std::string& out, uint32_t cp) {
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

template <size_t N>
bool in_ranges(uint32_t cp, const uint32_t (&r)[N][2]) {
  size_t lo = 0, hi = N;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    if (cp < r[mid][0]) hi = mid;
    else if (cp > r[mid][1]) lo = mid + 1;
    else return true;
  }
  return false;
}

bool is_letter(uint32_t cp) { return in_ranges(cp, kLetterRanges); }
bool is_number(uint32_t cp) { return in_ranges(cp, kNumberRanges); }
// The pattern's \s is RE2's: ASCII [\t\n\f\r ].
bool is_ws(uint32_t cp) { return cp == '\t' || cp == '\n' || cp == '\f' || cp == '\r' || cp == ' '; }
bool is_crlf(uint32_t cp) { return cp == '\r' || cp == '\n'; }
bool is_other(uint32_t cp) { return !is_ws(cp) && !is_letter(cp) && !is_number(cp); }

// ----------------------------------------------------- pre-tokenizer ---
// End (code point index) of the piece starting at i, for the reference's
// pattern (encode.cpp:61-62), alternatives in order, leftmost-first:
//   (?i:'s|'t|'re|'ve|'m|'ll|'d) | [^\r\n\p{L}\p{N}]?\p{L}+ | \p{N} |
//    ?[^\s\p{L}\p{N}]+[\r\n]* | \s*[\r\n]+ | \s+(?:$|[^\S]) | \s+
// Every code point starts some alternative, so pieces tile the text.
size_t piece_end(const std::vector<uint32_t>& c, size_t i) {
  const size_t n = c.size();
  auto lower = [](uint32_t x) { return x >= 'A' && x <= 'Z' ? x + 32 : x; };
  // 1. English contractions, case-insensitive (RE2 folds U+017F onto s).
  if (c[i] == '\'' && i + 1 < n) {
    const uint32_t a = lower(c[i + 1]);
    if (a == 's' || c[i + 1] == 0x17F || a == 't' || a == 'm' || a == 'd') return i + 2;
    if (i + 2 < n) {
      const uint32_t b = lower(c[i + 2]);
      if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) return i + 3;
    }
  }
  // 2. Letters, with one leading character that is none of CR, LF, letter,
  //    number.
  if (!is_crlf(c[i]) && !is_letter(c[i]) && !is_number(c[i]) && i + 1 < n && is_letter(c[i + 1])) {
    size_t j = i + 1;
    while (j < n && is_letter(c[j])) ++j;
    return j;
  }
  if (is_letter(c[i])) {
    size_t j = i;
    while (j < n && is_letter(c[j])) ++j;
    return j;
  }
  // 3. One number.
  if (is_number(c[i])) return i + 1;
  // 4. Other characters, an optional leading space, trailing CR / LF.
  {
    size_t j = i;
    if (c[j] == ' ' && j + 1 < n && is_other(c[j + 1])) ++j;
    if (is_other(c[j])) {
      while (j < n && is_other(c[j])) ++j;
      while (j < n && is_crlf(c[j])) ++j;
      return j;
    }
  }
  // The whitespace run from i.
  size_t w = i;
  while (w < n && is_ws(c[w])) ++w;
  // 5. Whitespace up to and including its last CR / LF.
  for (size_t m = w; m > i; --m)
    if (is_crlf(c[m - 1])) return m;
  // 6. Whitespace at the end of the text, or of at least two characters
  //    (the last one satisfies [^\S]).
  if (w == n || w - i >= 2) return w;
  // 7. Whitespace.
  return w;
}

// ------------------------------------------------------------- JSON ---
// Just enough JSON for tokenizer.json: objects, arrays, strings (with
// escapes and surrogate pairs), numbers, literals.
struct JValue {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  double number = 0;
  bool boolean = false;
  std::string str;
  std::vector<JValue> items;
  std::vector<std::pair<std::string, JValue>> members;

  const JValue* get(const char* key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class JsonReader {
 public:
  JsonReader(const char* p, const char* end) : p_(p), end_(end) {}
  bool parse(JValue& v) {
    if (!value(v, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  bool hex4(uint32_t& u) {
    if (end_ - p_ < 4) return false;
    u = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = *p_++;
      u <<= 4;
      if (h >= '0' && h <= '9') u |= h - '0';
      else if (h >= 'a' && h <= 'f') u |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') u |= h - 'A' + 10;
      else return false;
    }
    return true;
  }
  bool string(std::string& out) {
    if (p_ >= end_ || *p_ != '"') return false;
    ++p_;
    while (p_ < end_ && *p_ != '"') {
      if (*p_ != '\\') {
        out += *p_++;
        continue;
      }
      if (++p_ >= end_) return false;
      const char e = *p_++;
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
          uint32_t u;
          if (!hex4(u)) return false;
          if (u >= 0xD800 && u < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2;
            uint32_t lo;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8_append(out, u);
          break;
        }
        default: return false;
      }
    }
    if (p_ >= end_) return false;
    ++p_;
    return true;
  }
  bool value(JValue& v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p_ >= end_) return false;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = JValue::kObject;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p_ >= end_ || *p_++ != ':') return false;
        v.members.emplace_back(std::move(key), JValue());
        if (!value(v.members.back().second, depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = JValue::kArray;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        v.items.emplace_back();
        if (!value(v.items.back(), depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v.kind = JValue::kString;
      return string(v.str);
    }
    if (lit("true")) {
      v.kind = JValue::kBool;
      v.boolean = true;
      return true;
    }
    if (lit("false")) {
      v.kind = JValue::kBool;
      return true;
    }
    if (lit("null")) return true;
    char* e = nullptr;
    std::string num;
    while (p_ < end_ && (std::isdigit(static_cast<unsigned char>(*p_)) || *p_ == '-' || *p_ == '+' ||
                         *p_ == '.' || *p_ == 'e' || *p_ == 'E'))
      num += *p_++;
    if (num.empty()) return false;
    v.kind = JValue::kNumber;
    v.number = std::strtod(num.c_str(), &e);
    return e && *e == '\0';
  }

  const char* p_;
  const char* end_;
};

bool read_file(const std::string& path, std::string& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f.is_open()) return false;
  out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  return true;
}

// The byte-level alphabet's inverse: code point -> byte (the printable
// Latin-1 bytes stand for themselves, the others for U+0100 upwards in byte
// order).
int unicode_to_byte(uint32_t cp) {
  static int table[324];
  static bool init = false;
  if (!init) {
    for (int& t : table) t = -1;
    int extra = 0;
    for (int b = 0; b < 256; ++b) {
      const bool keep = (b >= '!' && b <= '~') || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
      table[keep ? b : 256 + extra++] = b;
    }
    init = true;
  }
  return cp < 324 ? table[cp] : -1;
}

// --------------------------------------------------------- protobuf ---
// Just enough of the protobuf wire format for a SentencePiece ModelProto.
struct PbReader {
  const unsigned char* p;
  const unsigned char* end;
  bool varint(uint64_t& v) {
    v = 0;
    for (int shift = 0; shift < 64 && p < end; shift += 7) {
      const unsigned char b = *p++;
      v |= static_cast<uint64_t>(b & 0x7F) << shift;
      if (!(b & 0x80)) return true;
    }
    return false;
  }
  // Next field: number, wire type, and for wire type 2 the payload bounds.
  bool field(uint32_t& num, uint32_t& wt, uint64_t& val, const unsigned char*& data, size_t& len) {
    uint64_t key;
    if (!varint(key)) return false;
    num = static_cast<uint32_t>(key >> 3);
    wt = static_cast<uint32_t>(key & 7);
    switch (wt) {
      case 0: return varint(val);
      case 1:
        if (end - p < 8) return false;
        std::memcpy(&val, p, 8);
        p += 8;
        return true;
      case 2: {
        uint64_t n;
        if (!varint(n) || n > static_cast<uint64_t>(end - p)) return false;
        data = p;
        len = static_cast<size_t>(n);
        p += n;
        return true;
      }
      case 5: {
        if (end - p < 4) return false;
        uint32_t w;
        std::memcpy(&w, p, 4);
        val = w;
        p += 4;
        return true;
      }
      default: return false;
    }
  }
};

const char kSpaceSymbol[] = "\xE2\x96\x81";  // U+2581, SentencePiece's escaped space

}  // namespace

// ======================================================= SentencePiece ===
SpeEncodeLayer::SpeEncodeLayer(std::string token_model_path, bool has_bos, bool has_eos)
    : EncodeLayerBase(std::move(token_model_path), has_bos, has_eos) {
  for (int32_t& b : byte_ids_) b = -1;
  std::string bytes;
  if (!read_file(token_model_path_, bytes)) {
    status_ = base::error::PathNotValid("cannot open the tokenizer model " + token_model_path_);
    return;
  }
  PbReader r{reinterpret_cast<const unsigned char*>(bytes.data()),
             reinterpret_cast<const unsigned char*>(bytes.data()) + bytes.size()};
  int model_type = 1;  // proto default: UNIGRAM
  std::string norm_name;
  bool charsmap = false;
  while (r.p < r.end) {
    uint32_t num, wt;
    uint64_t val = 0;
    const unsigned char* data = nullptr;
    size_t len = 0;
    if (!r.field(num, wt, val, data, len)) {
      status_ = base::error::ModelParseError("malformed SentencePiece model " + token_model_path_);
      return;
    }
    if (wt != 2 || (num != 1 && num != 2 && num != 3)) continue;
    // ModelProto: pieces = 1 {piece = 1, score = 2, type = 3},
    // trainer_spec = 2 {model_type = 3, byte_fallback = 35, unk_id = 40,
    // bos_id = 41, eos_id = 42}, normalizer_spec = 3 {name = 1,
    // precompiled_charsmap = 2, add_dummy_prefix = 3,
    // remove_extra_whitespaces = 4, escape_whitespaces = 5}.
    Piece pc;
    PbReader s{data, data + len};
    while (s.p < s.end) {
      uint32_t n2, w2;
      uint64_t v2 = 0;
      const unsigned char* d2 = nullptr;
      size_t l2 = 0;
      if (!s.field(n2, w2, v2, d2, l2)) {
        status_ = base::error::ModelParseError("malformed SentencePiece model " + token_model_path_);
        return;
      }
      if (num == 1) {
        if (n2 == 1 && w2 == 2) pc.text.assign(reinterpret_cast<const char*>(d2), l2);
        if (n2 == 2 && w2 == 5) {
          const uint32_t w = static_cast<uint32_t>(v2);
          std::memcpy(&pc.score, &w, 4);
        }
        if (n2 == 3 && w2 == 0) pc.type = static_cast<int>(v2);
      } else if (num == 2 && w2 == 0) {
        if (n2 == 3) model_type = static_cast<int>(v2);
        if (n2 == 35) byte_fallback_ = v2 != 0;
        if (n2 == 40) unk_id_ = static_cast<int32_t>(v2);
        if (n2 == 41) bos_id_ = static_cast<int32_t>(v2);
        if (n2 == 42) eos_id_ = static_cast<int32_t>(v2);
      } else if (num == 3) {
        if (n2 == 1 && w2 == 2) norm_name.assign(reinterpret_cast<const char*>(d2), l2);
        if (n2 == 2 && w2 == 2) charsmap = l2 > 0;
        if (n2 == 3 && w2 == 0) add_dummy_prefix_ = v2 != 0;
        if (n2 == 4 && w2 == 0) remove_extra_whitespaces_ = v2 != 0;
        if (n2 == 5 && w2 == 0) escape_whitespaces_ = v2 != 0;
      }
    }
    if (num == 1) pieces_.push_back(std::move(pc));
  }
  if (pieces_.empty()) {
    status_ = base::error::ModelParseError("no pieces in SentencePiece model " + token_model_path_);
    return;
  }
  if (model_type != 2) {
    status_ = base::error::FunctionNotImplement("only SentencePiece BPE models are supported");
    return;
  }
  if (charsmap) {
    status_ = base::error::FunctionNotImplement("SentencePiece normaliser '" + norm_name +
                                                "' is not supported (identity only)");
    return;
  }
  for (size_t i = 0; i < pieces_.size(); ++i) {
    const Piece& pc = pieces_[i];
    if (pc.type == 1 || pc.type == 4 || pc.type == 5) index_.emplace(pc.text, static_cast<int32_t>(i));
    if (pc.type == 6 && pc.text.size() == 6 && pc.text.compare(0, 3, "<0x") == 0) {
      const int b = static_cast<int>(std::strtol(pc.text.substr(3, 2).c_str(), nullptr, 16));
      if (b >= 0 && b < 256) byte_ids_[b] = static_cast<int32_t>(i);
    }
  }
  const int32_t np = static_cast<int32_t>(pieces_.size());
  if (unk_id_ < 0 || unk_id_ >= np) unk_id_ = 0;
}

std::vector<int32_t> SpeEncodeLayer::encode(const std::string& sentence) const {
  std::vector<int32_t> ids;
  if (!status_) return ids;
  // Normalisation (identity rule): optional whitespace cleanup, the dummy
  // prefix, spaces escaped as U+2581.
  std::string text = sentence;
  if (remove_extra_whitespaces_) {
    std::string t;
    bool prev_space = true;
    for (char ch : text) {
      if (ch == ' ') {
        if (!prev_space) t += ' ';
        prev_space = true;
      } else {
        t += ch;
        prev_space = false;
      }
    }
    while (!t.empty() && t.back() == ' ') t.pop_back();
    text.swap(t);
  }
  if (has_bos_) ids.push_back(bos_id_);
  if (!text.empty()) {
    if (add_dummy_prefix_) text.insert(text.begin(), ' ');
    std::string norm;
    for (char ch : text) {
      if (ch == ' ' && escape_whitespaces_) norm += kSpaceSymbol;
      else norm += ch;
    }
    // Symbols: user-defined pieces (longest prefix match, never merged) or
    // single characters.
    struct Sym {
      std::string piece;
      int prev, next;
      bool freeze;
    };
    std::vector<Sym> sym;
    for (size_t i = 0; i < norm.size();) {
      size_t best = 0;
      for (size_t len = std::min<size_t>(norm.size() - i, 64); len > 0 && best == 0; --len) {
        const auto it = index_.find(norm.substr(i, len));
        if (it != index_.end() && pieces_[it->second].type == 4) best = len;
      }
      size_t j = i;
      if (best == 0) utf8_next(norm, j);
      const size_t len = best ? best : j - i;
      const int idx = static_cast<int>(sym.size());
      sym.push_back({norm.substr(i, len), idx - 1, -1, best > 0});
      if (idx > 0) sym[idx - 1].next = idx;
      i += len;
    }
    // Merge the adjacent pair whose joint piece scores highest (the leftmost
    // on ties) until no joint piece is in the vocabulary.
    struct Pair {
      int left, right;
      float score;
      size_t size;
    };
    auto worse = [](const Pair& a, const Pair& b) {
      return a.score < b.score || (a.score == b.score && a.left > b.left);
    };
    std::priority_queue<Pair, std::vector<Pair>, decltype(worse)> agenda(worse);
    auto add_pair = [&](int l, int r) {
      if (l < 0 || r < 0 || sym[l].freeze || sym[r].freeze) return;
      const std::string joint = sym[l].piece + sym[r].piece;
      const auto it = index_.find(joint);
      if (it == index_.end()) return;
      agenda.push({l, r, pieces_[it->second].score, joint.size()});
    };
    for (size_t i = 1; i < sym.size(); ++i) add_pair(static_cast<int>(i) - 1, static_cast<int>(i));
    while (!agenda.empty()) {
      const Pair top = agenda.top();
      agenda.pop();
      Sym& l = sym[top.left];
      Sym& r = sym[top.right];
      if (l.piece.empty() || r.piece.empty() || l.piece.size() + r.piece.size() != top.size) continue;
      l.piece += r.piece;
      r.piece.clear();
      l.next = r.next;
      if (r.next >= 0) sym[r.next].prev = top.left;
      add_pair(l.prev, top.left);
      add_pair(top.left, l.next);
    }
    // A run of unknown pieces becomes one unknown id, as the library merges
    // them (its decoder then renders one " \u2047 " per run).
    const size_t first = ids.size();
    auto push = [&](int32_t id) {
      if (id == unk_id_ && ids.size() > first && ids.back() == unk_id_) return;
      ids.push_back(id);
    };
    for (int i = sym.empty() ? -1 : 0; i >= 0; i = sym[i].next) {
      const auto it = index_.find(sym[i].piece);
      if (it != index_.end()) {
        push(it->second);
      } else if (byte_fallback_) {
        for (unsigned char b : sym[i].piece) push(byte_ids_[b] >= 0 ? byte_ids_[b] : unk_id_);
      } else {
        push(unk_id_);
      }
    }
  }
  if (has_eos_) ids.push_back(eos_id_);
  return ids;
}

std::string SpeEncodeLayer::decode(const std::vector<int32_t>& token_ids) const {
  std::string out;
  if (!status_) return out;
  std::string bytes;  // a run of byte pieces, decoded as UTF-8 together
  auto flush = [&]() {
    for (size_t i = 0; i < bytes.size();) {
      size_t j = i;
      const uint32_t cp = utf8_next(bytes, j);
      if (j == i + 1 && static_cast<unsigned char>(bytes[i]) >= 0x80) utf8_append(out, 0xFFFD);
      else utf8_append(out, cp);
      i = j;
    }
    bytes.clear();
  };
  bool first = true;
  for (int32_t id : token_ids) {
    if (id < 0 || id >= static_cast<int32_t>(pieces_.size())) continue;
    const Piece& pc = pieces_[id];
    if (pc.type == 3) continue;  // control (<s>, </s>) decodes to nothing
    if (pc.type == 6) {
      bytes += static_cast<char>(std::strtol(pc.text.substr(3, 2).c_str(), nullptr, 16));
      first = false;
      continue;
    }
    flush();
    std::string piece = pc.type == 2 ? std::string(" \xE2\x81\x87 ") : pc.text;
    if (first && add_dummy_prefix_ && piece.compare(0, 3, kSpaceSymbol) == 0) piece.erase(0, 3);
    first = false;
    for (size_t k = 0; k < piece.size();) {
      if (piece.compare(k, 3, kSpaceSymbol) == 0) {
        out += ' ';
        k += 3;
      } else {
        out += piece[k++];
      }
    }
  }
  flush();
  return out;
}

std::string SpeEncodeLayer::decode(int32_t token_id) const {
  return decode(std::vector<int32_t>{token_id});
}

bool SpeEncodeLayer::is_sentence_ending(int32_t token_id) const { return token_id == eos_id_; }

int32_t SpeEncodeLayer::vocab_size() const { return static_cast<int32_t>(pieces_.size()); }

// ====================================================== byte-level BPE ===
BpeEncodeLayer::BpeEncodeLayer(std::string token_model_path, bool has_bos, bool has_eos)
    : EncodeLayerBase(std::move(token_model_path), has_bos, has_eos) {
  load("<|begin_of_text|>", "<|end_of_text|>", "<|eot_id|>");
}

BpeEncodeLayer::BpeEncodeLayer(Deferred, std::string token_model_path, bool has_bos, bool has_eos)
    : EncodeLayerBase(std::move(token_model_path), has_bos, has_eos) {}

QwenEncodeLayer::QwenEncodeLayer(std::string token_model_path, bool has_bos, bool has_eos)
    : BpeEncodeLayer(Deferred{}, std::move(token_model_path), has_bos, has_eos) {
  load("<|im_start|>", "<|im_end|>", "<|endoftext|>");
}

void BpeEncodeLayer::load(const char* bos, const char* eos, const char* stop2) {
  std::string text;
  if (!read_file(token_model_path_, text)) {
    status_ = base::error::PathNotValid("cannot open the tokenizer file " + token_model_path_);
    return;
  }
  JValue root;
  if (!JsonReader(text.data(), text.data() + text.size()).parse(root) || root.kind != JValue::kObject) {
    status_ = base::error::ModelParseError("the tokenizer file is not valid JSON: " + token_model_path_);
    return;
  }
  const JValue* added = root.get("added_tokens");
  const JValue* model = root.get("model");
  const JValue* vocab = model ? model->get("vocab") : nullptr;
  if (!vocab || vocab->kind != JValue::kObject) {
    status_ = base::error::ModelParseError("no model.vocab in " + token_model_path_);
    return;
  }
  for (const auto& m : vocab->members) {
    std::string raw;
    bool ok = true;
    for (size_t i = 0; i < m.first.size();) {
      const int b = unicode_to_byte(utf8_next(m.first, i));
      if (b < 0) {
        ok = false;
        break;
      }
      raw += static_cast<char>(b);
    }
    if (!ok) continue;  // not in the byte-level alphabet
    const int32_t id = static_cast<int32_t>(m.second.number);
    encoder_[raw] = id;
    decoder_[id] = raw;
  }
  // Every single byte must have an id: the byte-pair merge falls back to
  // them (the reference would throw from tiktoken's ranks.at()).
  for (int b = 0; b < 256; ++b) {
    if (!encoder_.count(std::string(1, static_cast<char>(b)))) {
      encoder_.clear();
      decoder_.clear();
      status_ = base::error::ModelParseError("the vocabulary of " + token_model_path_ +
                                             " lacks the byte-level base tokens");
      return;
    }
  }
  std::unordered_map<std::string, int32_t> named;
  if (added && added->kind == JValue::kArray) {
    for (const JValue& t : added->items) {
      const JValue* id = t.get("id");
      const JValue* content = t.get("content");
      if (!id || !content) continue;
      // An empty special token would match at every position and never
      // advance the encoder, so such a file is refused.
      if (content->str.empty()) {
        encoder_.clear();
        decoder_.clear();
        special_.clear();
        special_decoder_.clear();
        status_ = base::error::ModelParseError("an added token of " + token_model_path_ +
                                               " has empty content");
        return;
      }
      special_.emplace_back(content->str, static_cast<int32_t>(id->number));
      special_decoder_[static_cast<int32_t>(id->number)] = content->str;
      named[content->str] = static_cast<int32_t>(id->number);
    }
  }
  // At one position the longest special token is taken.
  std::stable_sort(special_.begin(), special_.end(),
                   [](const auto& a, const auto& b) { return a.first.size() > b.first.size(); });
  auto id_of = [&](const char* name) {
    const auto it = named.find(name);
    return it == named.end() ? -1 : it->second;
  };
  bos_id_ = id_of(bos);
  eos_id_ = id_of(eos);
  stop_token1_ = eos_id_;
  stop_token2_ = id_of(stop2);
  num_token_ = static_cast<int32_t>(encoder_.size() + special_.size());
  status_ = base::error::Success();
}

// tiktoken's byte-pair merge: repeatedly join the adjacent parts whose bytes
// together have the lowest rank (the first such pair on ties).
void BpeEncodeLayer::byte_pair_merge(const std::string& piece, std::vector<int32_t>& out) const {
  if (piece.size() == 1) {
    out.push_back(encoder_.at(piece));
    return;
  }
  constexpr int32_t kNone = std::numeric_limits<int32_t>::max();
  std::vector<size_t> start(piece.size() + 1);
  for (size_t i = 0; i < start.size(); ++i) start[i] = i;
  auto rank_of = [&](size_t i, size_t skip) -> int32_t {
    if (i + skip + 2 < start.size()) {
      const auto it = encoder_.find(piece.substr(start[i], start[i + skip + 2] - start[i]));
      if (it != encoder_.end()) return it->second;
    }
    return kNone;
  };
  std::vector<int32_t> rank(start.size(), kNone);
  for (size_t i = 0; i + 2 < start.size(); ++i) rank[i] = rank_of(i, 0);
  while (start.size() > 2) {
    int32_t best = kNone;
    size_t bi = 0;
    for (size_t i = 0; i + 1 < start.size(); ++i)
      if (rank[i] < best) {
        best = rank[i];
        bi = i;
      }
    if (best == kNone) break;
    rank[bi] = rank_of(bi, 1);
    if (bi > 0) rank[bi - 1] = rank_of(bi - 1, 1);
    start.erase(start.begin() + bi + 1);
    rank.erase(rank.begin() + bi + 1);
  }
  for (size_t i = 0; i + 1 < start.size(); ++i)
    out.push_back(encoder_.at(piece.substr(start[i], start[i + 1] - start[i])));
}

std::vector<int32_t> BpeEncodeLayer::encode_ordinary(const std::string& text) const {
  std::vector<int32_t> out;
  std::vector<uint32_t> cps;
  std::vector<size_t> off;
  for (size_t i = 0; i < text.size();) {
    off.push_back(i);
    cps.push_back(utf8_next(text, i));
  }
  off.push_back(text.size());
  for (size_t i = 0; i < cps.size();) {
    const size_t j = piece_end(cps, i);
    const std::string piece = text.substr(off[i], off[j] - off[i]);
    const auto it = encoder_.find(piece);
    if (it != encoder_.end()) out.push_back(it->second);
    else byte_pair_merge(piece, out);
    i = j;
  }
  return out;
}

std::vector<int32_t> BpeEncodeLayer::encode(const std::string& sentence) const {
  std::vector<int32_t> ids;
  if (!status_) return ids;
  if (has_bos_) ids.push_back(bos_id_);
  // encode.cpp:110-112: every space becomes U+0120 before the split.
  std::string text;
  for (char ch : sentence) {
    if (ch == ' ') text += "\xC4\xA0";
    else text += ch;
  }
  size_t pos = 0;
  while (true) {
    // The next special token (tiktoken.h:167-187), longest at a position.
    size_t at = std::string::npos;
    const std::pair<std::string, int32_t>* hit = nullptr;
    for (const auto& s : special_) {
      const size_t f = text.find(s.first, pos);
      if (f != std::string::npos && (f < at || (f == at && s.first.size() > hit->first.size()))) {
        at = f;
        hit = &s;
      }
    }
    const std::vector<int32_t> part = encode_ordinary(text.substr(pos, (hit ? at : text.size()) - pos));
    ids.insert(ids.end(), part.begin(), part.end());
    if (!hit) break;
    ids.push_back(hit->second);
    pos = at + hit->first.size();
  }
  if (has_eos_) ids.push_back(eos_id_);
  return ids;
}

std::string BpeEncodeLayer::decode(const std::vector<int32_t>& token_ids) const {
  std::string bytes;
  for (int32_t id : token_ids) {
    const auto it = decoder_.find(id);
    if (it != decoder_.end()) {
      bytes += it->second;
      continue;
    }
    const auto sp = special_decoder_.find(id);
    if (sp != special_decoder_.end()) bytes += sp->second;
  }
  // encode.cpp:129-131: U+0120 back to a space.
  std::string out;
  for (size_t i = 0; i < bytes.size(); ++i) {
    if (i + 1 < bytes.size() && bytes[i] == '\xC4' && bytes[i + 1] == '\xA0') {
      out += ' ';
      ++i;
    } else {
      out += bytes[i];
    }
  }
  return out;
}

// encode.cpp:124: a single id decodes to nothing in the reference's BPE layer.
std::string BpeEncodeLayer::decode(int32_t token_id) const { return std::string(); }

bool BpeEncodeLayer::is_sentence_ending(int32_t token_id) const {
  return token_id == stop_token1_ || token_id == stop_token2_;
}

int32_t BpeEncodeLayer::vocab_size() const { return num_token_; }

}  // namespace op
