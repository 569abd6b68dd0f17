// Minimal JSON reader (see json.h) for safetensors headers and config.json.
//
// Two layers: a scanner that turns the text into tokens (punctuation, string, number, literal), and a builder that
// assembles values with an explicit stack of open containers instead of recursion, so a deeply nested header cannot
// exhaust the C++ stack. String escapes are decoded into a list of UTF-16 code units first; surrogate pairs are then
// joined while those units are encoded as UTF-8.
#include "json.h"

#include <cerrno>
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace ijah::json {
namespace {

enum class Tok { LBrace, RBrace, LBrack, RBrack, Colon, Comma, String, Number, True, False, Null, End };

struct Token {
  Tok kind = Tok::End;
  size_t at = 0;         // byte offset of the token in the text
  std::string text;      // decoded string, or the number's characters
};

[[noreturn]] void bad(size_t at, const char *why) { throw Error(strfmt("json parse error (byte %zu): %s", at, why)); }

int hex_digit(char c) {
  if (c >= '0' && c <= '9') return c - '0';
  const char l = (char)(c | 0x20);
  if (l >= 'a' && l <= 'f') return 10 + (l - 'a');
  return -1;
}

// UTF-16 code units -> UTF-8; a high surrogate followed by a low one becomes one code point, a lone surrogate is
// encoded as its own 3-byte sequence.
void units_to_utf8(const std::vector<uint32_t> &u, std::string &out) {
  for (size_t k = 0; k < u.size(); k++) {
    uint32_t cp = u[k];
    if (cp >= 0xD800 && cp <= 0xDBFF && k + 1 < u.size() && u[k + 1] >= 0xDC00 && u[k + 1] <= 0xDFFF) {
      cp = 0x10000 + (((cp & 0x3FF) << 10) | (u[k + 1] & 0x3FF));
      k++;
    }
    const int n = cp < 0x80 ? 1 : cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
    static const uint8_t lead[5] = {0, 0x00, 0xC0, 0xE0, 0xF0};
    char buf[4];
    for (int b = n - 1; b > 0; b--) {
      buf[b] = (char)(0x80 | (cp & 0x3F));
      cp >>= 6;
    }
    buf[0] = (char)(lead[n] | cp);
    out.append(buf, (size_t)n);
  }
}

class Scanner {
 public:
  explicit Scanner(const std::string &t) : t_(t) {}

  Token next() {
    while (pos_ < t_.size() && strchr(" \t\r\n", t_[pos_]) && t_[pos_] != '\0') pos_++;
    Token k;
    k.at = pos_;
    if (pos_ >= t_.size()) return k;
    const char c = t_[pos_];
    switch (c) {
      case '{': pos_++; k.kind = Tok::LBrace; return k;
      case '}': pos_++; k.kind = Tok::RBrace; return k;
      case '[': pos_++; k.kind = Tok::LBrack; return k;
      case ']': pos_++; k.kind = Tok::RBrack; return k;
      case ':': pos_++; k.kind = Tok::Colon; return k;
      case ',': pos_++; k.kind = Tok::Comma; return k;
      case '"': k.kind = Tok::String; k.text = scan_string(); return k;
      default: break;
    }
    for (const auto &lit : {std::make_pair("true", Tok::True), std::make_pair("false", Tok::False),
                            std::make_pair("null", Tok::Null)}) {
      const size_t n = strlen(lit.first);
      if (t_.compare(pos_, n, lit.first) == 0) {
        pos_ += n;
        k.kind = lit.second;
        return k;
      }
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      const size_t st = pos_;
      while (pos_ < t_.size() && strchr("0123456789+-.eE", t_[pos_]) && t_[pos_] != '\0') pos_++;
      k.kind = Tok::Number;
      k.text = t_.substr(st, pos_ - st);
      return k;
    }
    bad(pos_, "no value starts with this character");
  }

 private:
  std::string scan_string() {
    const size_t open = pos_++;
    std::string out;
    std::vector<uint32_t> units;  // pending \u escapes (joined at the next plain character or the end)
    auto flush = [&] {
      units_to_utf8(units, out);
      units.clear();
    };
    while (true) {
      if (pos_ >= t_.size()) bad(open, "string has no closing quote");
      const char c = t_[pos_++];
      if (c == '"') break;
      if (c != '\\') {
        flush();
        out += c;
        continue;
      }
      if (pos_ >= t_.size()) bad(pos_, "backslash at end of text");
      const char e = t_[pos_++];
      if (e == 'u') {
        uint32_t v = 0;
        for (int d = 0; d < 4; d++) {
          const int h = pos_ < t_.size() ? hex_digit(t_[pos_]) : -1;
          if (h < 0) bad(pos_, "\\u needs four hex digits");
          v = v * 16 + (uint32_t)h;
          pos_++;
        }
        units.push_back(v);
        continue;
      }
      static const char from[] = "\"\\/bfnrt", to[] = "\"\\/\b\f\n\r\t";
      const char *hit = strchr(from, e);
      if (!hit || e == '\0') bad(pos_ - 1, "unknown escape letter");
      flush();
      out += to[hit - from];
    }
    flush();
    return out;
  }

  const std::string &t_;
  size_t pos_ = 0;
};

Value number_value(const Token &k) {
  Value v;
  v.kind = Value::Num;
  const char *b = k.text.c_str();
  char *end = nullptr;
  errno = 0;
  v.num = strtod(b, &end);
  if (end == b || *end != '\0') bad(k.at, "malformed number");
  const bool plain_int = k.text.find_first_of(".eE") == std::string::npos;
  if (plain_int) {
    const long long i = strtoll(b, &end, 10);
    v.inum = (errno == ERANGE) ? (int64_t)v.num : (int64_t)i;
  } else {
    v.inum = (int64_t)v.num;
  }
  return v;
}

}  // namespace

Value parse(const std::string &text) {
  Scanner sc(text);
  // open containers; for an object, the key waiting for its value
  struct Open {
    Value v;
    std::string key;
    bool have_key = false;
  };
  std::vector<Open> stack;
  Value root;
  bool done = false;
  // where a finished value goes: into the innermost open container, or it is the document
  auto place = [&](Value &&v, size_t at) {
    if (stack.empty()) {
      if (done) bad(at, "more than one top-level value");
      root = std::move(v);
      done = true;
      return;
    }
    Open &o = stack.back();
    if (o.v.kind == Value::Arr) {
      o.v.arr.push_back(std::move(v));
    } else {
      if (!o.have_key) bad(at, "object member without a key");
      o.v.obj.emplace_back(std::move(o.key), std::move(v));
      o.have_key = false;
    }
  };
  enum class Want { Value, KeyOrClose, Key, Colon, CommaOrClose, ValueOrClose } want = Want::Value;
  while (true) {
    Token k = sc.next();
    if (k.kind == Tok::End) {
      if (!done || !stack.empty()) bad(k.at, "text ends inside a value");
      return root;
    }
    if (done && stack.empty()) bad(k.at, "extra text after the top-level value");
    switch (want) {
      case Want::KeyOrClose:
      case Want::Key:
        if (k.kind == Tok::RBrace && want == Want::KeyOrClose) break;
        if (k.kind != Tok::String) bad(k.at, "expected a member name");
        stack.back().key = std::move(k.text);
        stack.back().have_key = true;
        want = Want::Colon;
        continue;
      case Want::Colon:
        if (k.kind != Tok::Colon) bad(k.at, "expected ':' after a member name");
        want = Want::Value;
        continue;
      case Want::CommaOrClose:
        if (k.kind == Tok::Comma) {
          want = stack.back().v.kind == Value::Obj ? Want::Key : Want::Value;
          continue;
        }
        if (k.kind != Tok::RBrace && k.kind != Tok::RBrack) bad(k.at, "expected ',' or a closing bracket");
        break;
      case Want::ValueOrClose:
        if (k.kind == Tok::RBrack) break;
        [[fallthrough]];
      case Want::Value:
        break;
    }
    // closing brackets
    if (k.kind == Tok::RBrace || k.kind == Tok::RBrack) {
      if (stack.empty()) bad(k.at, "unbalanced closing bracket");
      const Value::Kind need = k.kind == Tok::RBrace ? Value::Obj : Value::Arr;
      if (stack.back().v.kind != need) bad(k.at, "closing bracket does not match");
      Value v = std::move(stack.back().v);
      stack.pop_back();
      place(std::move(v), k.at);
      want = Want::CommaOrClose;
      continue;
    }
    // a value
    Value v;
    switch (k.kind) {
      case Tok::LBrace:
        stack.push_back(Open{});
        stack.back().v.kind = Value::Obj;
        want = Want::KeyOrClose;
        continue;
      case Tok::LBrack:
        stack.push_back(Open{});
        stack.back().v.kind = Value::Arr;
        want = Want::ValueOrClose;
        continue;
      case Tok::String: v.kind = Value::Str; v.str = std::move(k.text); break;
      case Tok::Number: v = number_value(k); break;
      case Tok::True: v.kind = Value::Bool; v.b = true; break;
      case Tok::False: v.kind = Value::Bool; v.b = false; break;
      case Tok::Null: break;
      default: bad(k.at, "expected a value");
    }
    place(std::move(v), k.at);
    want = Want::CommaOrClose;
  }
}

}  // namespace ijah::json
