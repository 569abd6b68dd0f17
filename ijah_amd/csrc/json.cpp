// Minimal JSON reader (see json.h). Recursive descent over the UTF-8 text; \u escapes become UTF-8.
#include "json.h"

#include <cstdlib>
#include <cstring>

#include "common.h"

namespace ijah::json {
namespace {

struct Parser {
  const std::string &s;
  size_t i = 0;

  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\n' || s[i] == '\r' || s[i] == '\t')) i++;
  }
  [[noreturn]] void fail(const char *what) { throw Error(strfmt("json: %s at offset %zu", what, i)); }
  char peek() {
    ws();
    if (i >= s.size()) fail("unexpected end");
    return s[i];
  }
  void expect(char c) {
    if (peek() != c) fail("unexpected character");
    i++;
  }

  static void put_utf8(std::string &o, uint32_t cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | (cp >> 6));
      o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      o += (char)(0xE0 | (cp >> 12));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    } else {
      o += (char)(0xF0 | (cp >> 18));
      o += (char)(0x80 | ((cp >> 12) & 0x3F));
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (i + 4 > s.size()) fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
      const char c = s[i++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string o;
    while (true) {
      if (i >= s.size()) fail("unterminated string");
      const char c = s[i++];
      if (c == '"') break;
      if (c != '\\') {
        o += c;
        continue;
      }
      if (i >= s.size()) fail("bad escape");
      const char e = s[i++];
      switch (e) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && i + 1 < s.size() && s[i] == '\\' && s[i + 1] == 'u') {
            i += 2;
            const uint32_t lo = hex4();
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(o, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
    return o;
  }
  Value value() {
    Value v;
    const char c = peek();
    if (c == '{') {
      i++;
      v.kind = Value::Obj;
      if (peek() == '}') {
        i++;
        return v;
      }
      while (true) {
        std::string k = string();
        expect(':');
        v.obj.emplace_back(std::move(k), value());
        const char d = peek();
        i++;
        if (d == '}') break;
        if (d != ',') fail("expected , or }");
      }
    } else if (c == '[') {
      i++;
      v.kind = Value::Arr;
      if (peek() == ']') {
        i++;
        return v;
      }
      while (true) {
        v.arr.push_back(value());
        const char d = peek();
        i++;
        if (d == ']') break;
        if (d != ',') fail("expected , or ]");
      }
    } else if (c == '"') {
      v.kind = Value::Str;
      v.str = string();
    } else if (c == 't' && s.compare(i, 4, "true") == 0) {
      i += 4;
      v.kind = Value::Bool;
      v.b = true;
    } else if (c == 'f' && s.compare(i, 5, "false") == 0) {
      i += 5;
      v.kind = Value::Bool;
    } else if (c == 'n' && s.compare(i, 4, "null") == 0) {
      i += 4;
    } else {
      const size_t st = i;
      bool integral = true;
      if (s[i] == '-') i++;
      while (i < s.size() && ((s[i] >= '0' && s[i] <= '9') || s[i] == '.' || s[i] == 'e' || s[i] == 'E' ||
                              s[i] == '+' || s[i] == '-')) {
        if (s[i] == '.' || s[i] == 'e' || s[i] == 'E') integral = false;
        i++;
      }
      if (i == st) fail("unexpected character");
      const std::string tok = s.substr(st, i - st);
      v.kind = Value::Num;
      v.num = strtod(tok.c_str(), nullptr);
      v.inum = integral ? strtoll(tok.c_str(), nullptr, 10) : (int64_t)v.num;
    }
    return v;
  }
};

}  // namespace

Value parse(const std::string &text) {
  Parser p{text};
  Value v = p.value();
  p.ws();
  if (p.i != text.size()) p.fail("trailing characters");
  return v;
}

}  // namespace ijah::json
