// Minimal JSON reader for safetensors headers and config.json (objects, arrays, strings, numbers, literals).
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace ijah::json {

struct Value {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  int64_t inum = 0;  // exact integer when the token had no fraction / exponent
  std::string str;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;  // insertion order kept

  const Value *get(const std::string &k) const {
    for (auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

// Throws ijah::Error on malformed input.
Value parse(const std::string &text);

}  // namespace ijah::json
