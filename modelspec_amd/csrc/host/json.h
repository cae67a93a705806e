// A small JSON reader for the records of a packed directory (binding.json, packed.json): objects,
// arrays, strings with the escapes JSON defines, numbers (kept as their text and as a double),
// true, false and null. Enough for the files a packed directory holds; no streaming.
#pragma once
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace msx::json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0;
  std::string text;  // a string's value, or a number's text as written
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> fields;  // in file order

  // The field `key` of an object; throws std::runtime_error naming `key` when absent.
  const Value& at(const std::string& key) const;
  const Value* find(const std::string& key) const;
  const std::string& str() const;
  double number() const;
  // A whole number in [0, 2^64) written without fraction or exponent.
  uint64_t u64() const;
};

// Parses `text`; throws std::runtime_error with the byte offset of the first error.
Value parse(const std::string& text);

// Builders: a number keeps the text it was made with.
Value uint(uint64_t v);
Value real(double v);  // serde_json's text of an f64
Value str(const std::string& s);
Value boolean(bool b);
Value array();
Value object();
// Appends to an array / object; returns the added value.
Value& push(Value& array, Value v);
Value& put(Value& object, const std::string& key, Value v);

// serde_json's pretty form: two-space indent, "key": value, empty containers as [] and {}.
std::string dump_pretty(const Value& v);

// `s` as a JSON string literal.
std::string quote(const std::string& s);

}  // namespace msx::json
