// The JSON reader of json.h.
#include "json.h"

#include <cstdio>
#include <cstdlib>
#include <stdexcept>

namespace msx::json {
namespace {

class Parser {
 public:
  explicit Parser(const std::string& t) : t_(t) {}

  Value document() {
    Value v = value(0);
    space();
    if (at_ != t_.size()) fail("text after the value");
    return v;
  }

 private:
  const std::string& t_;
  size_t at_ = 0;

  [[noreturn]] void fail(const std::string& what) const {
    throw std::runtime_error("JSON at byte " + std::to_string(at_) + ": " + what);
  }
  void space() {
    while (at_ < t_.size() && (t_[at_] == ' ' || t_[at_] == '\n' || t_[at_] == '\r' || t_[at_] == '\t')) ++at_;
  }
  bool take(char c) {
    space();
    if (at_ < t_.size() && t_[at_] == c) {
      ++at_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!take(c)) fail(std::string("expected '") + c + "'");
  }
  bool word(const char* w) {
    size_t n = std::char_traits<char>::length(w);
    if (t_.compare(at_, n, w) == 0) {
      at_ += n;
      return true;
    }
    return false;
  }

  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += char(cp);
    } else if (cp < 0x800) {
      out += char(0xC0 | (cp >> 6));
      out += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += char(0xE0 | (cp >> 12));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    } else {
      out += char(0xF0 | (cp >> 18));
      out += char(0x80 | ((cp >> 12) & 0x3F));
      out += char(0x80 | ((cp >> 6) & 0x3F));
      out += char(0x80 | (cp & 0x3F));
    }
  }
  uint32_t hex4() {
    if (at_ + 4 > t_.size()) fail("a short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      char c = t_[at_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= uint32_t(c - '0');
      else if (c >= 'a' && c <= 'f') v |= uint32_t(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= uint32_t(c - 'A' + 10);
      else fail("a bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (true) {
      if (at_ >= t_.size()) fail("an unterminated string");
      char c = t_[at_++];
      if (c == '"') return out;
      if (uint8_t(c) < 0x20) fail("a control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (at_ >= t_.size()) fail("an unterminated escape");
      char e = t_[at_++];
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
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {
            if (!word("\\u")) fail("a lone high surrogate");
            uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) fail("a bad low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: fail("an unknown escape");
      }
    }
  }
  Value value(int depth) {
    if (depth > 64) fail("nesting deeper than 64");
    space();
    if (at_ >= t_.size()) fail("a missing value");
    Value v;
    char c = t_[at_];
    if (c == '{') {
      ++at_;
      v.kind = Value::Object;
      if (take('}')) return v;
      do {
        space();
        std::string key = string();
        expect(':');
        v.fields.emplace_back(std::move(key), value(depth + 1));
      } while (take(','));
      expect('}');
    } else if (c == '[') {
      ++at_;
      v.kind = Value::Array;
      if (take(']')) return v;
      do v.items.push_back(value(depth + 1));
      while (take(','));
      expect(']');
    } else if (c == '"') {
      v.kind = Value::String;
      v.text = string();
    } else if (word("true")) {
      v.kind = Value::Bool;
      v.b = true;
    } else if (word("false")) {
      v.kind = Value::Bool;
    } else if (word("null")) {
      v.kind = Value::Null;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      size_t start = at_;
      if (t_[at_] == '-') ++at_;
      while (at_ < t_.size() && ((t_[at_] >= '0' && t_[at_] <= '9') || t_[at_] == '.' || t_[at_] == 'e' ||
                                 t_[at_] == 'E' || t_[at_] == '+' || t_[at_] == '-'))
        ++at_;
      v.kind = Value::Number;
      v.text = t_.substr(start, at_ - start);
      char* end = nullptr;
      v.num = std::strtod(v.text.c_str(), &end);
      if (!end || *end) fail("a malformed number");
    } else {
      fail("an unexpected character");
    }
    return v;
  }
};

}  // namespace

const Value* Value::find(const std::string& key) const {
  for (auto& [k, v] : fields)
    if (k == key) return &v;
  return nullptr;
}

const Value& Value::at(const std::string& key) const {
  if (kind != Object) throw std::runtime_error("`" + key + "` looked up in a value that is not an object");
  const Value* v = find(key);
  if (!v) throw std::runtime_error("no field `" + key + "`");
  return *v;
}

const std::string& Value::str() const {
  if (kind != String) throw std::runtime_error("a value that is not a string");
  return text;
}

double Value::number() const {
  if (kind != Number) throw std::runtime_error("a value that is not a number");
  return num;
}

uint64_t Value::u64() const {
  if (kind != Number || text.empty() || text[0] == '-' || text.find_first_of(".eE") != std::string::npos)
    throw std::runtime_error("a value that is not a whole number");
  if (text.size() > 20) throw std::runtime_error("a whole number beyond 64 bits");
  uint64_t v = 0;
  for (char c : text) {
    if (c < '0' || c > '9') throw std::runtime_error("a value that is not a whole number");
    uint64_t d = uint64_t(c - '0');
    if (v > (UINT64_MAX - d) / 10) throw std::runtime_error("a whole number beyond 64 bits");
    v = v * 10 + d;
  }
  return v;
}

Value parse(const std::string& text) { return Parser(text).document(); }

std::string quote(const std::string& s) {
  std::string out = "\"";
  for (char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (uint8_t(c) < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", unsigned(uint8_t(c)));
          out += buf;
        } else {
          out += c;
        }
    }
  }
  return out + "\"";
}

Value uint(uint64_t v) {
  Value x;
  x.kind = Value::Number;
  x.text = std::to_string(v);
  x.num = double(v);
  return x;
}

Value real(double v);  // defined with the checkpoint's f64 text

Value str(const std::string& s) {
  Value x;
  x.kind = Value::String;
  x.text = s;
  return x;
}

Value boolean(bool b) {
  Value x;
  x.kind = Value::Bool;
  x.b = b;
  return x;
}

Value array() {
  Value x;
  x.kind = Value::Array;
  return x;
}

Value object() {
  Value x;
  x.kind = Value::Object;
  return x;
}

Value& push(Value& a, Value v) {
  a.items.push_back(std::move(v));
  return a.items.back();
}

Value& put(Value& o, const std::string& key, Value v) {
  o.fields.emplace_back(key, std::move(v));
  return o.fields.back().second;
}

namespace {
void dump(const Value& v, int depth, std::string& out) {
  const std::string pad(size_t(2 * (depth + 1)), ' '), close(size_t(2 * depth), ' ');
  switch (v.kind) {
    case Value::Null: out += "null"; break;
    case Value::Bool: out += v.b ? "true" : "false"; break;
    case Value::Number: out += v.text; break;
    case Value::String: out += quote(v.text); break;
    case Value::Array:
      if (v.items.empty()) {
        out += "[]";
        break;
      }
      out += "[\n";
      for (size_t i = 0; i < v.items.size(); ++i) {
        out += pad;
        dump(v.items[i], depth + 1, out);
        out += i + 1 < v.items.size() ? ",\n" : "\n";
      }
      out += close + "]";
      break;
    case Value::Object:
      if (v.fields.empty()) {
        out += "{}";
        break;
      }
      out += "{\n";
      for (size_t i = 0; i < v.fields.size(); ++i) {
        out += pad + quote(v.fields[i].first) + ": ";
        dump(v.fields[i].second, depth + 1, out);
        out += i + 1 < v.fields.size() ? ",\n" : "\n";
      }
      out += close + "}";
      break;
  }
}
}  // namespace

std::string dump_pretty(const Value& v) {
  std::string out;
  dump(v, 0, out);
  return out;
}

}  // namespace msx::json
