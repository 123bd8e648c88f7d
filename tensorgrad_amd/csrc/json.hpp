// Small JSON DOM for the runtime's IR document. Numbers go through strtod (correctly
// rounded), so the f64 scalars baked into IR ops arrive exactly as serialised.
#pragma once
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace tgj {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool boolean = false;
  double number = 0;
  std::string string;
  std::vector<Value> items;
  std::vector<std::pair<std::string, Value>> members;

  bool null() const { return kind == Null; }
  const Value* get(const std::string& key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
  const Value& at(const std::string& key) const {
    const Value* v = get(key);
    if (!v) throw std::runtime_error("IR: missing field '" + key + "'");
    return *v;
  }
  double num() const {
    if (kind != Number) throw std::runtime_error("IR: expected a number");
    return number;
  }
  int64_t i64() const { return (int64_t)num(); }
  int i32() const { return (int)num(); }
  const std::string& str() const {
    if (kind != String) throw std::runtime_error("IR: expected a string");
    return string;
  }
};

class Reader {
 public:
  explicit Reader(const char* s) : p_(s) {}
  Value document() {
    Value v = value();
    skip();
    if (*p_) throw std::runtime_error("IR: trailing characters after JSON document");
    return v;
  }

 private:
  const char* p_;
  void skip() {
    while (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t') ++p_;
  }
  void expect(char c) {
    skip();
    if (*p_ != c) throw std::runtime_error(std::string("IR: expected '") + c + "'");
    ++p_;
  }
  std::string text() {
    expect('"');
    std::string out;
    for (;;) {
      char c = *p_++;
      if (c == '\0') throw std::runtime_error("IR: unterminated string");
      if (c == '"') break;
      if (c != '\\') { out += c; continue; }
      char e = *p_++;
      if (e == 'u') {
        unsigned cp = 0;
        for (int i = 0; i < 4; ++i) {
          char h = *p_++;
          cp = cp * 16 + (unsigned)(h <= '9' ? h - '0' : (h | 32) - 'a' + 10);
        }
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 63)); }
        else { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
      } else {
        out += e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
      }
    }
    return out;
  }
  Value value() {
    skip();
    Value v;
    if (*p_ == '{') {
      ++p_;
      v.kind = Value::Object;
      skip();
      if (*p_ == '}') { ++p_; return v; }
      for (;;) {
        std::string k = text();
        expect(':');
        v.members.emplace_back(std::move(k), value());
        skip();
        if (*p_ == ',') { ++p_; continue; }
        expect('}');
        return v;
      }
    }
    if (*p_ == '[') {
      ++p_;
      v.kind = Value::Array;
      skip();
      if (*p_ == ']') { ++p_; return v; }
      for (;;) {
        v.items.push_back(value());
        skip();
        if (*p_ == ',') { ++p_; continue; }
        expect(']');
        return v;
      }
    }
    if (*p_ == '"') { v.kind = Value::String; v.string = text(); return v; }
    if (!strncmp(p_, "true", 4)) { p_ += 4; v.kind = Value::Bool; v.boolean = true; return v; }
    if (!strncmp(p_, "false", 5)) { p_ += 5; v.kind = Value::Bool; return v; }
    if (!strncmp(p_, "null", 4)) { p_ += 4; return v; }
    char* end = nullptr;
    v.number = strtod(p_, &end);
    if (end == p_) throw std::runtime_error("IR: malformed JSON value");
    v.kind = Value::Number;
    p_ = end;
    return v;
  }
};

inline Value parse(const char* s) { return Reader(s).document(); }

// Serialise a document (numbers with 17 significant digits, so they read back exactly).
inline void dump_to(const Value& v, std::string& o) {
  switch (v.kind) {
    case Value::Null: o += "null"; return;
    case Value::Bool: o += v.boolean ? "true" : "false"; return;
    case Value::Number: { char b[32]; snprintf(b, sizeof b, "%.17g", v.number); o += b; return; }
    case Value::String:
      o += '"';
      for (char c : v.string) {
        if (c == '"' || c == '\\') { o += '\\'; o += c; }
        else if ((unsigned char)c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); o += b; }
        else o += c;
      }
      o += '"';
      return;
    case Value::Array:
      o += '[';
      for (size_t i = 0; i < v.items.size(); ++i) { if (i) o += ','; dump_to(v.items[i], o); }
      o += ']';
      return;
    case Value::Object:
      o += '{';
      for (size_t i = 0; i < v.members.size(); ++i) {
        if (i) o += ',';
        Value k; k.kind = Value::String; k.string = v.members[i].first;
        dump_to(k, o);
        o += ':';
        dump_to(v.members[i].second, o);
      }
      o += '}';
      return;
  }
}
inline std::string dump(const Value& v) { std::string o; dump_to(v, o); return o; }

}  // namespace tgj
