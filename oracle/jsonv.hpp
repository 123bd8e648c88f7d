// Minimal JSON reader for the oracle (test infrastructure, independent of the product's
// parser). Numbers are parsed with strtod, which is correctly rounded, so every f64
// literal in the IR arrives bit-identical to the double the front end serialised.
#pragma once
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace orc {

struct JV {
  enum T { NUL, BOOL, NUM, STR, ARR, OBJ } t = NUL;
  bool b = false;
  double n = 0;
  std::string s;
  std::vector<JV> a;
  std::vector<std::pair<std::string, JV>> o;

  bool is_null() const { return t == NUL; }
  const JV* find(const std::string& k) const {
    for (auto& kv : o) if (kv.first == k) return &kv.second;
    return nullptr;
  }
  const JV& operator[](const std::string& k) const {
    const JV* v = find(k);
    if (!v) throw std::runtime_error("json: missing key '" + k + "'");
    return *v;
  }
  const JV& operator[](size_t i) const { return a.at(i); }
  double num() const { if (t != NUM) throw std::runtime_error("json: not a number"); return n; }
  long long i64() const { return (long long)num(); }
  int i32() const { return (int)num(); }
  const std::string& str() const { if (t != STR) throw std::runtime_error("json: not a string"); return s; }
};

class JParser {
 public:
  explicit JParser(const char* p) : p_(p) {}
  JV parse() { JV v = value(); ws(); if (*p_) throw std::runtime_error("json: trailing data"); return v; }

 private:
  const char* p_;
  void ws() { while (*p_ == ' ' || *p_ == '\n' || *p_ == '\t' || *p_ == '\r') ++p_; }
  JV value() {
    ws();
    JV v;
    char c = *p_;
    if (c == '{') {
      ++p_; v.t = JV::OBJ; ws();
      if (*p_ == '}') { ++p_; return v; }
      for (;;) {
        ws(); std::string k = str(); ws();
        if (*p_++ != ':') throw std::runtime_error("json: expected ':'");
        v.o.emplace_back(k, value()); ws();
        if (*p_ == ',') { ++p_; continue; }
        if (*p_ == '}') { ++p_; return v; }
        throw std::runtime_error("json: expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_; v.t = JV::ARR; ws();
      if (*p_ == ']') { ++p_; return v; }
      for (;;) {
        v.a.push_back(value()); ws();
        if (*p_ == ',') { ++p_; continue; }
        if (*p_ == ']') { ++p_; return v; }
        throw std::runtime_error("json: expected ',' or ']'");
      }
    }
    if (c == '"') { v.t = JV::STR; v.s = str(); return v; }
    if (!strncmp(p_, "true", 4)) { p_ += 4; v.t = JV::BOOL; v.b = true; return v; }
    if (!strncmp(p_, "false", 5)) { p_ += 5; v.t = JV::BOOL; v.b = false; return v; }
    if (!strncmp(p_, "null", 4)) { p_ += 4; v.t = JV::NUL; return v; }
    char* end = nullptr;
    v.n = strtod(p_, &end);
    if (end == p_) throw std::runtime_error("json: bad value");
    v.t = JV::NUM; p_ = end;
    return v;
  }
  std::string str() {
    if (*p_ != '"') throw std::runtime_error("json: expected string");
    ++p_;
    std::string out;
    while (*p_ && *p_ != '"') {
      if (*p_ == '\\') {
        ++p_;
        char e = *p_++;
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {
            unsigned cp = (unsigned)strtoul(std::string(p_, 4).c_str(), nullptr, 16); p_ += 4;
            if (cp < 0x80) out += (char)cp;
            else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 63)); }
            else { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
            break;
          }
          default: out += e;
        }
      } else {
        out += *p_++;
      }
    }
    if (*p_ != '"') throw std::runtime_error("json: unterminated string");
    ++p_;
    return out;
  }
};

inline JV parse_json(const char* s) { return JParser(s).parse(); }

}  // namespace orc
