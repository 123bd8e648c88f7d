// safetensors container: index a buffer and write one. Host code only.
//
// Layout (the format's published definition): an 8-byte little-endian u64 header length
// N, an N-byte JSON header mapping each tensor name to {dtype, shape, data_offsets:
// [begin, end]} with byte offsets relative to the data blob that follows the header, and
// an optional "__metadata__" object of string values.
//
// Reading follows the reference loader (src/safetensors.ts:49-103): F32 tensors load;
// integer / bool tensors are skipped and reported; any other dtype is refused; a short
// buffer, a header past the end, invalid JSON, offsets out of range and a byte length
// that disagrees with the shape are errors, with the reference's messages.
#pragma once
#include <cstdint>
#include <cstring>
#include <map>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"

namespace tgst {

struct Entry {
  std::string name, dtype;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;   // byte offsets relative to the data blob
  // Element count, or -1 when the product of the dimensions overflows int64.
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape)
      if (__builtin_mul_overflow(n, d, &n)) return -1;
    return n;
  }
};

struct Index {
  std::vector<Entry> tensors;   // F32 tensors, header order
  std::vector<Entry> skipped;   // integer / bool tensors (shape kept, data never read)
  std::vector<std::pair<std::string, std::string>> metadata;
  int64_t data_start = 0;       // 8 + header length
  const Entry* find(const std::string& n) const {
    for (const Entry& e : tensors)
      if (e.name == n) return &e;
    return nullptr;
  }
  const std::string* meta(const std::string& k) const {
    for (const auto& m : metadata)
      if (m.first == k) return &m.second;
    return nullptr;
  }
};

inline bool integer_dtype(const std::string& d) {
  static const std::set<std::string> k = {"I64", "I32", "I16", "I8", "U8", "U16", "U32", "U64", "BOOL"};
  return k.count(d) > 0;
}

// Index a container held in memory. `raw_i32_ok` additionally accepts I32 tensors as
// loadable (used for runtime checkpoints, whose i32 state is stored as I32).
inline Index parse(const uint8_t* buf, uint64_t len, bool raw_i32_ok = false) {
  if (len < 8) throw std::runtime_error("loadSafetensors: buffer too small to hold the 8-byte header length");
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | buf[i];
  if (hlen > len - 8)
    throw std::runtime_error("loadSafetensors: header length " + std::to_string(hlen) + " exceeds buffer (" +
                             std::to_string(len) + " bytes)");
  const int64_t header_end = 8 + (int64_t)hlen;
  std::string text(reinterpret_cast<const char*>(buf + 8), (size_t)hlen);
  tgj::Value h;
  try {
    h = tgj::parse(text.c_str());
  } catch (std::exception& e) {
    throw std::runtime_error(std::string("loadSafetensors: header is not valid JSON: ") + e.what());
  }
  if (h.kind != tgj::Value::Object) throw std::runtime_error("loadSafetensors: header is not valid JSON: not an object");
  Index ix;
  ix.data_start = header_end;
  for (const auto& m : h.members) {
    const std::string& name = m.first;
    const tgj::Value& v = m.second;
    if (name == "__metadata__") {
      if (v.kind == tgj::Value::Object)
        for (const auto& kv : v.members)
          if (kv.second.kind == tgj::Value::String) ix.metadata.emplace_back(kv.first, kv.second.str());
      continue;
    }
    if (v.kind != tgj::Value::Object) throw std::runtime_error("loadSafetensors: tensor '" + name + "' entry is not an object");
    Entry e;
    e.name = name;
    const tgj::Value* dt = v.get("dtype");
    const tgj::Value* sh = v.get("shape");
    const tgj::Value* off = v.get("data_offsets");
    if (!dt || dt->kind != tgj::Value::String || !sh || sh->kind != tgj::Value::Array || !off ||
        off->kind != tgj::Value::Array || off->items.size() != 2)
      throw std::runtime_error("loadSafetensors: tensor '" + name + "' entry is malformed");
    e.dtype = dt->str();
    // JSON numbers arrive as doubles: only integers below 2^53 are exact, and only those
    // are converted (a larger value cannot be a valid size or offset of a buffer here).
    auto exact_count = [](const tgj::Value& x) {
      return x.kind == tgj::Value::Number && x.number >= 0 && x.number < 9007199254740992.0 &&
             x.number == (double)(int64_t)x.number;
    };
    for (const auto& d : sh->items) {
      if (!exact_count(d)) throw std::runtime_error("loadSafetensors: tensor '" + name + "' has a malformed shape");
      e.shape.push_back(d.i64());
    }
    for (const auto& o : off->items)
      if (!exact_count(o)) throw std::runtime_error("loadSafetensors: tensor '" + name + "' has malformed data_offsets");
    e.begin = off->items[0].i64();
    e.end = off->items[1].i64();
    if (e.dtype != "F32" && !(raw_i32_ok && e.dtype == "I32")) {
      if (integer_dtype(e.dtype)) { ix.skipped.push_back(e); continue; }
      throw std::runtime_error("loadSafetensors: tensor '" + name + "' has dtype '" + e.dtype +
                               "', but tensorgrad is f32-only. Convert the checkpoint to f32 offline before loading "
                               "(see README \"Constraints\").");
    }
    if (e.begin > e.end || (uint64_t)header_end + (uint64_t)e.end > len)
      throw std::runtime_error("loadSafetensors: tensor '" + name + "' data_offsets [" + std::to_string(e.begin) + ", " +
                               std::to_string(e.end) + "] out of range");
    const int64_t numel = e.numel();
    int64_t bytes = -1;
    if (numel < 0 || __builtin_mul_overflow(numel, (int64_t)4, &bytes))
      throw std::runtime_error("loadSafetensors: tensor '" + name + "' has a shape whose element count overflows");
    if (e.end - e.begin != bytes) {
      std::string s;
      for (size_t i = 0; i < e.shape.size(); ++i) s += (i ? ", " : "") + std::to_string(e.shape[i]);
      throw std::runtime_error("loadSafetensors: tensor '" + name + "' byte length " + std::to_string(e.end - e.begin) +
                               " != " + std::to_string(e.numel()) + " f32 elements * 4 (shape [" + s + "])");
    }
    ix.tensors.push_back(std::move(e));
  }
  return ix;
}

inline std::string quote(const std::string& s) {
  std::string o = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') { o += '\\'; o += c; }
    else if ((unsigned char)c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); o += b; }
    else o += c;
  }
  return o + "\"";
}

// Header for tensors laid out back to back in the given order, padded with spaces so
// the data blob starts on an 8-byte boundary (the format's convention).
struct OutTensor { std::string name, dtype; std::vector<int64_t> shape; int64_t bytes; };
inline std::string header(const std::vector<OutTensor>& ts, const std::vector<std::pair<std::string, std::string>>& meta) {
  std::ostringstream o;
  o << "{";
  bool first = true;
  if (!meta.empty()) {
    o << "\"__metadata__\":{";
    for (size_t i = 0; i < meta.size(); ++i) o << (i ? "," : "") << quote(meta[i].first) << ":" << quote(meta[i].second);
    o << "}";
    first = false;
  }
  int64_t off = 0;
  for (const auto& t : ts) {
    o << (first ? "" : ",") << quote(t.name) << ":{\"dtype\":\"" << t.dtype << "\",\"shape\":[";
    for (size_t i = 0; i < t.shape.size(); ++i) o << (i ? "," : "") << t.shape[i];
    o << "],\"data_offsets\":[" << off << "," << off + t.bytes << "]}";
    off += t.bytes;
    first = false;
  }
  o << "}";
  std::string h = o.str();
  while ((8 + h.size()) % 8) h += ' ';
  std::string out(8, '\0');
  uint64_t n = h.size();
  for (int i = 0; i < 8; ++i) out[i] = (char)((n >> (8 * i)) & 0xFF);
  return out + h;
}

}  // namespace tgst
