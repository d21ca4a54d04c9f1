// Minimal JSON value for diagnostics and reports. Every diagnostic is a JSON document, for
// programs and people alike; the reference builds the same document shapes with serde_json
// (src/graph.rs:229-239).
#pragma once
#include <charconv>
#include <cmath>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace rg {

class Json {
 public:
  enum class Kind { Null, Bool, Int, Num, Str, Arr, Obj };
  Json() : k_(Kind::Null) {}
  Json(std::nullptr_t) : k_(Kind::Null) {}
  Json(bool b) : k_(Kind::Bool), b_(b) {}
  Json(int v) : k_(Kind::Int), i_(v) {}
  Json(long v) : k_(Kind::Int), i_(v) {}
  Json(long long v) : k_(Kind::Int), i_(v) {}
  Json(unsigned v) : k_(Kind::Int), i_(v) {}
  Json(unsigned long v) : k_(Kind::Int), i_((int64_t)v) {}
  Json(unsigned long long v) : k_(Kind::Int), i_((int64_t)v) {}
  Json(double v) : k_(Kind::Num), d_(v) {}
  Json(const char* s) : k_(Kind::Str), s_(s) {}
  Json(std::string s) : k_(Kind::Str), s_(std::move(s)) {}
  template <class T>
  Json(const std::vector<T>& v) : k_(Kind::Arr) {
    for (auto& x : v) a_.push_back(Json(x));
  }
  static Json arr() {
    Json j;
    j.k_ = Kind::Arr;
    return j;
  }
  static Json obj() {
    Json j;
    j.k_ = Kind::Obj;
    return j;
  }
  Kind kind() const { return k_; }
  bool is_null() const { return k_ == Kind::Null; }
  Json& operator[](const std::string& key) {
    if (k_ == Kind::Null) k_ = Kind::Obj;
    for (auto& kv : o_)
      if (kv.first == key) return kv.second;
    o_.emplace_back(key, Json());
    return o_.back().second;
  }
  const Json* get(const std::string& key) const {
    for (auto& kv : o_)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  void push(Json v) {
    if (k_ == Kind::Null) k_ = Kind::Arr;
    a_.push_back(std::move(v));
  }
  std::vector<Json>& items() { return a_; }
  const std::vector<Json>& items() const { return a_; }
  const std::string& str() const { return s_; }
  bool operator==(const char* s) const { return k_ == Kind::Str && s_ == s; }
  std::string dump() const {
    std::string out;
    write(out);
    return out;
  }

 private:
  static void esc(std::string& out, const std::string& s) {
    out += '"';
    for (unsigned char c : s) {
      switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
          if (c < 0x20) {
            char buf[8];
            snprintf(buf, sizeof buf, "\\u%04x", c);
            out += buf;
          } else {
            out += (char)c;
          }
      }
    }
    out += '"';
  }
  void write(std::string& out) const {
    switch (k_) {
      case Kind::Null: out += "null"; break;
      case Kind::Bool: out += b_ ? "true" : "false"; break;
      case Kind::Int: out += std::to_string(i_); break;
      case Kind::Num: {
        if (!std::isfinite(d_)) {
          out += "null";
          break;
        }
        char buf[64];
        auto r = std::to_chars(buf, buf + sizeof buf, d_);
        std::string s(buf, r.ptr);
        if (s.find_first_of(".eE") == std::string::npos) s += ".0";
        out += s;
        break;
      }
      case Kind::Str: esc(out, s_); break;
      case Kind::Arr: {
        out += '[';
        for (size_t i = 0; i < a_.size(); i++) {
          if (i) out += ',';
          a_[i].write(out);
        }
        out += ']';
        break;
      }
      case Kind::Obj: {
        out += '{';
        for (size_t i = 0; i < o_.size(); i++) {
          if (i) out += ',';
          esc(out, o_[i].first);
          out += ':';
          o_[i].second.write(out);
        }
        out += '}';
        break;
      }
    }
  }
  Kind k_;
  bool b_ = false;
  int64_t i_ = 0;
  double d_ = 0;
  std::string s_;
  std::vector<Json> a_;
  std::vector<std::pair<std::string, Json>> o_;
};

// Non-finite doubles have no JSON number form; they are written as strings (src/validate.rs:28-39).
inline Json num(double x) {
  if (std::isfinite(x)) return Json(x);
  if (std::isnan(x)) return Json("nan");
  return Json(x > 0 ? "inf" : "-inf");
}

inline Json diag(const std::string& code, const std::string& severity, Json node, Json observation,
                 const std::string& cause, const std::string& certainty) {
  Json d = Json::obj();
  d["status"] = severity == "error" ? "validation_failed" : "warning";
  d["severity"] = severity;
  d["code"] = code;
  d["node"] = std::move(node);
  d["observation"] = std::move(observation);
  Json dx = Json::obj();
  dx["cause"] = cause;
  dx["certainty"] = certainty;
  d["diagnosis"] = std::move(dx);
  return d;
}

// A diagnostic travels as an exception through the engine and becomes rg.DiagnosticError.
struct DiagError {
  Json d;
};

}  // namespace rg
