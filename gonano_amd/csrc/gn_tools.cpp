// gn_tools.cpp - calculator tool and byte-level token codec used by the
// rollout state machine (inference/engine.go:279-297).
#include "gn_tools.h"
#include "gn_common.h"

#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace gn {

static const char* kSpecialNames[11] = {
    "<|bos|>", "<|user_start|>", "<|user_end|>", "<|assistant_start|>", "<|assistant_end|>",
    "<|tool_start|>", "<|tool_end|>", "<|tool_output_start|>", "<|tool_output_end|>",
    "<|think_start|>", "<|think_end|>"};

std::string decode_tokens(const std::vector<int>& ids) {
  std::string out;
  for (int id : ids) {
    if (id >= 0 && id < 256) out.push_back((char)(unsigned char)id);
    else if (id >= 256 && id < TOKENIZER_VOCAB) out += kSpecialNames[id - 256];
  }
  return out;
}

std::vector<int> encode_bytes(const std::string& s) {
  std::vector<int> ids;
  ids.reserve(s.size());
  for (unsigned char c : s) ids.push_back(c);
  return ids;
}

namespace {

// Recursive-descent arithmetic over + - * / ( ) and unary minus with
// float64 values; division by zero rejects the expression
// (inference/tooluse.go:156-184).
class Arith {
 public:
  explicit Arith(const std::string& s) : s_(s) {}
  bool parse(double* out) {
    if (!expr(out)) return false;
    space();
    return p_ == s_.size();
  }

 private:
  void space() {
    while (p_ < s_.size() && s_[p_] == ' ') p_++;
  }
  bool expr(double* out) {
    double v;
    if (!term(&v)) return false;
    for (;;) {
      space();
      if (p_ >= s_.size() || (s_[p_] != '+' && s_[p_] != '-')) break;
      char op = s_[p_++];
      double r;
      if (!term(&r)) return false;
      v = op == '+' ? v + r : v - r;
    }
    *out = v;
    return true;
  }
  bool term(double* out) {
    double v;
    if (!factor(&v)) return false;
    for (;;) {
      space();
      if (p_ >= s_.size() || (s_[p_] != '*' && s_[p_] != '/')) break;
      char op = s_[p_++];
      double r;
      if (!factor(&r)) return false;
      if (op == '*') v *= r;
      else {
        if (r == 0) return false;
        v /= r;
      }
    }
    *out = v;
    return true;
  }
  bool factor(double* out) {
    space();
    if (p_ >= s_.size()) return false;
    if (s_[p_] == '-') {
      p_++;
      double v;
      bool ok = factor(&v);
      *out = -v;
      return ok;
    }
    if (s_[p_] == '(') {
      p_++;
      double v;
      if (!expr(&v)) return false;
      space();
      if (p_ >= s_.size() || s_[p_] != ')') return false;
      p_++;
      *out = v;
      return true;
    }
    return number(out);
  }
  // Digits accumulate as v*10+d; fraction digits add d*f with f *= 0.1, in
  // float64, in that order (not strtod), so results match the reference bit
  // for bit.
  bool number(double* out) {
    size_t start = p_;
    bool seen = false;
    while (p_ < s_.size() && isdigit((unsigned char)s_[p_])) { p_++; seen = true; }
    if (p_ < s_.size() && s_[p_] == '.') {
      p_++;
      while (p_ < s_.size() && isdigit((unsigned char)s_[p_])) { p_++; seen = true; }
    }
    if (!seen) return false;
    double v = 0, f = 0.1;
    bool integer = true;
    for (size_t i = start; i < p_; i++) {
      if (s_[i] == '.') { integer = false; f = 0.1; continue; }
      double d = (double)(s_[i] - '0');
      if (integer) v = v * 10 + d;
      else { v += d * f; f *= 0.1; }
    }
    *out = v;
    return true;
  }
  const std::string& s_;
  size_t p_ = 0;
};

// formatNumber (inference/tooluse.go:186-191): integral values print as an
// int64; others use the shortest round-tripping digits in plain notation,
// like strconv.FormatFloat(v, 'f', -1, 64).
std::string format_number(double v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "+Inf" : "-Inf";
  if (v >= -9.2233720368547758e18 && v < 9.2233720368547758e18 && v == (double)(int64_t)v) {
    char b[32];
    snprintf(b, sizeof b, "%lld", (long long)(int64_t)v);
    return b;
  }
  char buf[64];
  for (int prec = 1; prec <= 17; prec++) {
    snprintf(buf, sizeof buf, "%.*e", prec - 1, v);
    if (strtod(buf, nullptr) == v) break;
  }
  std::string digits;
  bool neg = false;
  const char* c = buf;
  if (*c == '-') { neg = true; c++; }
  for (; *c && *c != 'e'; c++)
    if (isdigit((unsigned char)*c)) digits.push_back(*c);
  int point = atoi(c + 1) + 1;
  std::string out = neg ? "-" : "";
  if (point <= 0) {
    out += "0.";
    out.append((size_t)(-point), '0');
    out += digits;
  } else {
    for (int i = 0; i < point; i++) out.push_back(i < (int)digits.size() ? digits[i] : '0');
    if ((int)digits.size() > point) out += "." + digits.substr((size_t)point);
  }
  return out;
}

bool unquote(const std::string& t, std::string* out) {
  if (t.size() < 2) return false;
  char a = t.front(), b = t.back();
  if ((a == '"' && b == '"') || (a == '\'' && b == '\'')) {
    *out = t.substr(1, t.size() - 2);
    return true;
  }
  return false;
}

std::string trim(const std::string& s) {
  size_t a = 0, b = s.size();
  while (a < b && isspace((unsigned char)s[a])) a++;
  while (b > a && isspace((unsigned char)s[b - 1])) b--;
  return s.substr(a, b - a);
}

}  // namespace

std::optional<std::string> calculator(const std::string& expr_in) {
  std::string e;
  for (char c : expr_in)
    if (c != ',') e.push_back(c);
  // arithmetic (inference/tooluse.go:93-102)
  bool arith = !e.empty();
  for (char c : e)
    if (!(isdigit((unsigned char)c) || strchr("*+-/.() ", c) != nullptr) || c == 0) arith = false;
  if (arith) {
    if (e.find("**") != std::string::npos) return std::nullopt;
    double v;
    Arith p(e);
    if (p.parse(&v)) return format_number(v);
    return std::nullopt;
  }
  // "literal".count("sub") (inference/tooluse.go:104-144)
  for (char c : e) {
    bool ok = isalnum((unsigned char)c) || c == '\'' || c == '"' || c == '.' || c == '(' ||
              c == ')' || c == '_' || c == ' ';
    if (!ok || (unsigned char)c >= 128) return std::nullopt;
  }
  std::string lower = e;
  for (auto& c : lower) c = (char)tolower((unsigned char)c);
  static const char* forbidden[] = {"__",   "import", "exec",    "eval",    "compile", "open",
                                    "file", "input",  "globals", "locals",  "vars",    "dir",
                                    "getattr", "setattr", "delattr", "hasattr"};
  for (auto f : forbidden)
    if (lower.find(f) != std::string::npos) return std::nullopt;
  size_t dot = e.find(".count(");
  if (dot == std::string::npos) return std::nullopt;
  std::string lit = trim(e.substr(0, dot));
  std::string arg = trim(e.substr(dot + 7));
  if (arg.empty() || arg.back() != ')') return std::nullopt;
  arg = trim(arg.substr(0, arg.size() - 1));
  std::string text, sub;
  if (!unquote(lit, &text) || !unquote(arg, &sub)) return std::nullopt;
  long long count = 0;
  if (sub.empty()) count = (long long)text.size() + 1;
  else
    for (size_t i = 0; i + sub.size() <= text.size();) {
      if (text.compare(i, sub.size(), sub) == 0) { count++; i += sub.size(); }
      else i++;
    }
  return format_number((double)count);
}

}  // namespace gn

extern "C" int gn_use_calculator(const char* expression, char* out, size_t cap, int32_t* ok) {
  if (!expression || !out || !ok || cap == 0) {
    gn::set_last_error("gn_use_calculator: null argument");
    return GN_ERR_INVALID;
  }
  auto res = gn::calculator(expression);
  *ok = res ? 1 : 0;
  out[0] = 0;
  if (!res) return GN_OK;
  if (res->size() + 1 > cap) {
    gn::set_last_error("gn_use_calculator: result longer than the output buffer");
    return GN_ERR_INVALID;
  }
  memcpy(out, res->c_str(), res->size() + 1);
  return GN_OK;
}
