// Parameter sets from the reference's JSON layout (parameters/*.json, read by
// unittest/Testbed.h:95-179): log_degree, log_default_scale,
// default_encryption_level, main_primes, terminal_primes (optional),
// auxiliary_primes, level_config, additional_base (optional),
// dense_hamming_weight / sparse_hamming_weight (optional); keys for
// bootstrapping are accepted and ignored. A small recursive-descent reader
// for the JSON subset these files use (objects, arrays, integers, booleans,
// strings, null).
#include <cctype>
#include <cstdint>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "cheddar.h"

namespace cheddar {

namespace {

struct JValue {
  enum Kind { kNull, kBool, kInt, kFloat, kString, kArray, kObject } kind = kNull;
  bool b = false;
  int64_t i = 0;
  uint64_t u = 0;  // magnitude for non-negative integers up to 2^64 - 1
  bool neg = false;
  double f = 0;
  std::string s;
  std::vector<JValue> arr;
  std::map<std::string, JValue> obj;
};

class Reader {
 public:
  explicit Reader(const std::string &t) : t_(t) {}
  JValue Parse() {
    JValue v = Value();
    Skip();
    Check(p_ == t_.size(), "trailing characters");
    return v;
  }

 private:
  void Check(bool c, const std::string &what) const {
    if (!c)
      throw Error("JSON parameter file: " + what + " at offset " +
                  std::to_string(p_));
  }
  void Skip() {
    while (p_ < t_.size() && std::isspace(static_cast<unsigned char>(t_[p_])))
      p_++;
  }
  bool Eat(char c) {
    Skip();
    if (p_ < t_.size() && t_[p_] == c) {
      p_++;
      return true;
    }
    return false;
  }
  bool Word(const char *w) {
    const std::string s(w);
    if (t_.compare(p_, s.size(), s) == 0) {
      p_ += s.size();
      return true;
    }
    return false;
  }
  JValue Value() {
    Skip();
    Check(p_ < t_.size(), "unexpected end");
    JValue v;
    const char c = t_[p_];
    if (c == '{') {
      p_++;
      v.kind = JValue::kObject;
      if (Eat('}')) return v;
      do {
        Skip();
        Check(p_ < t_.size() && t_[p_] == '"', "expected a key");
        const std::string k = String();
        Check(Eat(':'), "expected ':'");
        v.obj[k] = Value();
      } while (Eat(','));
      Check(Eat('}'), "expected '}'");
    } else if (c == '[') {
      p_++;
      v.kind = JValue::kArray;
      if (Eat(']')) return v;
      do v.arr.push_back(Value());
      while (Eat(','));
      Check(Eat(']'), "expected ']'");
    } else if (c == '"') {
      v.kind = JValue::kString;
      v.s = String();
    } else if (Word("true")) {
      v.kind = JValue::kBool;
      v.b = true;
    } else if (Word("false")) {
      v.kind = JValue::kBool;
    } else if (Word("null")) {
      v.kind = JValue::kNull;
    } else {
      Number(v);
    }
    return v;
  }
  std::string String() {
    p_++;  // opening quote
    std::string s;
    while (p_ < t_.size() && t_[p_] != '"') {
      if (t_[p_] == '\\') {
        p_++;
        Check(p_ < t_.size(), "bad escape");
      }
      s.push_back(t_[p_++]);
    }
    Check(p_ < t_.size(), "unterminated string");
    p_++;
    return s;
  }
  void Number(JValue &v) {
    const size_t start = p_;
    if (p_ < t_.size() && (t_[p_] == '-' || t_[p_] == '+')) p_++;
    bool is_float = false;
    while (p_ < t_.size() &&
           (std::isdigit(static_cast<unsigned char>(t_[p_])) || t_[p_] == '.' ||
            t_[p_] == 'e' || t_[p_] == 'E' || t_[p_] == '-' || t_[p_] == '+')) {
      if (!std::isdigit(static_cast<unsigned char>(t_[p_]))) is_float = true;
      p_++;
    }
    const std::string num = t_.substr(start, p_ - start);
    Check(!num.empty() && num != "-" && num != "+", "expected a value");
    if (is_float) {
      v.kind = JValue::kFloat;
      v.f = std::stod(num);
      return;
    }
    v.kind = JValue::kInt;
    v.neg = num[0] == '-';
    const std::string digits = num.substr(num[0] == '-' || num[0] == '+');
    uint64_t u = 0;
    for (char d : digits) {
      const uint64_t x = static_cast<uint64_t>(d - '0');
      Check(u <= (std::numeric_limits<uint64_t>::max() - x) / 10,
            "integer out of range");
      u = u * 10 + x;
    }
    v.u = u;
    v.i = v.neg ? -static_cast<int64_t>(u) : static_cast<int64_t>(u);
  }

  const std::string &t_;
  size_t p_ = 0;
};

void Need(bool c, const std::string &msg) {
  if (!c) throw Error(msg);
}

const JValue &Field(const JValue &root, const char *name) {
  auto it = root.obj.find(name);
  Need(it != root.obj.end(),
       std::string("Missing ") + name + " in JSON file");
  return it->second;
}

int IntField(const JValue &root, const char *name) {
  const JValue &v = Field(root, name);
  Need(v.kind == JValue::kInt && v.i >= std::numeric_limits<int>::min() &&
           v.i <= std::numeric_limits<int>::max(),
       std::string(name) + " should be an integer");
  return static_cast<int>(v.i);
}

std::vector<uint32_t> PrimeArray(const JValue &v, const char *name) {
  Need(v.kind == JValue::kArray, std::string(name) + " should be an array");
  std::vector<uint32_t> r;
  for (const JValue &p : v.arr) {
    Need(p.kind == JValue::kInt && !p.neg,
         std::string(name) + " should be an array of integers");
    Need(p.u < (uint64_t{1} << 32),
         std::string(name) + ": prime " + std::to_string(p.u) +
             " does not fit the 32-bit word of this build");
    r.push_back(static_cast<uint32_t>(p.u));
  }
  return r;
}

}  // namespace

// unittest/Testbed.h:95-179 (the checks and their messages), then the
// Parameter constructor of Parameter.h:42-47
std::unique_ptr<Parameter<uint32_t>> ParameterFromJson(
    const std::string &text) {
  const JValue root = Reader(text).Parse();
  Need(root.kind == JValue::kObject, "JSON parameter file: not an object");
  const int log_degree = IntField(root, "log_degree");
  const int log_scale = IntField(root, "log_default_scale");
  Need(log_scale >= 0 && log_scale < 64, "log_default_scale out of range");
  const double scale = static_cast<double>(uint64_t{1} << log_scale);
  const int del = IntField(root, "default_encryption_level");
  const std::vector<uint32_t> main_p =
      PrimeArray(Field(root, "main_primes"), "main_primes");
  std::vector<uint32_t> ter_p;
  if (root.obj.count("terminal_primes"))
    ter_p = PrimeArray(root.obj.at("terminal_primes"), "terminal_primes");
  const std::vector<uint32_t> aux_p =
      PrimeArray(Field(root, "auxiliary_primes"), "auxiliary_primes");
  const JValue &lc = Field(root, "level_config");
  Need(lc.kind == JValue::kArray, "level_config should be an array");
  std::vector<std::pair<int, int>> levels;
  for (const JValue &pr : lc.arr) {
    Need(pr.kind == JValue::kArray && pr.arr.size() == 2 &&
             pr.arr[0].kind == JValue::kInt && pr.arr[1].kind == JValue::kInt,
         "level_config should be an array of pairs");
    levels.emplace_back(static_cast<int>(pr.arr[0].i),
                        static_cast<int>(pr.arr[1].i));
  }
  std::pair<int, int> additional{0, 0};
  if (root.obj.count("additional_base")) {
    const JValue &ab = root.obj.at("additional_base");
    Need(ab.kind == JValue::kArray && ab.arr.size() == 2 &&
             ab.arr[0].kind == JValue::kInt && ab.arr[1].kind == JValue::kInt,
         "additional_base should be an array of pairs");
    additional = {static_cast<int>(ab.arr[0].i),
                  static_cast<int>(ab.arr[1].i)};
  }
  for (const char *k : {"dense_hamming_weight", "sparse_hamming_weight"})
    if (root.obj.count(k))
      Need(root.obj.at(k).kind == JValue::kInt,
           std::string(k) + " should be an integer");
  return std::make_unique<Parameter<uint32_t>>(
      log_degree, scale, del, levels, main_p, aux_p, ter_p, additional);
}

}  // namespace cheddar
