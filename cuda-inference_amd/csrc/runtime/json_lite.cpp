// Recursive-descent JSON parser and serializer (no third-party dependency).
#include "gpu_inference/json_lite.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>

#include "gpu_inference/error.h"

namespace gie {
namespace json {

Value& Value::operator[](const std::string& key) {
  if (type_ == Type::kNull) type_ = Type::kObject;
  if (type_ != Type::kObject) throw Error(StatusCode::kInternal, "json: operator[] on a non-object");
  for (auto& kv : obj_)
    if (kv.first == key) return kv.second;
  obj_.emplace_back(key, Value());
  return obj_.back().second;
}

const Value* Value::find(const std::string& key) const {
  if (type_ != Type::kObject) return nullptr;
  for (const auto& kv : obj_)
    if (kv.first == key) return &kv.second;
  return nullptr;
}

namespace {

void escape_to(std::string& out, const std::string& s) {
  out.push_back('"');
  for (unsigned char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", c);
          out += buf;
        } else {
          out.push_back(char(c));
        }
    }
  }
  out.push_back('"');
}

void newline(std::string& out, int indent, int level) {
  if (indent < 0) return;
  out.push_back('\n');
  out.append(size_t(indent * level), ' ');
}

class Parser {
 public:
  explicit Parser(const std::string& t) : t_(t) {}
  Value parse_document() {
    ws();
    Value v = value();
    ws();
    if (i_ != t_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const std::string& what) const {
    size_t line = 1, col = 1;
    for (size_t k = 0; k < i_ && k < t_.size(); ++k) {
      if (t_[k] == '\n') {
        ++line;
        col = 1;
      } else {
        ++col;
      }
    }
    std::ostringstream os;
    os << "json parse error at line " << line << ", column " << col << ": " << what;
    throw Error(StatusCode::kIo, os.str());
  }
  void ws() {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\n' || t_[i_] == '\r' || t_[i_] == '\t')) ++i_;
  }
  bool eat(char c) {
    if (i_ < t_.size() && t_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  void expect_word(const char* w) {
    for (const char* p = w; *p; ++p)
      if (!eat(*p)) fail(std::string("expected '") + w + "'");
  }
  Value value() {
    if (i_ >= t_.size()) fail("unexpected end of input");
    const char c = t_[i_];
    if (c == '{') return object();
    if (c == '[') return array();
    if (c == '"') return Value(string());
    if (c == 't') { expect_word("true"); return Value(true); }
    if (c == 'f') { expect_word("false"); return Value(false); }
    if (c == 'n') { expect_word("null"); return Value(); }
    if (c == '-' || (c >= '0' && c <= '9')) return number();
    fail(std::string("unexpected character '") + c + "'");
  }
  Value object() {
    Value v = Value::object();
    eat('{');
    ws();
    if (eat('}')) return v;
    for (;;) {
      ws();
      if (i_ >= t_.size() || t_[i_] != '"') fail("expected a string key");
      std::string k = string();
      ws();
      if (!eat(':')) fail("expected ':'");
      ws();
      v[k] = value();
      ws();
      if (eat(',')) continue;
      if (eat('}')) return v;
      fail("expected ',' or '}'");
    }
  }
  Value array() {
    Value v = Value::array();
    eat('[');
    ws();
    if (eat(']')) return v;
    for (;;) {
      ws();
      v.push_back(value());
      ws();
      if (eat(',')) continue;
      if (eat(']')) return v;
      fail("expected ',' or ']'");
    }
  }
  static void put_utf8(std::string& out, unsigned cp) {
    if (cp < 0x80) {
      out.push_back(char(cp));
    } else if (cp < 0x800) {
      out.push_back(char(0xC0 | (cp >> 6)));
      out.push_back(char(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      out.push_back(char(0xE0 | (cp >> 12)));
      out.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
      out.push_back(char(0x80 | (cp & 0x3F)));
    } else {
      out.push_back(char(0xF0 | (cp >> 18)));
      out.push_back(char(0x80 | ((cp >> 12) & 0x3F)));
      out.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
      out.push_back(char(0x80 | (cp & 0x3F)));
    }
  }
  unsigned hex4() {
    if (i_ + 4 > t_.size()) fail("truncated \\u escape");
    unsigned v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = t_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= unsigned(c - '0');
      else if (c >= 'a' && c <= 'f') v |= unsigned(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= unsigned(c - 'A' + 10);
      else fail("bad hex digit in \\u escape");
    }
    return v;
  }
  std::string string() {
    eat('"');
    std::string out;
    for (;;) {
      if (i_ >= t_.size()) fail("unterminated string");
      const char c = t_[i_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) fail("control character in string");
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (i_ >= t_.size()) fail("unterminated escape");
      const char e = t_[i_++];
      switch (e) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && i_ + 1 < t_.size() && t_[i_] == '\\' && t_[i_ + 1] == 'u') {
            i_ += 2;
            const unsigned lo = hex4();
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
  }
  Value number() {
    const size_t start = i_;
    eat('-');
    if (i_ >= t_.size() || !(t_[i_] >= '0' && t_[i_] <= '9')) fail("bad number");
    while (i_ < t_.size() && ((t_[i_] >= '0' && t_[i_] <= '9') || t_[i_] == '.' || t_[i_] == 'e' || t_[i_] == 'E' ||
                              t_[i_] == '+' || t_[i_] == '-'))
      ++i_;
    const std::string s = t_.substr(start, i_ - start);
    char* end = nullptr;
    const double v = std::strtod(s.c_str(), &end);
    if (end == s.c_str() || *end != '\0') fail("bad number '" + s + "'");
    return Value(v);
  }
  const std::string& t_;
  size_t i_ = 0;
};

}  // namespace

void Value::dump_to(std::string& out, int indent, int level) const {
  switch (type_) {
    case Type::kNull: out += "null"; break;
    case Type::kBool: out += bool_ ? "true" : "false"; break;
    case Type::kNumber: {
      if (!std::isfinite(num_)) {
        out += "null";
      } else if (num_ == std::floor(num_) && std::fabs(num_) < 9.0e15) {
        out += std::to_string(int64_t(num_));
      } else {
        char buf[40];
        std::snprintf(buf, sizeof(buf), "%.17g", num_);
        out += buf;
      }
      break;
    }
    case Type::kString: escape_to(out, str_); break;
    case Type::kArray: {
      out.push_back('[');
      for (size_t k = 0; k < arr_.size(); ++k) {
        if (k) out.push_back(',');
        newline(out, indent, level + 1);
        arr_[k].dump_to(out, indent, level + 1);
      }
      if (!arr_.empty()) newline(out, indent, level);
      out.push_back(']');
      break;
    }
    case Type::kObject: {
      out.push_back('{');
      for (size_t k = 0; k < obj_.size(); ++k) {
        if (k) out.push_back(',');
        newline(out, indent, level + 1);
        escape_to(out, obj_[k].first);
        out += indent >= 0 ? ": " : ":";
        obj_[k].second.dump_to(out, indent, level + 1);
      }
      if (!obj_.empty()) newline(out, indent, level);
      out.push_back('}');
      break;
    }
  }
}

std::string Value::dump(int indent) const {
  std::string out;
  dump_to(out, indent, 0);
  return out;
}

Value parse(const std::string& text) { return Parser(text).parse_document(); }

Value parse_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw Error(StatusCode::kIo, "cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return parse(ss.str());
}

void write_file(const std::string& path, const Value& v, int indent) {
  const std::string tmp = path + ".tmp" + std::to_string(std::rand());
  {
    std::ofstream f(tmp, std::ios::binary | std::ios::trunc);
    if (!f) throw Error(StatusCode::kIo, "cannot write " + tmp);
    f << v.dump(indent) << "\n";
    if (!f) throw Error(StatusCode::kIo, "write failed for " + tmp);
  }
  if (std::rename(tmp.c_str(), path.c_str()) != 0) {
    std::remove(tmp.c_str());
    throw Error(StatusCode::kIo, "cannot rename " + tmp + " -> " + path);
  }
}

}  // namespace json
}  // namespace gie
