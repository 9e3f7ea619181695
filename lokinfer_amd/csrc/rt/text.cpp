// Model text: the reference's line-oriented model format (lariaus/lokinfer docs/impl-notes/design-ir.md §5, §7),
// printed and parsed so that print(parse(print(m))) == print(m).
//
//   model {
//     init -> buffer<f32[4]> { ... return %w }
//     exec(%x: buffer<f32[N]>, %kv: buffer<f32[8]> mutable) state(%w2: buffer<f32[4]>) -> buffer<f32[N]> {
//       %o = buffer.alloc {output = true} : buffer<f32[N]>
//       kernel "add_f32_gpu"(%x, %x) outs(%o) {alpha = 1.0}
//       return %o
//     }
//   }
//
// Printing: a formatter per op kind (a table indexed by OpKind) appends one line; values get their names on first
// mention. Parsing: a lexer turns the whole text into tokens first (a dim keeps its exact source span, so the dim
// parser sees the text as written), then a recursive-descent reader walks the tokens and dispatches each op on its
// keyword through a table.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unordered_set>

#include "ir.h"

namespace lkrt {

namespace {

// ---- number formats ----------------------------------------------------------------------------------------------

// IEEE half -> float: subnormals are m * 2^-24, normals (1024 + m) * 2^(e - 25).
float halfToFloat(uint16_t h) {
  const int e = (h >> 10) & 31, m = h & 1023;
  const float sign = (h & 0x8000u) ? -1.0f : 1.0f;
  if (e == 31) return m ? std::nanf("") : sign * INFINITY;
  if (e == 0) return sign * std::ldexp(static_cast<float>(m), -24);
  return sign * std::ldexp(static_cast<float>(1024 + m), e - 25);
}

// float -> IEEE half, round to nearest even (the scaled significand is rounded by nearbyint in the default mode).
uint16_t floatToHalf(float f) {
  const uint16_t sign = std::signbit(f) ? 0x8000u : 0;
  if (std::isnan(f)) return sign | 0x7e00u;
  const float a = std::fabs(f);
  if (a >= 65520.0f) return sign | 0x7c00u;
  if (a < std::ldexp(1.0f, -14))  // subnormal range: units of 2^-24
    return sign | static_cast<uint16_t>(std::nearbyint(std::ldexp(a, 24)));
  int e;
  std::frexp(a, &e);  // a = x * 2^e, x in [0.5, 1): the half exponent is e - 1
  e -= 1;
  int q = static_cast<int>(std::nearbyint(std::ldexp(a, 10 - e)));  // 1024 .. 2048
  if (q == 2048) {
    q = 1024;
    ++e;
  }
  if (e + 15 >= 31) return sign | 0x7c00u;
  return sign | static_cast<uint16_t>(((e + 15) << 10) | (q - 1024));
}

float bf16ToFloat(uint16_t h) {
  const uint32_t bits = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// float -> bfloat16, round to nearest even on the 16 dropped bits; NaN stays a quiet NaN.
uint16_t floatToBf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if (std::isnan(f)) return static_cast<uint16_t>((x >> 16) | 0x40u);
  const uint32_t hi = x >> 16, lo = x & 0xffffu;
  const bool up = lo > 0x8000u || (lo == 0x8000u && (hi & 1u));
  return static_cast<uint16_t>(hi + (up ? 1u : 0u));
}

// %.<digits>g, with ".0" added to a bare integer; nan / inf / -inf spelled out
std::string numberText(double v, int digits) {
  if (std::isnan(v)) return "nan";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  char buf[48];
  std::snprintf(buf, sizeof buf, "%.*g", digits, v);
  std::string s(buf);
  return s.find('.') == std::string::npos && s.find('e') == std::string::npos ? s + ".0" : s;
}

std::string quote(std::string_view s) {
  std::string q(1, '"');
  for (char c : s) {
    if (c == '\\' || c == '"') q.push_back('\\');
    q.push_back(c);
  }
  q.push_back('"');
  return q;
}

// One element of const.inline data as the text shows it.
std::string elementText(DType t, const uint8_t* p) {
  auto load = [p](auto v) {
    std::memcpy(&v, p, sizeof v);
    return v;
  };
  switch (t) {
    case DType::F32: return numberText(load(0.0f), 9);
    case DType::F16: return numberText(halfToFloat(load(uint16_t{0})), 9);
    case DType::BF16: return numberText(bf16ToFloat(load(uint16_t{0})), 9);
    case DType::I8: return std::to_string(load(int8_t{0}));
    case DType::U8: return std::to_string(load(uint8_t{0}));
    case DType::Bool: return p[0] ? "1" : "0";
    case DType::I16: return std::to_string(load(int16_t{0}));
    case DType::I32: return std::to_string(load(int32_t{0}));
    case DType::I64: return std::to_string(load(int64_t{0}));
  }
  return "?";
}

// ---- printer -----------------------------------------------------------------------------------------------------

struct Printer {
  const Model& m;
  std::string out;
  std::unordered_map<ValueId, std::string> given;  // value -> "%name"
  std::unordered_set<std::string> used;
  int nextNumber = 0;

  // A value prints under its name hint, made unique by _1, _2, ...; a value without a hint takes the lowest free
  // number.
  const std::string& ref(ValueId v) {
    if (auto it = given.find(v); it != given.end()) return it->second;
    const std::string& hint = m.nameOf(v);
    std::string n = hint;
    if (hint.empty()) {
      for (n = std::to_string(nextNumber++); used.count(n); n = std::to_string(nextNumber++)) {
      }
    } else {
      for (int k = 1; used.count(n); ++k) n = hint + "_" + std::to_string(k);
    }
    used.insert(n);
    return given[v] = "%" + n;
  }
  std::string typeText(ValueId v) const { return m.types().str(m.typeOf(v)); }

  void refs(const std::vector<ValueId>& vs) {
    for (size_t i = 0; i < vs.size(); ++i) {
      if (i) out += ", ";
      out += ref(vs[i]);
    }
  }
  void typed(const std::vector<ValueId>& vs, const Region* flags) {
    for (size_t i = 0; i < vs.size(); ++i) {
      if (i) out += ", ";
      out += ref(vs[i]);
      out += ": ";
      out += typeText(vs[i]);
      if (flags && flags->isMutable(i)) out += " mutable";
    }
  }
  // " -> T" or " -> (T, U)" from the region's return; nothing for an empty return
  void header(const Region& r) {
    if (r.ops.empty() || r.ops.back().kind != OpKind::Return || r.ops.back().operands.empty()) return;
    const auto& ret = r.ops.back().operands;
    out += ret.size() == 1 ? " -> " : " -> (";
    for (size_t i = 0; i < ret.size(); ++i) out += (i ? ", " : "") + typeText(ret[i]);
    if (ret.size() != 1) out += ")";
  }
  std::string attrText(const AttrValue& a) const {
    struct V {
      const Model& m;
      std::string operator()(bool b) const { return b ? "true" : "false"; }
      std::string operator()(int64_t i) const { return std::to_string(i); }
      std::string operator()(double d) const { return numberText(d, 17); }
      std::string operator()(const std::string& s) const { return quote(s); }
      std::string operator()(const Ints& v) const {
        std::string s = "[";
        for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
        return s + "]";
      }
      std::string operator()(const Floats& v) const {
        std::string s = "f[";
        for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + numberText(v[i], 17);
        return s + "]";
      }
      std::string operator()(Dim d) const { return "dim<" + m.dims().str(d) + ">"; }
    };
    return std::visit(V{m}, a);
  }
  void attrs(const Op& op) {
    if (op.attrs.empty()) return;
    out += " {";
    for (size_t i = 0; i < op.attrs.size(); ++i)
      out += (i ? ", " : "") + op.attrs[i].name + " = " + attrText(op.attrs[i].value);
    out += "}";
  }
  void resultTypes(const Op& op) {
    for (size_t i = 0; i < op.results.size(); ++i) out += (i ? ", " : " : ") + typeText(op.results[i]);
  }
};

using Formatter = void (*)(Printer&, const Op&);

void fmtKernel(Printer& p, const Op& op) {
  p.out += "kernel " + quote(op.name) + "(";
  p.refs(op.operands);
  p.out += ")";
  if (!op.outs.empty()) {
    p.out += " outs(";
    p.refs(op.outs);
    p.out += ")";
  }
  p.attrs(op);
  p.resultTypes(op);
}
void fmtConstInline(Printer& p, const Op& op) {
  const DType dt = p.m.typeOf(op.results[0])->dtype;
  const size_t es = dtypeSize(dt);
  p.out += "const.inline dense<[";
  for (size_t at = 0; at < op.data.size(); at += es) p.out += (at ? ", " : "") + elementText(dt, &op.data[at]);
  p.out += "]>";
  p.attrs(op);
  p.resultTypes(op);
}
void fmtConstNamed(Printer& p, const Op& op) {
  p.out += std::string(opKindName(op.kind)) + " @" + quote(op.name);
  p.attrs(op);
  p.resultTypes(op);
}
void fmtView(Printer& p, const Op& op) {
  p.out += "view " + p.ref(op.operands[0]) + "[" + p.m.dims().str(op.dims[0]) + "]";
  p.attrs(op);
  p.resultTypes(op);
}
void fmtAlloc(Printer& p, const Op& op) {
  p.out += "buffer.alloc";
  p.attrs(op);
  p.resultTypes(op);
}
void fmtFree(Printer& p, const Op& op) {
  p.out += "buffer.free ";
  p.refs(op.operands);
}
void fmtMemPlan(Printer& p, const Op& op) {
  const DimPool& d = p.m.dims();
  p.out += "mem.plan sizes[";
  for (size_t i = 0; i < op.dims.size(); ++i) p.out += (i ? ", " : "") + d.str(op.dims[i]);
  p.out += "] live[";
  for (size_t i = 0; i + 1 < op.ints.size(); ++i) p.out += (i ? ", " : "") + std::to_string(op.ints[i]);
  p.out += "] align " + std::to_string(op.ints.back()) + " ->";
  for (size_t i = 0; i < op.symbols.size(); ++i) p.out += (i ? ", " : " ") + d.symbolName(op.symbols[i]);
  p.attrs(op);
  p.resultTypes(op);
}
void fmtDimRead(Printer& p, const Op& op) {
  p.out += "dim.read " + p.ref(op.operands[0]) + "[" + std::to_string(op.ints[0]) + "] -> " +
           p.m.dims().symbolName(op.symbols[0]);
}
void fmtSync(Printer& p, const Op& op) {
  p.out += op.ints[0] == kGpuToCpu ? "sync gpu_to_cpu" : "sync cpu_to_gpu";
  if (op.operands.empty()) return;
  p.out += " " + p.ref(op.operands[0]);
  p.resultTypes(op);
}
void fmtReturn(Printer& p, const Op& op) {
  p.out += "return";
  if (op.operands.empty()) return;
  p.out += " ";
  p.refs(op.operands);
}

// indexed by OpKind
const Formatter kFormatters[] = {fmtKernel, fmtConstInline, fmtConstNamed, fmtConstNamed, fmtView,  fmtAlloc,
                                 fmtFree,   fmtMemPlan,     fmtDimRead,    fmtSync,       fmtReturn};

void printOps(Printer& p, const Region& r) {
  for (const Op& op : r.ops) {
    p.out += "    ";
    if (!op.results.empty()) {
      p.refs(op.results);
      p.out += " = ";
    }
    kFormatters[static_cast<int>(op.kind)](p, op);
    p.out += "\n";
  }
}

}  // namespace

std::string printModel(const Model& m) {
  Printer p{m, {}, {}, {}, 0};
  p.out = "model {\n  init";
  p.header(m.init);
  p.out += " {\n";
  printOps(p, m.init);
  p.out += "  }\n  exec(";
  p.typed(m.exec.args, &m.exec);
  p.out += ")";
  if (!m.exec.state.empty()) {
    p.out += " state(";
    p.typed(m.exec.state, nullptr);
    p.out += ")";
  }
  p.header(m.exec);
  p.out += " {\n";
  printOps(p, m.exec);
  p.out += "  }\n}\n";
  return p.out;
}

// ---- lexer -------------------------------------------------------------------------------------------------------
namespace {

enum class Tok : uint8_t { Word, Value, Str, Num, Punct, Op, End };

struct Token {
  Tok kind;
  std::string_view text;  // the source span (for Str: without the quotes, escapes still in)
  int line;
  size_t pos;             // byte offset of the span's first character in the source
};

bool wordChar(char c) { return std::isalnum(static_cast<unsigned char>(c)) || c == '_' || c == '.'; }
bool nameChar(char c) { return std::isalnum(static_cast<unsigned char>(c)) || c == '_'; }
bool digit(char c) { return c >= '0' && c <= '9'; }

// Splits the text into tokens. "//" starts a comment outside square brackets and dim<...>, and is the floor
// division inside them; "%" followed by a name character starts a value, else it is the modulo operator.
bool lex(std::string_view s, std::vector<Token>& toks, std::string& err) {
  int line = 1, square = 0, dimAngle = 0;
  size_t i = 0;
  auto push = [&](Tok k, size_t b, size_t e) { toks.push_back({k, s.substr(b, e - b), line, b}); };
  while (i < s.size()) {
    const char c = s[i];
    if (c == '\n') {
      ++line;
      ++i;
      continue;
    }
    if (std::isspace(static_cast<unsigned char>(c))) {
      ++i;
      continue;
    }
    const bool inDim = square > 0 || dimAngle > 0;
    if (c == '/' && i + 1 < s.size() && s[i + 1] == '/') {
      if (inDim) {
        push(Tok::Op, i, i + 2);
        i += 2;
      } else {
        while (i < s.size() && s[i] != '\n') ++i;
      }
      continue;
    }
    if (c == '"') {
      size_t j = i + 1;
      while (j < s.size() && s[j] != '"') j += s[j] == '\\' ? 2 : 1;
      if (j >= s.size()) {
        err = "line " + std::to_string(line) + ": unterminated string";
        return false;
      }
      push(Tok::Str, i + 1, j);
      i = j + 1;
      continue;
    }
    if (c == '%' && i + 1 < s.size() && nameChar(s[i + 1])) {
      size_t j = i + 1;
      while (j < s.size() && nameChar(s[j])) ++j;
      push(Tok::Value, i + 1, j);
      i = j;
      continue;
    }
    if (c == '-' && i + 1 < s.size() && s[i + 1] == '>') {
      push(Tok::Punct, i, i + 2);
      i += 2;
      continue;
    }
    const bool sign = (c == '-' || c == '+') && i + 1 < s.size();
    if (digit(c) || (sign && (digit(s[i + 1]) || s.compare(i + 1, 3, "inf") == 0))) {
      size_t j = i + (sign ? 1 : 0);
      if (s.compare(j, 3, "inf") == 0) {
        j += 3;
      } else {
        while (j < s.size()) {
          const char d = s[j];
          if (digit(d) || d == '.') {
            ++j;
          } else if ((d == 'e' || d == 'E') && j + 1 < s.size() &&
                     (digit(s[j + 1]) || ((s[j + 1] == '-' || s[j + 1] == '+') && j + 2 < s.size() && digit(s[j + 2])))) {
            j += 2;
          } else {
            break;
          }
        }
      }
      push(Tok::Num, i, j);
      i = j;
      continue;
    }
    if (wordChar(c)) {
      size_t j = i;
      while (j < s.size() && wordChar(s[j])) ++j;
      push(Tok::Word, i, j);
      i = j;
      if (s.compare(toks.back().pos, 3, "dim") == 0 && toks.back().text.size() == 3 && i < s.size() && s[i] == '<') {
        push(Tok::Punct, i, i + 1);
        ++dimAngle;
        ++i;
      }
      continue;
    }
    if (std::strchr("{}()[]<>,:=@", c)) {
      if (c == '[') ++square;
      if (c == ']' && square > 0) --square;
      if (c == '>' && dimAngle > 0 && square == 0) --dimAngle;
      push(Tok::Punct, i, i + 1);
      ++i;
      continue;
    }
    if (std::strchr("*+-/%", c)) {
      push(Tok::Op, i, i + 1);
      ++i;
      continue;
    }
    err = "line " + std::to_string(line) + ": unexpected character '" + std::string(1, c) + "'";
    return false;
  }
  toks.push_back({Tok::End, s.substr(s.size()), line, s.size()});
  return true;
}

std::string unescape(std::string_view raw) {
  std::string s;
  for (size_t i = 0; i < raw.size(); ++i) s.push_back(raw[i] == '\\' && i + 1 < raw.size() ? raw[++i] : raw[i]);
  return s;
}

// ---- parser ------------------------------------------------------------------------------------------------------

struct Number {
  double d = 0;
  int64_t i = 0;
  bool integral = false;
};

class Reader {
 public:
  Reader(std::string_view src, std::vector<Token> toks) : src_(src), t_(std::move(toks)), m_(std::make_unique<Model>()) {}

  std::unique_ptr<Model> model(Status& st) {
    if (!parseModelText()) {
      st = Status::error(err_.empty() ? "parse error" : err_);
      return nullptr;
    }
    return std::move(m_);
  }

 private:
  using OpReader = bool (Reader::*)(Op&, const std::vector<std::string>&);
  struct OpEntry {
    OpKind kind;
    OpReader read;
  };

  // -- token cursor
  const Token& cur() const { return t_[at_]; }
  bool is(Tok k, std::string_view text) const { return cur().kind == k && cur().text == text; }
  bool isPunct(std::string_view p) const { return is(Tok::Punct, p); }
  bool isWord(std::string_view w) const { return is(Tok::Word, w); }
  bool take(Tok k, std::string_view text) {
    if (!is(k, text)) return false;
    ++at_;
    return true;
  }
  bool takePunct(std::string_view p) { return take(Tok::Punct, p); }
  bool takeWord(std::string_view w) { return take(Tok::Word, w); }
  bool needPunct(std::string_view p) { return takePunct(p) || error("expected '" + std::string(p) + "'"); }
  bool needWord(std::string_view w) { return takeWord(w) || error("expected '" + std::string(w) + "'"); }
  bool error(const std::string& what) {
    if (err_.empty()) {
      const size_t pos = std::min(cur().pos, src_.size());
      err_ = "line " + std::to_string(cur().line) + ": " + what + " near '" +
             std::string(src_.substr(pos, std::min<size_t>(30, src_.size() - pos))) + "'";
    }
    return false;
  }
  bool name(std::string& out) {
    if (cur().kind != Tok::Word) return error("expected a name");
    out = std::string(cur().text);
    ++at_;
    return true;
  }
  bool string(std::string& out) {
    if (cur().kind != Tok::Str) return error("expected a string");
    out = unescape(cur().text);
    ++at_;
    return true;
  }
  bool number(Number& n) {
    const Token& k = cur();
    std::string text(k.text);
    if (k.kind == Tok::Word && (text == "nan" || text == "inf")) {
      n = {text == "nan" ? NAN : INFINITY, 0, false};
    } else if (k.kind == Tok::Num) {
      n.integral = text.find_first_of(".eEn") == std::string::npos;
      n.d = text == "-inf" ? -INFINITY : text == "+inf" ? INFINITY : std::strtod(text.c_str(), nullptr);
      n.i = n.integral ? std::strtoll(text.c_str(), nullptr, 10) : 0;
    } else {
      return error("expected number");
    }
    ++at_;
    return true;
  }
  template <class F>
  bool commaList(std::string_view close, F item) {
    if (takePunct(close)) return true;
    do {
      if (!item()) return false;
    } while (takePunct(","));
    return needPunct(close);
  }

  // A dim: the tokens up to a ',' or `close` outside parentheses, handed to the dim parser as their source text.
  bool dim(std::string_view close, Dim& out) {
    const size_t first = at_;
    int depth = 0;
    for (; cur().kind != Tok::End; ++at_) {
      if (isPunct("(")) ++depth;
      if (isPunct(")")) --depth;
      if (depth < 0 || (depth == 0 && (isPunct(",") || isPunct(close)))) break;
    }
    const size_t b = t_[first].pos, e = at_ > first ? t_[at_ - 1].pos + t_[at_ - 1].text.size() : b;
    std::string why;
    out = m_->dims().parse(src_.substr(b, e - b), why);
    if (out) return true;
    at_ = first;
    return error(why);
  }

  // -- values and types
  bool define(const std::string& n, Type t, ValueId& id) {
    if (byName_.count(n)) return error("redefinition of %" + n);
    const bool numbered = n.find_first_not_of("0123456789") == std::string::npos;
    id = m_->newValue(t, numbered ? std::string() : n);
    byName_.emplace(n, id);
    return true;
  }
  bool use(ValueId& id) {
    if (cur().kind != Tok::Value) return error("expected a value");
    auto it = byName_.find(std::string(cur().text));
    if (it == byName_.end()) return error("use of undefined value %" + std::string(cur().text));
    id = it->second;
    ++at_;
    return true;
  }
  bool useList(std::vector<ValueId>& out, std::string_view close) {
    return commaList(close, [&] {
      ValueId v;
      return use(v) && (out.push_back(v), true);
    });
  }
  bool type(Type& t) {
    std::string w;
    if (!name(w)) return false;
    if (auto dt = dtypeFromName(w)) {
      t = m_->types().scalar(*dt);
      return true;
    }
    if (w != "tensor" && w != "buffer") return error("expected type");
    std::string dts;
    if (!needPunct("<") || !name(dts)) return false;
    auto dt = dtypeFromName(dts);
    if (!dt) return error("expected dtype");
    std::vector<Dim> shape;
    if (!needPunct("[") || !commaList("]", [&] {
          Dim d;
          return dim("]", d) && (shape.push_back(d), true);
        }) ||
        !needPunct(">"))
      return false;
    t = m_->types().get(w == "tensor" ? TypeKind::Tensor : TypeKind::Buffer, *dt, shape);
    return true;
  }
  // "-> T" or "-> (T, ...)", absent: no declaration
  bool declaredResults(std::optional<std::vector<Type>>& out) {
    if (!takePunct("->")) return true;
    auto& v = out.emplace();
    auto one = [&] {
      Type t;
      return type(t) && (v.push_back(t), true);
    };
    if (!takePunct("(")) return one();
    return commaList(")", one);
  }
  bool checkDeclared(const Region& r, const std::optional<std::vector<Type>>& decl, const char* region) {
    if (!decl) return true;
    const auto& ret = r.ops.back().operands;
    if (ret.size() != decl->size())
      return error(std::string(region) + " header declares " + std::to_string(decl->size()) +
                   " result types, return has " + std::to_string(ret.size()));
    for (size_t i = 0; i < ret.size(); ++i)
      if (m_->typeOf(ret[i]) != (*decl)[i])
        return error(std::string(region) + " result #" + std::to_string(i) + " is " +
                     m_->types().str(m_->typeOf(ret[i])) + ", header declares " + m_->types().str((*decl)[i]));
    return true;
  }
  bool argList(std::vector<ValueId>& out, std::vector<uint8_t>* mutableFlags) {
    std::vector<uint8_t> flags;
    bool any = false;
    const bool ok = commaList(")", [&] {
      if (cur().kind != Tok::Value) return error("expected a value");
      const std::string n(cur().text);
      ++at_;
      Type t;
      ValueId id;
      if (!needPunct(":") || !type(t) || !define(n, t, id)) return false;
      out.push_back(id);
      const bool mut = mutableFlags && takeWord("mutable");
      flags.push_back(mut ? 1 : 0);
      any = any || mut;
      return true;
    });
    if (ok && any) *mutableFlags = flags;
    return ok;
  }

  // -- attributes
  bool attrValue(AttrValue& a) {
    if (cur().kind == Tok::Str) {
      std::string s;
      string(s);
      a = std::move(s);
      return true;
    }
    if (isWord("true") || isWord("false")) {
      a = cur().text == "true";
      ++at_;
      return true;
    }
    if (isWord("dim")) {
      ++at_;
      Dim d;
      if (!needPunct("<") || !dim(">", d) || !needPunct(">")) return false;
      a = d;
      return true;
    }
    bool floats = false;
    if (isWord("f") && t_[at_ + 1].kind == Tok::Punct && t_[at_ + 1].text == "[") {
      ++at_;
      floats = true;
    }
    if (takePunct("[")) {
      Ints iv;
      Floats fv;
      if (!commaList("]", [&] {
            Number n;
            if (!number(n)) return false;
            iv.push_back(n.i);
            fv.push_back(n.d);
            floats = floats || !n.integral;
            return true;
          }))
        return false;
      if (floats) a = std::move(fv);
      else a = std::move(iv);
      return true;
    }
    Number n;
    if (!number(n)) return false;
    if (n.integral) a = n.i;
    else a = n.d;
    return true;
  }
  bool attrDict(Op& op) {
    if (!takePunct("{")) return true;
    return commaList("}", [&] {
      std::string key;
      AttrValue v;
      if (cur().kind != Tok::Word) return error("expected attribute name");
      if (!name(key) || !needPunct("=") || !attrValue(v)) return false;
      op.setAttr(std::move(key), std::move(v));
      return true;
    });
  }
  // ": T, U" for the names on the left of '='
  bool resultTypes(Op& op, const std::vector<std::string>& names) {
    if (names.empty()) return true;
    if (!needPunct(":")) return false;
    for (size_t i = 0; i < names.size(); ++i) {
      Type t;
      ValueId id;
      if ((i && !needPunct(",")) || !type(t) || !define(names[i], t, id)) return false;
      op.results.push_back(id);
    }
    return true;
  }
  bool tail(Op& op, const std::vector<std::string>& names) { return attrDict(op) && resultTypes(op, names); }
  bool symbolName(Op& op) {
    std::string s;
    if (!name(s)) return false;
    op.symbols.push_back(m_->dims().sym(s)->value);
    return true;
  }

  // -- ops (dispatched by keyword)
  bool readKernel(Op& op, const std::vector<std::string>& names) {
    if (!string(op.name) || !needPunct("(") || !useList(op.operands, ")")) return false;
    if (takeWord("outs") && (!needPunct("(") || !useList(op.outs, ")"))) return false;
    return tail(op, names);
  }
  bool readConstInline(Op& op, const std::vector<std::string>& names) {
    std::vector<Number> nums;
    if (!needWord("dense") || !needPunct("<") || !needPunct("[") || !commaList("]", [&] {
          Number n;
          return number(n) && (nums.push_back(n), true);
        }) ||
        !needPunct(">") || !tail(op, names))
      return false;
    if (op.results.size() != 1) return error("const.inline must have one result");
    const DType dt = m_->typeOf(op.results[0])->dtype;
    const size_t es = dtypeSize(dt);
    op.data.assign(nums.size() * es, 0);
    for (size_t k = 0; k < nums.size(); ++k) {
      uint8_t* p = op.data.data() + k * es;
      const Number& n = nums[k];
      if (dt == DType::F32) {
        const float f = static_cast<float>(n.d);
        std::memcpy(p, &f, 4);
      } else if (dt == DType::F16 || dt == DType::BF16) {
        const uint16_t h = dt == DType::F16 ? floatToHalf(static_cast<float>(n.d)) : floatToBf16(static_cast<float>(n.d));
        std::memcpy(p, &h, 2);
      } else {
        if (!n.integral) return error("expected integer constant");
        const int64_t v = n.i;
        std::memcpy(p, &v, es);  // little-endian: the low bytes
      }
    }
    return true;
  }
  bool readConstNamed(Op& op, const std::vector<std::string>& names) {
    if (!needPunct("@") || !string(op.name) || !tail(op, names)) return false;
    if (op.kind == OpKind::ConstInternal && !m_->findConstant(op.name))
      m_->addConstant(Constant{op.name, m_->typeOf(op.results[0]), nullptr, nullptr, 0});
    return true;
  }
  bool readView(Op& op, const std::vector<std::string>& names) {
    ValueId src;
    Dim off;
    if (!use(src) || !needPunct("[") || !dim("]", off) || !needPunct("]")) return false;
    op.operands.push_back(src);
    op.dims.push_back(off);
    return tail(op, names);
  }
  bool readAlloc(Op& op, const std::vector<std::string>& names) { return tail(op, names); }
  bool readFree(Op& op, const std::vector<std::string>&) {
    ValueId v;
    return use(v) && (op.operands.push_back(v), true);
  }
  bool readMemPlan(Op& op, const std::vector<std::string>& names) {
    if (!needWord("sizes") || !needPunct("[") || !commaList("]", [&] {
          Dim d;
          return dim("]", d) && (op.dims.push_back(d), true);
        }))
      return false;
    if (!needWord("live") || !needPunct("[") || !commaList("]", [&] {
          Number n;
          if (!number(n)) return false;
          if (!n.integral) return error("expected integer");
          op.ints.push_back(n.i);
          return true;
        }))
      return false;
    Number align;
    if (!needWord("align") || !number(align) || !needPunct("->")) return false;
    op.ints.push_back(align.i);
    do {
      if (!symbolName(op)) return false;
    } while (takePunct(","));
    return tail(op, names);
  }
  bool readDimRead(Op& op, const std::vector<std::string>&) {
    ValueId src;
    Number idx;
    if (!use(src) || !needPunct("[") || !number(idx) || !needPunct("]") || !needPunct("->")) return false;
    op.operands.push_back(src);
    op.ints.push_back(idx.i);
    return symbolName(op);
  }
  bool readSync(Op& op, const std::vector<std::string>& names) {
    if (takeWord("gpu_to_cpu")) op.ints.push_back(kGpuToCpu);
    else if (takeWord("cpu_to_gpu")) op.ints.push_back(kCpuToGpu);
    else return error("expected gpu_to_cpu or cpu_to_gpu");
    if (names.empty()) return true;
    ValueId v;
    if (!use(v)) return false;
    op.operands.push_back(v);
    return resultTypes(op, names);
  }
  bool readReturn(Op& op, const std::vector<std::string>&) {
    if (cur().kind != Tok::Value) return true;
    do {
      ValueId v;
      if (!use(v)) return false;
      op.operands.push_back(v);
    } while (takePunct(","));
    return true;
  }

  static const std::unordered_map<std::string_view, OpEntry>& opTable() {
    static const std::unordered_map<std::string_view, OpEntry> t = {
        {"kernel", {OpKind::Kernel, &Reader::readKernel}},
        {"const.inline", {OpKind::ConstInline, &Reader::readConstInline}},
        {"const.internal", {OpKind::ConstInternal, &Reader::readConstNamed}},
        {"const.external", {OpKind::ConstExternal, &Reader::readConstNamed}},
        {"view", {OpKind::View, &Reader::readView}},
        {"buffer.alloc", {OpKind::BufferAlloc, &Reader::readAlloc}},
        {"buffer.free", {OpKind::BufferFree, &Reader::readFree}},
        {"mem.plan", {OpKind::MemPlan, &Reader::readMemPlan}},
        {"dim.read", {OpKind::DimRead, &Reader::readDimRead}},
        {"sync", {OpKind::Sync, &Reader::readSync}},
        {"return", {OpKind::Return, &Reader::readReturn}},
    };
    return t;
  }

  // one line: [%a, %b =] keyword ...
  bool opLine(Region& r) {
    std::vector<std::string> names;
    if (cur().kind == Tok::Value) {
      do {
        if (cur().kind != Tok::Value) return error("expected value name");
        names.emplace_back(cur().text);
        ++at_;
      } while (takePunct(","));
      if (!needPunct("=")) return false;
    }
    const std::string_view kw = cur().kind == Tok::Word ? cur().text : std::string_view();
    auto it = opTable().find(kw);
    if (it == opTable().end()) return error("unknown op '" + std::string(kw) + "'");
    ++at_;
    Op op;
    op.kind = it->second.kind;
    if (!(this->*(it->second.read))(op, names)) return false;
    r.ops.push_back(std::move(op));
    return true;
  }
  bool region(Region& r) {
    while (!takePunct("}")) {
      if (cur().kind == Tok::End) return error("expected '}'");
      if (!opLine(r)) return false;
    }
    if (r.ops.empty() || r.ops.back().kind != OpKind::Return) return error("region must end with return");
    return true;
  }

  bool parseModelText() {
    std::optional<std::vector<Type>> initDecl, execDecl;
    if (!needWord("model") || !needPunct("{") || !needWord("init") || !declaredResults(initDecl) ||
        !needPunct("{") || !region(m_->init) || !checkDeclared(m_->init, initDecl, "init"))
      return false;
    if (!needWord("exec") || !needPunct("(") || !argList(m_->exec.args, &m_->exec.mutableArgs)) return false;
    if (takeWord("state") && (!needPunct("(") || !argList(m_->exec.state, nullptr))) return false;
    if (!declaredResults(execDecl) || !needPunct("{") || !region(m_->exec) ||
        !checkDeclared(m_->exec, execDecl, "exec") || !needPunct("}"))
      return false;
    if (cur().kind != Tok::End) return error("trailing text after model");
    return true;
  }

  std::string_view src_;
  std::vector<Token> t_;
  size_t at_ = 0;
  std::string err_;
  std::unique_ptr<Model> m_;
  std::unordered_map<std::string, ValueId> byName_;
};

}  // namespace

std::unique_ptr<Model> parseModel(std::string_view text, Status& st) {
  std::vector<Token> toks;
  std::string err;
  if (!lex(text, toks, err)) {
    st = Status::error(err);
    return nullptr;
  }
  return Reader(text, std::move(toks)).model(st);
}

}  // namespace lkrt
