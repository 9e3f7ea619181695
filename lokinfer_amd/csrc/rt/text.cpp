// Textual IR: printer and parser for the reference's line-oriented, MLIR-like model text (format:
// lariaus/lokinfer docs/impl-notes/design-ir.md §5, §7). print(parse(print(m))) == print(m).
//
//   model {
//     init -> buffer<f32[4]> { ... return %w }
//     exec(%x: buffer<f32[N]>, %kv: buffer<f32[8]> mutable) state(%w2: buffer<f32[4]>) -> buffer<f32[N]> {
//       %o = buffer.alloc {output = true} : buffer<f32[N]>
//       kernel "add_f32_gpu"(%x, %x) outs(%o) {alpha = 1.0}
//       ...
//       return %o
//     }
//   }
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unordered_set>

#include "ir.h"

namespace lkrt {

// ---- scalars ---------------------------------------------------------------------------------------------------
namespace {

float halfBitsToFloat(uint16_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  int32_t e = (h >> 10) & 0x1f;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {  // subnormal: normalize
      e = 1;
      while (!(m & 0x400u)) {
        m <<= 1;
        --e;
      }
      m &= 0x3ffu;
      bits = sign | static_cast<uint32_t>(e + 112) << 23 | (m << 13);
    }
  } else {
    bits = sign | static_cast<uint32_t>(e + 112) << 23 | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// round to nearest even
uint16_t floatToHalfBits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0);
  if (ax >= 0x477ff000u) return sign | 0x7c00u;  // rounds to >= 65520: infinity
  if (ax < 0x38800000u) {                         // below the smallest normal half: subnormal or zero
    float af;
    std::memcpy(&af, &ax, 4);
    const float scaled = af * 16777216.0f;  // units of 2^-24
    return sign | static_cast<uint16_t>(std::nearbyint(scaled));
  }
  const uint32_t e = (ax >> 23) - 112;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return sign | static_cast<uint16_t>(h);
}

float bf16BitsToFloat(uint16_t h) {
  const uint32_t bits = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t floatToBf16Bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return static_cast<uint16_t>(x >> 16);
}

std::string formatDouble(double v, int precision) {
  if (std::isnan(v)) return "nan";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.*g", precision, v);
  std::string s = buf;
  if (s.find_first_of(".e") == std::string::npos) s += ".0";
  return s;
}

std::string quoted(std::string_view s) {
  std::string out = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') out += '\\';
    out += c;
  }
  return out + "\"";
}

std::string formatScalar(DType t, const uint8_t* p) {
  switch (t) {
    case DType::F32: {
      float f;
      std::memcpy(&f, p, 4);
      return formatDouble(f, 9);
    }
    case DType::F16:
    case DType::BF16: {
      uint16_t h;
      std::memcpy(&h, p, 2);
      return formatDouble(t == DType::F16 ? halfBitsToFloat(h) : bf16BitsToFloat(h), 9);
    }
    case DType::I8: return std::to_string(static_cast<int8_t>(*p));
    case DType::U8: return std::to_string(*p);
    case DType::Bool: return *p ? "1" : "0";
    case DType::I16: {
      int16_t v;
      std::memcpy(&v, p, 2);
      return std::to_string(v);
    }
    case DType::I32: {
      int32_t v;
      std::memcpy(&v, p, 4);
      return std::to_string(v);
    }
    case DType::I64: {
      int64_t v;
      std::memcpy(&v, p, 8);
      return std::to_string(v);
    }
  }
  return "?";
}

}  // namespace

// ---- printer ---------------------------------------------------------------------------------------------------
namespace {

class TextWriter {
 public:
  explicit TextWriter(const Model& m) : m_(m) {}

  std::string run() {
    s_ = "model {\n  init" + regionResults(m_.init) + " {\n";
    ops(m_.init);
    s_ += "  }\n  exec(" + args(m_.exec.args, &m_.exec) + ")";
    if (!m_.exec.state.empty()) s_ += " state(" + args(m_.exec.state, nullptr) + ")";
    s_ += regionResults(m_.exec) + " {\n";
    ops(m_.exec);
    s_ += "  }\n}\n";
    return s_;
  }

 private:
  // Values print under their name hint, made unique with a _1, _2, ... suffix; unnamed values get the next free
  // number.
  const std::string& name(ValueId v) {
    auto it = names_.find(v);
    if (it != names_.end()) return it->second;
    const std::string& hint = m_.nameOf(v);
    std::string n;
    if (hint.empty()) {
      do n = std::to_string(counter_++);
      while (taken_.count(n));
    } else {
      n = hint;
      for (int k = 1; taken_.count(n); ++k) n = hint + "_" + std::to_string(k);
    }
    taken_.insert(n);
    return names_.emplace(v, "%" + n).first->second;
  }
  std::string type(ValueId v) { return m_.types().str(m_.typeOf(v)); }
  std::string list(const std::vector<ValueId>& vs) {
    std::string s;
    for (size_t i = 0; i < vs.size(); ++i) s += (i ? ", " : "") + name(vs[i]);
    return s;
  }
  std::string args(const std::vector<ValueId>& vs, const Region* r) {
    std::string s;
    for (size_t i = 0; i < vs.size(); ++i) {
      s += (i ? ", " : "") + name(vs[i]) + ": " + type(vs[i]);
      if (r && r->isMutable(i)) s += " mutable";
    }
    return s;
  }
  std::string regionResults(const Region& r) {
    if (r.ops.empty() || r.ops.back().kind != OpKind::Return || r.ops.back().operands.empty()) return "";
    const auto& vs = r.ops.back().operands;
    std::string s;
    for (size_t i = 0; i < vs.size(); ++i) s += (i ? ", " : "") + type(vs[i]);
    return vs.size() == 1 ? " -> " + s : " -> (" + s + ")";
  }
  std::string attrText(const AttrValue& a) {
    switch (a.index()) {
      case 0: return std::get<bool>(a) ? "true" : "false";
      case 1: return std::to_string(std::get<int64_t>(a));
      case 2: return formatDouble(std::get<double>(a), 17);
      case 3: return quoted(std::get<std::string>(a));
      case 4: {
        std::string s = "[";
        const Ints& v = std::get<Ints>(a);
        for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
        return s + "]";
      }
      case 5: {
        std::string s = "f[";
        const Floats& v = std::get<Floats>(a);
        for (size_t i = 0; i < v.size(); ++i) s += (i ? ", " : "") + formatDouble(v[i], 17);
        return s + "]";
      }
      default: return "dim<" + m_.dims().str(std::get<Dim>(a)) + ">";
    }
  }
  std::string attrs(const Op& op) {
    if (op.attrs.empty()) return "";
    std::string s = " {";
    for (size_t i = 0; i < op.attrs.size(); ++i)
      s += (i ? ", " : "") + op.attrs[i].name + " = " + attrText(op.attrs[i].value);
    return s + "}";
  }
  std::string resultTypes(const Op& op) {
    if (op.results.empty()) return "";
    std::string s = " : ";
    for (size_t i = 0; i < op.results.size(); ++i) s += (i ? ", " : "") + type(op.results[i]);
    return s;
  }
  void ops(const Region& r) {
    for (const Op& op : r.ops) {
      s_ += "    ";
      if (!op.results.empty()) s_ += list(op.results) + " = ";
      one(op);
      s_ += "\n";
    }
  }
  void one(const Op& op) {
    const DimPool& d = m_.dims();
    switch (op.kind) {
      case OpKind::Kernel:
        s_ += "kernel " + quoted(op.name) + "(" + list(op.operands) + ")";
        if (!op.outs.empty()) s_ += " outs(" + list(op.outs) + ")";
        s_ += attrs(op) + resultTypes(op);
        return;
      case OpKind::ConstInline: {
        const DType dt = m_.typeOf(op.results[0])->dtype;
        const size_t es = dtypeSize(dt);
        s_ += "const.inline dense<[";
        for (size_t i = 0; i * es < op.data.size(); ++i) s_ += (i ? ", " : "") + formatScalar(dt, &op.data[i * es]);
        s_ += "]>" + attrs(op) + resultTypes(op);
        return;
      }
      case OpKind::ConstInternal:
      case OpKind::ConstExternal:
        s_ += std::string(opKindName(op.kind)) + " @" + quoted(op.name) + attrs(op) + resultTypes(op);
        return;
      case OpKind::View:
        s_ += "view " + name(op.operands[0]) + "[" + d.str(op.dims[0]) + "]" + attrs(op) + resultTypes(op);
        return;
      case OpKind::BufferAlloc:
        s_ += "buffer.alloc" + attrs(op) + resultTypes(op);
        return;
      case OpKind::BufferFree:
        s_ += "buffer.free " + list(op.operands);
        return;
      case OpKind::MemPlan: {
        s_ += "mem.plan sizes[";
        for (size_t i = 0; i < op.dims.size(); ++i) s_ += (i ? ", " : "") + d.str(op.dims[i]);
        s_ += "] live[";
        for (size_t i = 0; i + 1 < op.ints.size(); ++i) s_ += (i ? ", " : "") + std::to_string(op.ints[i]);
        s_ += "] align " + std::to_string(op.ints.back()) + " ->";
        for (size_t i = 0; i < op.symbols.size(); ++i) s_ += (i ? ", " : " ") + d.symbolName(op.symbols[i]);
        s_ += attrs(op) + resultTypes(op);
        return;
      }
      case OpKind::DimRead:
        s_ += "dim.read " + name(op.operands[0]) + "[" + std::to_string(op.ints[0]) + "] -> " +
              d.symbolName(op.symbols[0]);
        return;
      case OpKind::Sync:
        s_ += op.ints[0] == kGpuToCpu ? "sync gpu_to_cpu" : "sync cpu_to_gpu";
        if (!op.operands.empty()) s_ += " " + name(op.operands[0]) + resultTypes(op);
        return;
      case OpKind::Return:
        s_ += "return";
        if (!op.operands.empty()) s_ += " " + list(op.operands);
        return;
    }
  }

  const Model& m_;
  std::string s_;
  std::unordered_map<ValueId, std::string> names_;
  std::unordered_set<std::string> taken_;
  int counter_ = 0;
};

}  // namespace

std::string printModel(const Model& m) { return TextWriter(m).run(); }

// ---- parser ----------------------------------------------------------------------------------------------------
namespace {

class TextReader {
 public:
  explicit TextReader(std::string_view s) : s_(s), m_(std::make_unique<Model>()) {}

  std::unique_ptr<Model> run(Status& st) {
    if (!model()) {
      st = Status::error(err_.empty() ? "parse error" : err_);
      return nullptr;
    }
    return std::move(m_);
  }

 private:
  bool model() {
    std::optional<std::vector<Type>> initTypes, execTypes;
    if (!keyword("model") || !tok("{") || !keyword("init") || !headerTypes(initTypes) || !tok("{")) return false;
    if (!opsUntilClose(m_->init) || !matchHeader(m_->init, initTypes, "init")) return false;
    if (!keyword("exec") || !tok("(") || !argList(m_->exec.args, &m_->exec.mutableArgs)) return false;
    if (peekKeyword("state")) {
      keyword("state");
      if (!tok("(") || !argList(m_->exec.state, nullptr)) return false;
    }
    if (!headerTypes(execTypes) || !tok("{") || !opsUntilClose(m_->exec) ||
        !matchHeader(m_->exec, execTypes, "exec") || !tok("}"))
      return false;
    ws();
    if (i_ != s_.size()) return fail("trailing text after model");
    return true;
  }

  // -- lexing
  void ws() {
    while (i_ < s_.size()) {
      const char c = s_[i_];
      if (c == '\n') {
        ++line_;
        ++i_;
      } else if (std::isspace(static_cast<unsigned char>(c))) {
        ++i_;
      } else if (c == '/' && i_ + 1 < s_.size() && s_[i_ + 1] == '/') {
        while (i_ < s_.size() && s_[i_] != '\n') ++i_;
      } else {
        break;
      }
    }
  }
  bool peekTok(std::string_view t) {
    ws();
    return s_.compare(i_, t.size(), t) == 0;
  }
  bool acceptTok(std::string_view t) {
    if (!peekTok(t)) return false;
    i_ += t.size();
    return true;
  }
  bool tok(std::string_view t) { return acceptTok(t) || fail("expected '" + std::string(t) + "'"); }
  static bool identChar(char c) { return std::isalnum(static_cast<unsigned char>(c)) || c == '_' || c == '.'; }
  std::string_view word() {
    ws();
    const size_t b = i_;
    while (i_ < s_.size() && identChar(s_[i_])) ++i_;
    return s_.substr(b, i_ - b);
  }
  bool peekKeyword(std::string_view w) {
    const size_t save = i_;
    const bool ok = word() == w;
    i_ = save;
    return ok;
  }
  bool keyword(std::string_view w) {
    const size_t save = i_;
    if (word() == w) return true;
    i_ = save;
    return fail("expected '" + std::string(w) + "'");
  }
  bool fail(const std::string& msg) {
    if (err_.empty()) {
      const size_t n = std::min<size_t>(30, s_.size() - std::min(i_, s_.size()));
      err_ = "line " + std::to_string(line_) + ": " + msg + " near '" + std::string(s_.substr(i_, n)) + "'";
    }
    return false;
  }
  bool string(std::string& out) {
    if (!tok("\"")) return false;
    out.clear();
    while (i_ < s_.size() && s_[i_] != '"') {
      if (s_[i_] == '\\' && i_ + 1 < s_.size()) ++i_;
      out += s_[i_++];
    }
    if (i_ >= s_.size()) return fail("unterminated string");
    ++i_;
    return true;
  }
  // a dim up to `close` or a top-level ','
  bool dimUntil(char close, Dim& out) {
    ws();
    const size_t b = i_;
    int depth = 0;
    for (; i_ < s_.size(); ++i_) {
      const char c = s_[i_];
      if (c == '(') ++depth;
      else if (c == ')') --depth;
      if (depth < 0 || (depth == 0 && (c == close || c == ','))) break;
    }
    std::string e;
    out = m_->dims().parse(s_.substr(b, i_ - b), e);
    return out ? true : fail(e);
  }
  bool number(double& d, bool& isInt, int64_t& i) {
    ws();
    for (const char* special : {"nan", "inf", "-inf"}) {
      if (s_.compare(i_, std::strlen(special), special) == 0) {
        i_ += std::strlen(special);
        d = special[0] == 'n' ? NAN : special[0] == '-' ? -INFINITY : INFINITY;
        isInt = false;
        return true;
      }
    }
    size_t p = i_;
    if (p < s_.size() && (s_[p] == '-' || s_[p] == '+')) ++p;
    bool digit = false, flt = false;
    for (; p < s_.size(); ++p) {
      const char c = s_[p];
      if (std::isdigit(static_cast<unsigned char>(c))) digit = true;
      else if (c == '.' || c == 'e' || c == 'E') flt = true;
      else if ((c == '-' || c == '+') && (s_[p - 1] == 'e' || s_[p - 1] == 'E')) continue;
      else break;
    }
    if (!digit) return fail("expected number");
    const std::string t(s_.substr(i_, p - i_));
    i_ = p;
    isInt = !flt;
    if (isInt) i = std::strtoll(t.c_str(), nullptr, 10);
    d = std::strtod(t.c_str(), nullptr);
    return true;
  }

  // -- values
  bool valueName(std::string& n) {
    if (!tok("%")) return false;
    const size_t b = i_;
    while (i_ < s_.size() && (std::isalnum(static_cast<unsigned char>(s_[i_])) || s_[i_] == '_')) ++i_;
    if (i_ == b) return fail("expected value name");
    n = std::string(s_.substr(b, i_ - b));
    return true;
  }
  bool define(const std::string& n, Type t, ValueId& id) {
    if (values_.count(n)) return fail("redefinition of %" + n);
    const bool numeric = n.find_first_not_of("0123456789") == std::string::npos;
    id = m_->newValue(t, numeric ? "" : n);
    values_[n] = id;
    return true;
  }
  bool use(ValueId& id) {
    std::string n;
    if (!valueName(n)) return false;
    auto it = values_.find(n);
    if (it == values_.end()) return fail("use of undefined value %" + n);
    id = it->second;
    return true;
  }
  bool uses(std::vector<ValueId>& out, std::string_view close) {
    if (acceptTok(close)) return true;
    do {
      ValueId v;
      if (!use(v)) return false;
      out.push_back(v);
    } while (acceptTok(","));
    return tok(close);
  }
  bool type(Type& t) {
    const std::string_view w = word();
    if (auto dt = dtypeFromName(w)) {
      t = m_->types().scalar(*dt);
      return true;
    }
    TypeKind kind;
    if (w == "tensor") kind = TypeKind::Tensor;
    else if (w == "buffer") kind = TypeKind::Buffer;
    else return fail("expected type");
    if (!tok("<")) return false;
    auto dt = dtypeFromName(word());
    if (!dt) return fail("expected dtype");
    if (!tok("[")) return false;
    std::vector<Dim> shape;
    if (!acceptTok("]")) {
      do {
        Dim d;
        if (!dimUntil(']', d)) return false;
        shape.push_back(d);
      } while (acceptTok(","));
      if (!tok("]")) return false;
    }
    if (!tok(">")) return false;
    t = m_->types().get(kind, *dt, shape);
    return true;
  }
  bool headerTypes(std::optional<std::vector<Type>>& out) {
    if (!acceptTok("->")) return true;
    std::vector<Type>& v = out.emplace();
    Type t;
    if (!acceptTok("(")) {
      if (!type(t)) return false;
      v.push_back(t);
      return true;
    }
    if (acceptTok(")")) return true;
    do {
      if (!type(t)) return false;
      v.push_back(t);
    } while (acceptTok(","));
    return tok(")");
  }
  bool matchHeader(const Region& r, const std::optional<std::vector<Type>>& declared, const char* what) {
    if (!declared) return true;
    const auto& ret = r.ops.back().operands;
    if (ret.size() != declared->size())
      return fail(std::string(what) + " header declares " + std::to_string(declared->size()) +
                  " result types, return has " + std::to_string(ret.size()));
    for (size_t i = 0; i < ret.size(); ++i)
      if (m_->typeOf(ret[i]) != (*declared)[i])
        return fail(std::string(what) + " result #" + std::to_string(i) + " is " +
                    m_->types().str(m_->typeOf(ret[i])) + ", header declares " + m_->types().str((*declared)[i]));
    return true;
  }
  bool argList(std::vector<ValueId>& out, std::vector<uint8_t>* flagsOut) {
    if (acceptTok(")")) return true;
    std::vector<uint8_t> flags;
    do {
      std::string n;
      Type t;
      ValueId id;
      if (!valueName(n) || !tok(":") || !type(t) || !define(n, t, id)) return false;
      out.push_back(id);
      bool mut = false;
      if (flagsOut && peekKeyword("mutable")) {
        keyword("mutable");
        mut = true;
      }
      flags.push_back(mut);
    } while (acceptTok(","));
    if (flagsOut && std::find(flags.begin(), flags.end(), 1) != flags.end()) *flagsOut = flags;
    return tok(")");
  }
  bool attrValue(AttrValue& a) {
    ws();
    if (peekTok("\"")) {
      std::string s;
      if (!string(s)) return false;
      a = std::move(s);
      return true;
    }
    if (peekKeyword("true") || peekKeyword("false")) {
      a = word() == "true";
      return true;
    }
    if (acceptTok("dim<")) {
      Dim d;
      if (!dimUntil('>', d) || !tok(">")) return false;
      a = d;
      return true;
    }
    bool floats = acceptTok("f[");
    if (floats || acceptTok("[")) {
      Ints iv;
      Floats fv;
      if (!acceptTok("]")) {
        do {
          double d;
          bool isInt;
          int64_t i = 0;
          if (!number(d, isInt, i)) return false;
          iv.push_back(i);
          fv.push_back(d);
          floats = floats || !isInt;
        } while (acceptTok(","));
        if (!tok("]")) return false;
      }
      if (floats) a = std::move(fv);
      else a = std::move(iv);
      return true;
    }
    double d;
    bool isInt;
    int64_t i = 0;
    if (!number(d, isInt, i)) return false;
    if (isInt) a = i;
    else a = d;
    return true;
  }
  bool attrDict(Op& op) {
    if (!acceptTok("{") || acceptTok("}")) return true;
    do {
      std::string n(word());
      if (n.empty()) return fail("expected attribute name");
      AttrValue a;
      if (!tok("=") || !attrValue(a)) return false;
      op.setAttr(std::move(n), std::move(a));
    } while (acceptTok(","));
    return tok("}");
  }
  bool results(Op& op, const std::vector<std::string>& names) {
    if (names.empty()) return true;
    if (!tok(":")) return false;
    for (size_t i = 0; i < names.size(); ++i) {
      Type t;
      ValueId id;
      if ((i && !tok(",")) || !type(t) || !define(names[i], t, id)) return false;
      op.results.push_back(id);
    }
    return true;
  }
  bool encode(DType t, double d, int64_t i, bool isInt, std::vector<uint8_t>& out) {
    const size_t at = out.size();
    out.resize(at + dtypeSize(t));
    uint8_t* p = out.data() + at;
    switch (t) {
      case DType::F32: {
        const float f = static_cast<float>(d);
        std::memcpy(p, &f, 4);
        return true;
      }
      case DType::F16:
      case DType::BF16: {
        const uint16_t h = t == DType::F16 ? floatToHalfBits(static_cast<float>(d)) : floatToBf16Bits(static_cast<float>(d));
        std::memcpy(p, &h, 2);
        return true;
      }
      default:
        if (!isInt) return fail("expected integer constant");
        if (t == DType::I8 || t == DType::U8 || t == DType::Bool) {
          *p = static_cast<uint8_t>(i);
        } else if (t == DType::I16) {
          const int16_t v = static_cast<int16_t>(i);
          std::memcpy(p, &v, 2);
        } else if (t == DType::I32) {
          const int32_t v = static_cast<int32_t>(i);
          std::memcpy(p, &v, 4);
        } else {
          std::memcpy(p, &i, 8);
        }
        return true;
    }
  }
  bool opsUntilClose(Region& r) {
    while (true) {
      if (acceptTok("}")) {
        if (r.ops.empty() || r.ops.back().kind != OpKind::Return) return fail("region must end with return");
        return true;
      }
      std::vector<std::string> names;
      if (peekTok("%")) {
        do {
          std::string n;
          if (!valueName(n)) return false;
          names.push_back(n);
        } while (acceptTok(","));
        if (!tok("=")) return false;
      }
      Op op;
      if (!oneOp(op, names)) return false;
      r.ops.push_back(std::move(op));
    }
  }
  bool oneOp(Op& op, const std::vector<std::string>& names) {
    const std::string kw(word());
    if (kw == "kernel") {
      op.kind = OpKind::Kernel;
      if (!string(op.name) || !tok("(") || !uses(op.operands, ")")) return false;
      if (peekKeyword("outs")) {
        word();
        if (!tok("(") || !uses(op.outs, ")")) return false;
      }
      return attrDict(op) && results(op, names);
    }
    if (kw == "const.inline") {
      op.kind = OpKind::ConstInline;
      if (!keyword("dense") || !tok("<") || !tok("[")) return false;
      struct Num {
        double d;
        int64_t i;
        bool isInt;
      };
      std::vector<Num> nums;
      if (!acceptTok("]")) {
        do {
          Num n{};
          if (!number(n.d, n.isInt, n.i)) return false;
          nums.push_back(n);
        } while (acceptTok(","));
        if (!tok("]")) return false;
      }
      if (!tok(">") || !attrDict(op) || !results(op, names)) return false;
      if (op.results.size() != 1) return fail("const.inline must have one result");
      const DType dt = m_->typeOf(op.results[0])->dtype;
      for (const Num& n : nums)
        if (!encode(dt, n.d, n.i, n.isInt, op.data)) return false;
      return true;
    }
    if (kw == "const.internal" || kw == "const.external") {
      op.kind = kw == "const.internal" ? OpKind::ConstInternal : OpKind::ConstExternal;
      if (!tok("@") || !string(op.name) || !attrDict(op) || !results(op, names)) return false;
      if (op.kind == OpKind::ConstInternal && !m_->findConstant(op.name))
        m_->addConstant(Constant{op.name, m_->typeOf(op.results[0]), nullptr, nullptr, 0});
      return true;
    }
    if (kw == "view") {
      op.kind = OpKind::View;
      ValueId src;
      Dim off;
      if (!use(src) || !tok("[") || !dimUntil(']', off) || !tok("]")) return false;
      op.operands.push_back(src);
      op.dims.push_back(off);
      return attrDict(op) && results(op, names);
    }
    if (kw == "buffer.alloc") {
      op.kind = OpKind::BufferAlloc;
      return attrDict(op) && results(op, names);
    }
    if (kw == "buffer.free") {
      op.kind = OpKind::BufferFree;
      ValueId v;
      if (!use(v)) return false;
      op.operands.push_back(v);
      return true;
    }
    if (kw == "mem.plan") {
      op.kind = OpKind::MemPlan;
      if (!keyword("sizes") || !tok("[")) return false;
      if (!acceptTok("]")) {
        do {
          Dim d;
          if (!dimUntil(']', d)) return false;
          op.dims.push_back(d);
        } while (acceptTok(","));
        if (!tok("]")) return false;
      }
      if (!keyword("live") || !tok("[")) return false;
      if (!acceptTok("]")) {
        do {
          double d;
          bool isInt;
          int64_t i = 0;
          if (!number(d, isInt, i) || !isInt) return fail("expected integer");
          op.ints.push_back(i);
        } while (acceptTok(","));
        if (!tok("]")) return false;
      }
      double d;
      bool isInt;
      int64_t align = 0;
      if (!keyword("align") || !number(d, isInt, align) || !tok("->")) return false;
      op.ints.push_back(align);
      do {
        const std::string_view s = word();
        if (s.empty()) return fail("expected symbol name");
        op.symbols.push_back(m_->dims().sym(s)->value);
      } while (acceptTok(","));
      return attrDict(op) && results(op, names);
    }
    if (kw == "dim.read") {
      op.kind = OpKind::DimRead;
      ValueId src;
      double d;
      bool isInt;
      int64_t idx = 0;
      if (!use(src) || !tok("[") || !number(d, isInt, idx) || !tok("]") || !tok("->")) return false;
      const std::string_view s = word();
      if (s.empty()) return fail("expected symbol name");
      op.operands.push_back(src);
      op.ints.push_back(idx);
      op.symbols.push_back(m_->dims().sym(s)->value);
      return true;
    }
    if (kw == "sync") {
      op.kind = OpKind::Sync;
      const std::string_view k = word();
      if (k == "gpu_to_cpu") op.ints.push_back(kGpuToCpu);
      else if (k == "cpu_to_gpu") op.ints.push_back(kCpuToGpu);
      else return fail("expected gpu_to_cpu or cpu_to_gpu");
      if (names.empty()) return true;
      ValueId v;
      if (!use(v)) return false;
      op.operands.push_back(v);
      return results(op, names);
    }
    if (kw == "return") {
      op.kind = OpKind::Return;
      if (peekTok("%")) {
        do {
          ValueId v;
          if (!use(v)) return false;
          op.operands.push_back(v);
        } while (acceptTok(","));
      }
      return true;
    }
    return fail("unknown op '" + kw + "'");
  }

  std::string_view s_;
  size_t i_ = 0;
  int line_ = 1;
  std::string err_;
  std::unique_ptr<Model> m_;
  std::unordered_map<std::string, ValueId> values_;
};

}  // namespace

std::unique_ptr<Model> parseModel(std::string_view text, Status& st) { return TextReader(text).run(st); }

}  // namespace lkrt
