// Dims, types and model bookkeeping of the runtime IR (formats: lariaus/lokinfer include/lokinfer/ir/dim.h,
// types.h, ir.h; canonical forms: docs/impl-notes/design-ir.md §3).
#include "ir.h"

#include <algorithm>
#include <cctype>
#include <climits>
#include <functional>

namespace lkrt {

// ---- dtypes ----------------------------------------------------------------------------------------------------
namespace {
struct DTypeInfo {
  const char* name;
  size_t size;
};
constexpr DTypeInfo kDTypes[] = {{"f32", 4}, {"f16", 2}, {"bf16", 2}, {"i8", 1}, {"u8", 1},
                                 {"i16", 2}, {"i32", 4}, {"i64", 8}, {"bool", 1}};
}  // namespace

size_t dtypeSize(DType t) { return kDTypes[static_cast<int>(t)].size; }
const char* dtypeName(DType t) { return kDTypes[static_cast<int>(t)].name; }
std::optional<DType> dtypeFromName(std::string_view n) {
  for (int i = 0; i < 9; ++i)
    if (n == kDTypes[i].name) return static_cast<DType>(i);
  return std::nullopt;
}

// ---- integer helpers (floor semantics) --------------------------------------------------------------------------
namespace {
int64_t floorDivI(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}
int64_t ceilDivI(int64_t a, int64_t b) { return -floorDivI(-a, b); }
int64_t floorModI(int64_t a, int64_t b) { return a - floorDivI(a, b) * b; }
}  // namespace

// ---- dim pool --------------------------------------------------------------------------------------------------
size_t DimPool::KeyHash::operator()(const Key& k) const {
  size_t h = std::hash<int64_t>()(k.v) * 1315423911u + static_cast<size_t>(k.k);
  for (Dim d : k.args) h = (h ^ std::hash<const void*>()(d)) * 1099511628211ull;
  return h;
}

Dim DimPool::node(DimKind k, int64_t v, const std::vector<Dim>& args) {
  Key key{k, v, args};
  auto it = table_.find(key);
  if (it != table_.end()) return it->second;
  nodes_.push_back(DimNode{k, v, args, static_cast<uint32_t>(nodes_.size())});
  Dim d = &nodes_.back();
  table_.emplace(std::move(key), d);
  return d;
}

Dim DimPool::constant(int64_t v) { return node(DimKind::Const, v, {}); }

Dim DimPool::sym(std::string_view name) {
  auto it = symIds_.find(std::string(name));
  if (it != symIds_.end()) return symNodes_[static_cast<size_t>(it->second)];
  const int64_t id = static_cast<int64_t>(symNames_.size());
  symNames_.emplace_back(name);
  symIds_.emplace(std::string(name), id);
  Dim d = node(DimKind::Sym, id, {});
  symNodes_.push_back(d);
  return d;
}

int64_t DimPool::findSymbol(std::string_view name) const {
  auto it = symIds_.find(std::string(name));
  return it == symIds_.end() ? -1 : it->second;
}

int DimPool::order(Dim a, Dim b) const {
  if (a == b) return 0;
  if (a->kind != b->kind) return a->kind < b->kind ? -1 : 1;
  if (a->kind == DimKind::Sym) {
    const int c = symNames_[a->value].compare(symNames_[b->value]);
    return c < 0 ? -1 : c > 0 ? 1 : 0;
  }
  if (a->value != b->value) return a->value < b->value ? -1 : 1;
  const size_t n = std::min(a->args.size(), b->args.size());
  for (size_t i = 0; i < n; ++i)
    if (const int c = order(a->args[i], b->args[i])) return c;
  if (a->args.size() == b->args.size()) return 0;
  return a->args.size() < b->args.size() ? -1 : 1;
}

// d == coef * rest (rest == nullptr for a constant)
std::pair<int64_t, Dim> DimPool::coefficient(Dim d) {
  if (d->isConst()) return {d->value, nullptr};
  if (d->kind == DimKind::Mul && d->args[0]->isConst()) {
    if (d->args.size() == 2) return {d->args[0]->value, d->args[1]};
    return {d->args[0]->value, node(DimKind::Mul, 0, std::vector<Dim>(d->args.begin() + 1, d->args.end()))};
  }
  return {1, d};
}

Dim DimPool::sum(std::vector<Dim> terms) {
  int64_t c = 0;
  std::vector<std::pair<Dim, int64_t>> like;  // (rest, coefficient) in first-appearance order
  std::function<void(Dim)> visit = [&](Dim t) {
    if (t->kind == DimKind::Add) {
      for (Dim x : t->args) visit(x);
      return;
    }
    auto [k, rest] = coefficient(t);
    if (!rest) {
      c += k;
      return;
    }
    for (auto& e : like)
      if (e.first == rest) {
        e.second += k;
        return;
      }
    like.emplace_back(rest, k);
  };
  for (Dim t : terms) visit(t);
  std::vector<Dim> out;
  for (auto& [rest, k] : like)
    if (k != 0) out.push_back(k == 1 ? rest : product({constant(k), rest}));
  if (c != 0 || out.empty()) out.push_back(constant(c));
  if (out.size() == 1) return out[0];
  std::sort(out.begin(), out.end(), [&](Dim a, Dim b) { return order(a, b) < 0; });
  return node(DimKind::Add, 0, out);
}

Dim DimPool::product(std::vector<Dim> factors) {
  int64_t c = 1;
  std::vector<Dim> rest;
  std::function<void(Dim)> visit = [&](Dim f) {
    if (f->kind == DimKind::Mul) {
      for (Dim x : f->args) visit(x);
    } else if (f->isConst()) {
      c *= f->value;
    } else {
      rest.push_back(f);
    }
  };
  for (Dim f : factors) visit(f);
  if (c == 0 || rest.empty()) return constant(c);
  if (c != 1 && rest.size() == 1 && rest[0]->kind == DimKind::Add) {  // k * (a + b) -> k*a + k*b
    std::vector<Dim> terms;
    for (Dim t : rest[0]->args) terms.push_back(product({constant(c), t}));
    return sum(std::move(terms));
  }
  std::sort(rest.begin(), rest.end(), [&](Dim a, Dim b) { return order(a, b) < 0; });
  if (c == 1 && rest.size() == 1) return rest[0];
  if (c != 1) rest.insert(rest.begin(), constant(c));
  return node(DimKind::Mul, 0, rest);
}

// d / c when every term of d is a multiple of c, else nullptr
Dim DimPool::divideExactly(Dim d, int64_t c) {
  if (c == 1) return d;
  if (d->isConst()) return d->value % c == 0 ? constant(d->value / c) : nullptr;
  if (d->kind == DimKind::Add) {
    std::vector<Dim> q;
    for (Dim t : d->args) {
      Dim x = divideExactly(t, c);
      if (!x) return nullptr;
      q.push_back(x);
    }
    return sum(std::move(q));
  }
  if (d->kind == DimKind::Mul) {
    auto [k, rest] = coefficient(d);
    return k % c == 0 ? product({constant(k / c), rest}) : nullptr;
  }
  return nullptr;
}

// a = q * c + r with r constant: every non-constant term of a must be an exact multiple of c
bool DimPool::splitMultiple(Dim a, int64_t c, Dim& q, int64_t& r) {
  std::vector<Dim> terms;
  r = 0;
  std::vector<Dim> parts = a->kind == DimKind::Add ? a->args : std::vector<Dim>{a};
  for (Dim t : parts) {
    if (t->isConst()) {
      r += t->value;
      continue;
    }
    Dim x = divideExactly(t, c);
    if (!x) return false;
    terms.push_back(x);
  }
  q = terms.empty() ? constant(0) : sum(std::move(terms));
  return true;
}

Dim DimPool::floorDiv(Dim a, Dim b) {
  if (a->isConst() && b->isConst()) return constant(floorDivI(a->value, b->value));
  if (b->isConst(1) || a->isConst(0)) return a;
  if (a == b) return constant(1);
  if (b->isConst() && b->value > 0) {
    Dim q;
    int64_t r;
    if (splitMultiple(a, b->value, q, r)) return add(q, constant(floorDivI(r, b->value)));
  }
  return node(DimKind::FloorDiv, 0, {a, b});
}

Dim DimPool::ceilDiv(Dim a, Dim b) {
  if (a->isConst() && b->isConst()) return constant(ceilDivI(a->value, b->value));
  if (b->isConst(1) || a->isConst(0)) return a;
  if (a == b) return constant(1);
  if (b->isConst() && b->value > 0) {
    Dim q;
    int64_t r;
    if (splitMultiple(a, b->value, q, r)) return add(q, constant(ceilDivI(r, b->value)));
  }
  return node(DimKind::CeilDiv, 0, {a, b});
}

Dim DimPool::mod(Dim a, Dim b) {
  if (a->isConst() && b->isConst()) return constant(floorModI(a->value, b->value));
  if (b->isConst(1) || a == b || a->isConst(0)) return constant(0);
  if (b->isConst() && b->value > 0) {
    Dim q;
    int64_t r;
    if (splitMultiple(a, b->value, q, r)) return constant(floorModI(r, b->value));
  }
  return node(DimKind::Mod, 0, {a, b});
}

Dim DimPool::min(Dim a, Dim b) {
  if (a->isConst() && b->isConst()) return constant(std::min(a->value, b->value));
  if (a == b) return a;
  if (order(b, a) < 0) std::swap(a, b);
  return node(DimKind::Min, 0, {a, b});
}

Dim DimPool::max(Dim a, Dim b) {
  if (a->isConst() && b->isConst()) return constant(std::max(a->value, b->value));
  if (a == b) return a;
  if (order(b, a) < 0) std::swap(a, b);
  return node(DimKind::Max, 0, {a, b});
}

std::optional<int64_t> DimPool::eval(Dim d, const std::vector<int64_t>& sv, int64_t unbound) const {
  switch (d->kind) {
    case DimKind::Const: return d->value;
    case DimKind::Sym:
      if (static_cast<size_t>(d->value) >= sv.size() || sv[static_cast<size_t>(d->value)] == unbound)
        return std::nullopt;
      return sv[static_cast<size_t>(d->value)];
    case DimKind::Add:
    case DimKind::Mul: {
      int64_t r = d->kind == DimKind::Add ? 0 : 1;
      for (Dim x : d->args) {
        auto v = eval(x, sv, unbound);
        if (!v) return std::nullopt;
        r = d->kind == DimKind::Add ? r + *v : r * *v;
      }
      return r;
    }
    default: {
      auto a = eval(d->args[0], sv, unbound), b = eval(d->args[1], sv, unbound);
      if (!a || !b) return std::nullopt;
      switch (d->kind) {
        case DimKind::FloorDiv: return *b ? std::optional<int64_t>(floorDivI(*a, *b)) : std::nullopt;
        case DimKind::CeilDiv: return *b ? std::optional<int64_t>(ceilDivI(*a, *b)) : std::nullopt;
        case DimKind::Mod: return *b ? std::optional<int64_t>(floorModI(*a, *b)) : std::nullopt;
        case DimKind::Min: return std::min(*a, *b);
        default: return std::max(*a, *b);
      }
    }
  }
}

void collectSymbols(Dim d, std::vector<int64_t>& out) {
  if (d->kind == DimKind::Sym) {
    out.push_back(d->value);
    return;
  }
  for (Dim x : d->args) collectSymbols(x, out);
}

// Printing: sums as "a + 2*b - 3", products as "2*N*T", "a // b", "a % b", "ceildiv(a, b)", "min(a, b)",
// "max(a, b)"; operands that are not atoms (a non-negative constant, a symbol, ceildiv / min / max) in parentheses.
std::string DimPool::str(Dim d) const {
  auto atom = [](Dim x) {
    return (x->isConst() && x->value >= 0) || x->kind == DimKind::Sym || x->kind == DimKind::CeilDiv ||
           x->kind == DimKind::Min || x->kind == DimKind::Max;
  };
  auto wrapped = [&](Dim x) { return atom(x) ? str(x) : "(" + str(x) + ")"; };
  switch (d->kind) {
    case DimKind::Const: return std::to_string(d->value);
    case DimKind::Sym: return symNames_[static_cast<size_t>(d->value)];
    case DimKind::Add: {
      std::string s;
      Dim c = nullptr;
      for (Dim t : d->args) {
        if (t->isConst()) {
          c = t;
          continue;
        }
        bool neg = false;
        std::string body;
        if (t->kind == DimKind::Mul && t->args[0]->isConst()) {
          const int64_t k = t->args[0]->value;
          neg = k < 0;
          std::string rest;
          for (size_t i = 1; i < t->args.size(); ++i) rest += (i > 1 ? "*" : "") + wrapped(t->args[i]);
          const int64_t mag = neg ? -k : k;
          body = mag == 1 ? rest : std::to_string(mag) + "*" + rest;
        } else {
          body = str(t);
        }
        s += s.empty() ? (neg ? "-" : "") + body : (neg ? " - " : " + ") + body;
      }
      if (c) s += (c->value < 0 ? " - " : " + ") + std::to_string(c->value < 0 ? -c->value : c->value);
      return s;
    }
    case DimKind::Mul: {
      std::string s;
      size_t i0 = 0;
      if (d->args[0]->isConst() && d->args[0]->value < 0) {
        const int64_t mag = -d->args[0]->value;
        s = mag == 1 ? "-" : "-" + std::to_string(mag) + "*";
        i0 = 1;
      }
      for (size_t i = i0; i < d->args.size(); ++i) s += (i > i0 ? "*" : "") + wrapped(d->args[i]);
      return s;
    }
    case DimKind::FloorDiv: return wrapped(d->args[0]) + " // " + wrapped(d->args[1]);
    case DimKind::Mod: return wrapped(d->args[0]) + " % " + wrapped(d->args[1]);
    case DimKind::CeilDiv: return "ceildiv(" + str(d->args[0]) + ", " + str(d->args[1]) + ")";
    case DimKind::Min: return "min(" + str(d->args[0]) + ", " + str(d->args[1]) + ")";
    case DimKind::Max: return "max(" + str(d->args[0]) + ", " + str(d->args[1]) + ")";
  }
  return "?";
}

// Recursive descent over:  expr := term (('+' | '-') term)* ; term := unary (('*' | '//' | '%') unary)* ;
// unary := '-' unary | primary ; primary := INT | NAME | (ceildiv | min | max) '(' expr ',' expr ')' | '(' expr ')'
namespace {
class DimReader {
 public:
  DimReader(DimPool& p, std::string_view s) : p_(p), s_(s) {}
  Dim all(std::string& err) {
    Dim d = expr(0);
    ws();
    if (err_.empty() && i_ != s_.size()) err_ = "unexpected '" + std::string(s_.substr(i_)) + "' in dim";
    err = err_;
    return err_.empty() ? d : nullptr;
  }

 private:
  void ws() {
    while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
  }
  bool eat(std::string_view t) {
    ws();
    if (s_.compare(i_, t.size(), t) != 0) return false;
    i_ += t.size();
    return true;
  }
  Dim bad(std::string m) {
    if (err_.empty()) err_ = std::move(m);
    return p_.constant(0);
  }
  Dim div(Dim a, Dim b, int kind) {
    if (!err_.empty()) return a;
    if (b->isConst(0)) return bad("division by zero in dim expression");
    return kind == 0 ? p_.floorDiv(a, b) : kind == 1 ? p_.ceilDiv(a, b) : p_.mod(a, b);
  }
  Dim expr(int depth) {
    if (depth > 64) return bad("dim expression nested too deeply");
    Dim a = term(depth);
    while (err_.empty()) {
      if (eat("+")) a = p_.add(a, term(depth));
      else if (eat("-")) a = p_.sub(a, term(depth));
      else break;
    }
    return a;
  }
  Dim term(int depth) {
    Dim a = unary(depth);
    while (err_.empty()) {
      if (eat("//")) a = div(a, unary(depth), 0);
      else if (eat("*")) a = p_.mul(a, unary(depth));
      else if (eat("%")) a = div(a, unary(depth), 2);
      else break;
    }
    return a;
  }
  Dim unary(int depth) {
    if (depth > 64) return bad("dim expression nested too deeply");
    if (eat("-")) return p_.mul(p_.constant(-1), unary(depth + 1));
    return primary(depth);
  }
  Dim primary(int depth) {
    ws();
    if (i_ >= s_.size()) return bad("unexpected end of dim expression");
    const char c = s_[i_];
    if (c == '(') {
      ++i_;
      Dim d = expr(depth + 1);
      return eat(")") ? d : bad("expected ')' in dim expression");
    }
    if (std::isdigit(static_cast<unsigned char>(c))) {
      int64_t v = 0;
      while (i_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_]))) {
        const int dg = s_[i_++] - '0';
        if (v > (INT64_MAX - dg) / 10) return bad("integer too large in dim expression");
        v = v * 10 + dg;
      }
      return p_.constant(v);
    }
    if (std::isalpha(static_cast<unsigned char>(c)) || c == '_') {
      const size_t b = i_;
      while (i_ < s_.size() && (std::isalnum(static_cast<unsigned char>(s_[i_])) || s_[i_] == '_')) ++i_;
      const std::string_view name = s_.substr(b, i_ - b);
      const size_t after = i_;
      if ((name == "ceildiv" || name == "min" || name == "max") && eat("(")) {
        Dim x = expr(depth + 1);
        if (!eat(",")) return bad("expected ',' in " + std::string(name) + "(...)");
        Dim y = expr(depth + 1);
        if (!eat(")")) return bad("expected ')' in " + std::string(name) + "(...)");
        if (name == "ceildiv") return div(x, y, 1);
        return name == "min" ? p_.min(x, y) : p_.max(x, y);
      }
      i_ = after;
      return p_.sym(name);
    }
    return bad(std::string("unexpected character '") + c + "' in dim expression");
  }

  DimPool& p_;
  std::string_view s_;
  size_t i_ = 0;
  std::string err_;
};
}  // namespace

Dim DimPool::parse(std::string_view text, std::string& err) { return DimReader(*this, text).all(err); }

// ---- types -----------------------------------------------------------------------------------------------------
Type TypePool::get(TypeKind kind, DType dt, const std::vector<Dim>& shape) {
  size_t h = static_cast<size_t>(kind) * 131 + static_cast<size_t>(dt);
  for (Dim d : shape) h = (h ^ std::hash<const void*>()(d)) * 1099511628211ull;
  auto range = table_.equal_range(h);
  for (auto it = range.first; it != range.second; ++it) {
    Type t = it->second;
    if (t->kind == kind && t->dtype == dt && t->shape == shape) return t;
  }
  nodes_.push_back(TypeNode{kind, dt, shape, static_cast<uint32_t>(nodes_.size())});
  Type t = &nodes_.back();
  table_.emplace(h, t);
  return t;
}

Dim TypePool::numElements(Type t) {
  Dim n = dims_.constant(1);
  for (Dim d : t->shape) n = dims_.mul(n, d);
  return n;
}

Dim TypePool::numBytes(Type t) {
  return dims_.mul(numElements(t), dims_.constant(static_cast<int64_t>(dtypeSize(t->dtype))));
}

std::string TypePool::str(Type t) const {
  if (t->isScalar()) return dtypeName(t->dtype);
  std::string s = t->isTensor() ? "tensor<" : "buffer<";
  s += dtypeName(t->dtype);
  s += "[";
  for (size_t i = 0; i < t->shape.size(); ++i) s += (i ? ", " : "") + dims_.str(t->shape[i]);
  return s + "]>";
}

// ---- ops and model ---------------------------------------------------------------------------------------------
const char* opKindName(OpKind k) {
  static const char* const names[] = {"kernel",      "const.inline", "const.internal", "const.external",
                                      "view",        "buffer.alloc", "buffer.free",    "mem.plan",
                                      "dim.read",    "sync",         "return"};
  return names[static_cast<int>(k)];
}

bool isStructuralAttr(std::string_view n) {
  static const char* const names[] = {"nohoist", "inplace", "output", "arena", "device",
                                      "persistent", "inout", "gpu_only", "elem"};
  for (const char* s : names)
    if (n == s) return true;
  return false;
}

bool isGpuKernelName(std::string_view name) {
  size_t b = 0;
  while (b <= name.size()) {
    size_t e = name.find('_', b);
    if (e == std::string_view::npos) e = name.size();
    if (name.substr(b, e - b) == "gpu") return true;
    b = e + 1;
  }
  return false;
}

const AttrValue* Op::attr(std::string_view n) const {
  for (const NamedAttr& a : attrs)
    if (a.name == n) return &a.value;
  return nullptr;
}

void Op::setAttr(std::string n, AttrValue v) {
  auto it = std::lower_bound(attrs.begin(), attrs.end(), n,
                             [](const NamedAttr& a, const std::string& k) { return a.name < k; });
  if (it != attrs.end() && it->name == n) it->value = std::move(v);
  else attrs.insert(it, NamedAttr{std::move(n), std::move(v)});
}

bool Op::flag(std::string_view n) const {
  const AttrValue* a = attr(n);
  return a && std::holds_alternative<bool>(*a) && std::get<bool>(*a);
}

void Model::addConstant(Constant c) {
  constIndex_[c.name] = constants.size();
  constants.push_back(std::move(c));
}

const Constant* Model::findConstant(std::string_view name) const {
  auto it = constIndex_.find(std::string(name));
  return it == constIndex_.end() ? nullptr : &constants[it->second];
}

Constant* Model::findConstant(std::string_view name) {
  auto it = constIndex_.find(std::string(name));
  return it == constIndex_.end() ? nullptr : &constants[it->second];
}

}  // namespace lkrt
