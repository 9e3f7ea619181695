// In-memory IR of lokinfer's compiled models, host side of the MI355X runtime.
//
// The model format is the reference's (lariaus/lokinfer include/lokinfer/ir/ir.h, types.h, dim.h): a model owns
// hash-consed symbolic dims, interned types, a value table and two regions, `init` (runs once when an executable is
// created) and `exec` (runs per call). The enum values below are the .lkm v2 encoding and must not change.
#pragma once

#include <cstdint>
#include <deque>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <unordered_map>
#include <variant>
#include <vector>

namespace lkrt {

// ---- status --------------------------------------------------------------------------------------------------
class Status {
 public:
  Status() = default;
  static Status error(std::string msg) {
    Status s;
    s.msg_ = std::make_shared<std::string>(std::move(msg));
    return s;
  }
  bool ok() const { return !msg_; }
  explicit operator bool() const { return ok(); }
  const std::string& message() const {
    static const std::string empty;
    return msg_ ? *msg_ : empty;
  }

 private:
  std::shared_ptr<std::string> msg_;
};

#define LKRT_TRY(expr)              \
  do {                              \
    ::lkrt::Status s_ = (expr);     \
    if (!s_.ok()) return s_;        \
  } while (0)

// ---- dtypes ----------------------------------------------------------------------------------------------------
enum class DType : uint8_t { F32, F16, BF16, I8, U8, I16, I32, I64, Bool };
size_t dtypeSize(DType t);
const char* dtypeName(DType t);
std::optional<DType> dtypeFromName(std::string_view n);

// ---- symbolic dims ---------------------------------------------------------------------------------------------
enum class DimKind : uint8_t { Const, Sym, Add, Mul, FloorDiv, CeilDiv, Mod, Min, Max };

struct DimNode {
  DimKind kind;
  int64_t value;                       // Const: the value; Sym: symbol id; else 0
  std::vector<const DimNode*> args;    // Add / Mul: n-ary, sorted; Min / Max: sorted pair; others: (a, b)
  uint32_t id;                         // creation index (dense tables)
  bool isConst() const { return kind == DimKind::Const; }
  bool isConst(int64_t v) const { return kind == DimKind::Const && value == v; }
};
using Dim = const DimNode*;

// Owns every dim node of a model. Construction canonicalizes (constant folding, flattened and sorted Add / Mul,
// like terms merged, a constant factor distributed over a single sum, exact affine division), so two equal forms
// are one pointer.
class DimPool {
 public:
  Dim constant(int64_t v);
  Dim sym(std::string_view name);
  Dim add(Dim a, Dim b) { return sum({a, b}); }
  Dim sub(Dim a, Dim b) { return sum({a, mul(constant(-1), b)}); }
  Dim mul(Dim a, Dim b) { return product({a, b}); }
  Dim floorDiv(Dim a, Dim b);
  Dim ceilDiv(Dim a, Dim b);
  Dim mod(Dim a, Dim b);
  Dim min(Dim a, Dim b);
  Dim max(Dim a, Dim b);

  size_t numSymbols() const { return symNames_.size(); }
  size_t numNodes() const { return nodes_.size(); }
  const std::string& symbolName(int64_t id) const { return symNames_[static_cast<size_t>(id)]; }
  int64_t findSymbol(std::string_view name) const;

  std::string str(Dim d) const;
  // Parses str()'s form (and redundant parentheses); error text in `err`.
  Dim parse(std::string_view text, std::string& err);
  // Structural order used to sort operands (independent of creation order).
  int order(Dim a, Dim b) const;

  // Evaluates with symbol values indexed by symbol id; nullopt when a needed symbol is `unbound` or a divisor is 0.
  std::optional<int64_t> eval(Dim d, const std::vector<int64_t>& sv, int64_t unbound) const;

 private:
  Dim node(DimKind k, int64_t v, const std::vector<Dim>& args);
  Dim sum(std::vector<Dim> terms);
  Dim product(std::vector<Dim> factors);
  std::pair<int64_t, Dim> coefficient(Dim d);
  Dim divideExactly(Dim d, int64_t c);
  bool splitMultiple(Dim a, int64_t c, Dim& q, int64_t& r);

  struct Key {
    DimKind k;
    int64_t v;
    std::vector<Dim> args;
    bool operator==(const Key& o) const { return k == o.k && v == o.v && args == o.args; }
  };
  struct KeyHash {
    size_t operator()(const Key& k) const;
  };
  std::deque<DimNode> nodes_;
  std::unordered_map<Key, Dim, KeyHash> table_;
  std::vector<std::string> symNames_;
  std::vector<Dim> symNodes_;
  std::unordered_map<std::string, int64_t> symIds_;
};

void collectSymbols(Dim d, std::vector<int64_t>& out);

// ---- types -----------------------------------------------------------------------------------------------------
enum class TypeKind : uint8_t { Scalar, Tensor, Buffer };

struct TypeNode {
  TypeKind kind;
  DType dtype;
  std::vector<Dim> shape;
  uint32_t id;
  bool isScalar() const { return kind == TypeKind::Scalar; }
  bool isTensor() const { return kind == TypeKind::Tensor; }
  bool isBuffer() const { return kind == TypeKind::Buffer; }
};
using Type = const TypeNode*;

class TypePool {
 public:
  explicit TypePool(DimPool& dims) : dims_(dims) {}
  Type get(TypeKind kind, DType dt, const std::vector<Dim>& shape);
  Type scalar(DType dt) { return get(TypeKind::Scalar, dt, {}); }
  Type buffer(DType dt, const std::vector<Dim>& shape) { return get(TypeKind::Buffer, dt, shape); }
  Type withKind(Type t, TypeKind k) { return get(k, t->dtype, t->shape); }
  Dim numElements(Type t);
  Dim numBytes(Type t);
  std::string str(Type t) const;
  size_t size() const { return nodes_.size(); }

 private:
  DimPool& dims_;
  std::deque<TypeNode> nodes_;
  std::unordered_multimap<size_t, Type> table_;
};

// ---- ops -------------------------------------------------------------------------------------------------------
using ValueId = uint32_t;
constexpr ValueId kNoValue = ~0u;

// Attribute values; the variant index is the .lkm attribute tag.
using Ints = std::vector<int64_t>;
using Floats = std::vector<double>;
using AttrValue = std::variant<bool, int64_t, double, std::string, Ints, Floats, Dim>;
struct NamedAttr {
  std::string name;
  AttrValue value;
};

enum class OpKind : uint8_t {
  Kernel, ConstInline, ConstInternal, ConstExternal, View, BufferAlloc, BufferFree, MemPlan, DimRead, Sync, Return
};
const char* opKindName(OpKind k);
enum SyncKind : int64_t { kGpuToCpu = 0, kCpuToGpu = 1 };

// Compiler / runtime attributes, never part of a kernel's int / float arguments.
bool isStructuralAttr(std::string_view name);
// A kernel runs on the GPU iff one '_'-separated token of its name is "gpu".
bool isGpuKernelName(std::string_view name);

struct Op {
  OpKind kind = OpKind::Return;
  std::string name;
  std::vector<ValueId> operands, outs, results;
  std::vector<NamedAttr> attrs;  // sorted by name
  std::vector<uint8_t> data;     // const.inline bytes
  std::vector<Dim> dims;         // view: offset; mem.plan: sizes
  std::vector<int64_t> ints;     // mem.plan: live pairs then alignment; dim.read: index; sync: kind
  std::vector<int64_t> symbols;  // symbols this op defines

  const AttrValue* attr(std::string_view n) const;
  void setAttr(std::string n, AttrValue v);
  bool flag(std::string_view n) const;
};

struct Region {
  std::vector<ValueId> args;
  std::vector<uint8_t> mutableArgs;  // exec: empty, or one flag per arg
  std::vector<ValueId> state;        // exec: init's results, by position
  std::vector<Op> ops;               // ends with a Return
  bool isMutable(size_t i) const { return i < mutableArgs.size() && mutableArgs[i]; }
};

struct Constant {
  std::string name;
  Type type = nullptr;
  std::shared_ptr<const void> owner;  // keeps `bytes` alive (an mmapped file, an owned copy, a caller's array)
  const uint8_t* bytes = nullptr;
  size_t size = 0;
};

class Model {
 public:
  Model() : types_(dims_) {}
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  DimPool& dims() { return dims_; }
  const DimPool& dims() const { return dims_; }
  TypePool& types() { return types_; }
  const TypePool& types() const { return types_; }

  ValueId newValue(Type t, std::string name = {}) {
    values_.push_back({t, std::move(name)});
    return static_cast<ValueId>(values_.size() - 1);
  }
  Type typeOf(ValueId v) const { return values_[v].type; }
  void setType(ValueId v, Type t) { values_[v].type = t; }
  const std::string& nameOf(ValueId v) const { return values_[v].name; }
  size_t numValues() const { return values_.size(); }

  void addConstant(Constant c);
  const Constant* findConstant(std::string_view name) const;
  Constant* findConstant(std::string_view name);

  Region init, exec;
  std::vector<Constant> constants;

 private:
  struct Value {
    Type type;
    std::string name;
  };
  DimPool dims_;
  TypePool types_;
  std::vector<Value> values_;
  std::unordered_map<std::string, size_t> constIndex_;
};

// ---- text, binary, verification, passes -----------------------------------------------------------------------
std::string printModel(const Model& m);
// const.internal names without data become constants with no bytes (bound later, or from a .lkm).
std::unique_ptr<Model> parseModel(std::string_view text, Status& st);

std::vector<uint8_t> writeLkm(const Model& m, Status& st);
// `owner` keeps `bytes` alive; constants point into it (zero copy).
std::unique_ptr<Model> readLkm(const uint8_t* bytes, size_t size, std::shared_ptr<const void> owner, Status& st);
Status writeLkmFile(const Model& m, const std::string& path);
std::unique_ptr<Model> readLkmFile(const std::string& path, Status& st);

Status verifyModel(const Model& m);

Status runPass(Model& m, std::string_view name);
const std::vector<std::string>& defaultPipeline();
// const.external -> const.internal for the externals whose bytes are given (copy = true: the model owns a copy).
struct ExternalBytes {
  std::string name;
  const uint8_t* bytes;
  size_t size;
  std::shared_ptr<const void> owner;
};
Status internalize(Model& m, const std::vector<ExternalBytes>& data, bool copy);

// Greedy-by-size, best-fit offset assignment for buffers with [start, end] op-index lifetimes (shared by the
// compiler's static arenas and the runtime's mem.plan).
struct PlanItem {
  int64_t bytes, start, end;
};
int64_t planOffsets(const std::vector<PlanItem>& items, int64_t align, std::vector<int64_t>& offsets);

}  // namespace lkrt
