// Model verifier: structural rules (SSA order, op shapes, symbol binding, buffer form), device residency across
// explicit sync ops, and in-place write rules (the reference's rules: lariaus/lokinfer src/ir/verify.cpp,
// verify_devices.cpp, docs/verifier.md). It never changes the model.
#include <algorithm>

#include "ir.h"

namespace lkrt {

namespace {

int64_t staticBytes(Type t) {
  int64_t n = static_cast<int64_t>(dtypeSize(t->dtype));
  for (Dim d : t->shape) {
    if (!d->isConst() || d->value < 0) return -1;
    n *= d->value;
  }
  return n;
}

bool bufferForm(const Region& r) {
  for (const Op& op : r.ops)
    if ((op.kind == OpKind::Kernel && !op.outs.empty()) || op.kind == OpKind::BufferFree ||
        op.kind == OpKind::MemPlan)
      return true;
  return false;
}

class Checker {
 public:
  explicit Checker(const Model& m)
      : m_(m), defined_(m.numValues(), 0), bound_(m.dims().numSymbols(), 0),
        buffersOnly_(bufferForm(m.init) || bufferForm(m.exec)) {}

  Status run() {
    if (!m_.init.args.empty() || !m_.init.state.empty()) return fail("init must not have arguments");
    LKRT_TRY(region(m_.init, "init"));
    for (ValueId v : m_.exec.args) bindTypeSymbols(m_.typeOf(v));
    const Op& ret = m_.init.ops.back();
    if (ret.operands.size() != m_.exec.state.size())
      return fail("exec state count (" + std::to_string(m_.exec.state.size()) + ") != init results (" +
                  std::to_string(ret.operands.size()) + ")");
    for (size_t i = 0; i < m_.exec.state.size(); ++i)
      if (m_.typeOf(ret.operands[i]) != m_.typeOf(m_.exec.state[i]))
        return fail("exec state #" + std::to_string(i) + " type differs from init result");
    std::fill(defined_.begin(), defined_.end(), 0);
    for (ValueId v : m_.exec.args) LKRT_TRY(define(v, "exec argument"));
    for (ValueId v : m_.exec.state) LKRT_TRY(define(v, "exec state"));
    LKRT_TRY(region(m_.exec, "exec"));
    return writes();
  }

 private:
  Status fail(const std::string& msg) const { return Status::error("verify: " + msg); }
  Status failOp(const Op& op, const std::string& msg) const {
    return fail(std::string(opKindName(op.kind)) + " " + op.name + ": " + msg);
  }
  void bindTypeSymbols(Type t) {
    std::vector<int64_t> syms;
    for (Dim d : t->shape) collectSymbols(d, syms);
    for (int64_t s : syms)
      if (s >= 0 && static_cast<size_t>(s) < bound_.size()) bound_[s] = 1;
  }
  int64_t unboundIn(Dim d) const {
    std::vector<int64_t> syms;
    collectSymbols(d, syms);
    for (int64_t s : syms)
      if (s < 0 || static_cast<size_t>(s) >= bound_.size() || !bound_[s]) return s;
    return -1;
  }
  Status define(ValueId v, const char* what) {
    if (v >= m_.numValues()) return fail(std::string(what) + ": invalid value id");
    if (defined_[v]) return fail(std::string(what) + ": value defined twice");
    defined_[v] = 1;
    Type t = m_.typeOf(v);
    if (buffersOnly_ && t->isTensor()) return fail(std::string(what) + " has tensor type after bufferization");
    for (Dim d : t->shape)
      if (int64_t s = unboundIn(d); s >= 0)
        return fail(std::string(what) + " uses unbound symbol " + m_.dims().symbolName(s));
    return Status();
  }
  Status region(const Region& r, const char* name) {
    if (r.ops.empty() || r.ops.back().kind != OpKind::Return) return fail(std::string(name) + " must end with return");
    for (size_t i = 0; i < r.ops.size(); ++i) {
      const Op& op = r.ops[i];
      if (op.kind == OpKind::Return && i + 1 != r.ops.size()) return fail(std::string(name) + ": return not last");
      for (const auto* vs : {&op.operands, &op.outs})
        for (ValueId v : *vs)
          if (v >= m_.numValues() || !defined_[v]) return failOp(op, "use of a value not defined before it in this region");
      LKRT_TRY(shape(op));
      for (int64_t s : op.symbols) {
        if (s < 0 || static_cast<size_t>(s) >= bound_.size()) return failOp(op, "invalid symbol id");
        bound_[s] = 1;
      }
      for (Dim d : op.dims)
        if (int64_t s = unboundIn(d); s >= 0) return failOp(op, "uses unbound symbol " + m_.dims().symbolName(s));
      for (ValueId v : op.results) LKRT_TRY(define(v, opKindName(op.kind)));
    }
    return Status();
  }
  Status arity(const Op& op, size_t operands, size_t results) const {
    if (op.operands.size() != operands || op.results.size() != results)
      return failOp(op, "expected " + std::to_string(operands) + " operands and " + std::to_string(results) +
                            " results");
    return Status();
  }
  Status shape(const Op& op) const {
    auto type = [&](ValueId v) { return m_.typeOf(v); };
    switch (op.kind) {
      case OpKind::Kernel:
        if (op.name.empty()) return failOp(op, "missing kernel name");
        for (ValueId v : op.outs)
          if (!type(v)->isBuffer()) return failOp(op, "outs must be buffers");
        return Status();
      case OpKind::ConstInline: {
        LKRT_TRY(arity(op, 0, 1));
        const int64_t n = staticBytes(type(op.results[0]));
        if (n < 0) return failOp(op, "inline constant must have a static shape");
        if (op.data.size() != static_cast<size_t>(n))
          return failOp(op, "data has " + std::to_string(op.data.size()) + " bytes, type needs " + std::to_string(n));
        return Status();
      }
      case OpKind::ConstInternal:
        LKRT_TRY(arity(op, 0, 1));
        return m_.findConstant(op.name) ? Status() : failOp(op, "unknown internal constant");
      case OpKind::ConstExternal:
        return arity(op, 0, 1);
      case OpKind::View: {
        LKRT_TRY(arity(op, 1, 1));
        if (op.dims.size() != 1) return failOp(op, "missing offset");
        Type src = type(op.operands[0]), dst = type(op.results[0]);
        if (src->kind != dst->kind || src->isScalar()) return failOp(op, "view must map tensor->tensor or buffer->buffer");
        const int64_t sb = staticBytes(src), db = staticBytes(dst);
        if (sb >= 0 && db >= 0 && op.dims[0]->isConst()) {
          const int64_t off = op.dims[0]->value * static_cast<int64_t>(dtypeSize(dst->dtype));
          if (op.dims[0]->value < 0 || off + db > sb) return failOp(op, "view out of bounds of its source");
        }
        return Status();
      }
      case OpKind::BufferAlloc:
        LKRT_TRY(arity(op, 0, 1));
        return type(op.results[0])->isBuffer() ? Status() : failOp(op, "result must be a buffer");
      case OpKind::BufferFree:
        LKRT_TRY(arity(op, 1, 0));
        return type(op.operands[0])->isBuffer() ? Status() : failOp(op, "operand must be a buffer");
      case OpKind::MemPlan: {
        LKRT_TRY(arity(op, 0, 1));
        if (op.ints.size() != 2 * op.dims.size() + 1) return failOp(op, "live list must have 2 entries per size");
        if (op.symbols.size() != op.dims.size() + 1) return failOp(op, "must define arena size + one offset per size");
        if (!type(op.results[0])->isBuffer()) return failOp(op, "result must be a buffer");
        if (const AttrValue* e = op.attr("elem")) {
          const Ints* v = std::get_if<Ints>(e);
          if (!v || v->size() != op.dims.size()) return failOp(op, "elem must list one element size per buffer");
          for (int64_t b : *v)
            if (b <= 0 || op.ints.back() % b != 0) return failOp(op, "elem sizes must be positive divisors of align");
        }
        return Status();
      }
      case OpKind::DimRead: {
        LKRT_TRY(arity(op, 1, 0));
        Type t = type(op.operands[0]);
        if (t->isScalar() || (t->dtype != DType::I32 && t->dtype != DType::I64))
          return failOp(op, "operand must be an i32/i64 tensor or buffer");
        if (op.symbols.size() != 1 || op.ints.size() != 1) return failOp(op, "malformed");
        if (op.ints[0] < 0) return failOp(op, "negative index");
        const int64_t n = staticBytes(t);
        if (n >= 0 && op.ints[0] * static_cast<int64_t>(dtypeSize(t->dtype)) >= n) return failOp(op, "index out of bounds");
        return Status();
      }
      case OpKind::Sync:
        if (op.ints.size() != 1 || (op.ints[0] != 0 && op.ints[0] != 1)) return failOp(op, "malformed");
        if (op.operands.empty()) return arity(op, 0, 0);
        LKRT_TRY(arity(op, 1, 1));
        return type(op.operands[0]) == type(op.results[0]) ? Status() : failOp(op, "result type must equal operand type");
      case OpKind::Return:
        return op.results.empty() ? Status() : failOp(op, "return has no results");
    }
    return failOp(op, "unknown op kind");
  }

  // In-place writes (`inout` operands) may only target a mutable exec input or persistent state, and neither may
  // be returned (a mutable input stays the caller's, persistent state stays the model's).
  Status writes() const {
    const Region& r = m_.exec;
    if (!r.mutableArgs.empty() && r.mutableArgs.size() != r.args.size()) return fail("exec: mutable flags != args");
    const size_t nv = m_.numValues();
    std::vector<ValueId> root(nv, kNoValue);
    auto rootOf = [&](ValueId v) { return root[v] == kNoValue ? v : root[v]; };
    std::vector<uint8_t> writable(nv, 0);  // 1 mutable input, 2 persistent
    {
      std::vector<ValueId> iroot(nv, kNoValue);
      std::vector<uint8_t> persistent(nv, 0);
      auto irootOf = [&](ValueId v) { return iroot[v] == kNoValue ? v : iroot[v]; };
      for (const Op& op : m_.init.ops) {
        if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
          iroot[op.results[0]] = irootOf(op.operands[0]);
        if (op.kind == OpKind::BufferAlloc && op.flag("persistent")) persistent[op.results[0]] = 1;
      }
      const Op& ret = m_.init.ops.back();
      for (size_t i = 0; i < r.state.size() && i < ret.operands.size(); ++i)
        if (persistent[irootOf(ret.operands[i])]) writable[r.state[i]] = 2;
    }
    for (size_t i = 0; i < r.args.size(); ++i) {
      if (!r.isMutable(i)) continue;
      if (!m_.typeOf(r.args[i])->isBuffer()) return fail("exec argument #" + std::to_string(i) + " is mutable but not a buffer");
      writable[r.args[i]] = 1;
    }
    for (const Op& op : r.ops) {
      if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
        root[op.results[0]] = rootOf(op.operands[0]);
      if (op.kind == OpKind::BufferAlloc && op.flag("persistent")) writable[op.results[0]] = 2;
      if (op.kind == OpKind::Kernel)
        if (const AttrValue* io = op.attr("inout")) {
          const Ints* idx = std::get_if<Ints>(io);
          if (!idx) return failOp(op, "inout must be an int list");
          for (int64_t j : *idx) {
            if (j < 0 || static_cast<size_t>(j) >= op.operands.size()) return failOp(op, "inout index out of range");
            if (!writable[rootOf(op.operands[static_cast<size_t>(j)])])
              return failOp(op, "writes operand #" + std::to_string(j) +
                                    " in place, but it is neither a mutable input nor persistent state: declare the "
                                    "input mutable");
          }
        }
      if (op.kind == OpKind::Return)
        for (ValueId v : op.operands)
          if (writable[rootOf(v)])
            return failOp(op, std::string("returns ") + (writable[rootOf(v)] == 1 ? "a mutable input" : "persistent state") +
                                  " (or a view of it); return a copy");
    }
    return Status();
  }

  const Model& m_;
  std::vector<uint8_t> defined_, bound_;
  bool buffersOnly_;
};

// Residency: constants and persistent allocs sit on their `device` attr; kernel results (and inout operands) on the
// kernel's device; views on their source's; a sync's result on its target; inputs on either. A kernel may not read
// a value resident on the other device, and dim.read (a host read) may not read a GPU-resident value.
enum class Res : uint8_t { Any, Cpu, Gpu };

Status residency(const Model& m, const Region& r, const char* name, const std::vector<std::pair<ValueId, Res>>& seed,
                 std::vector<Res>* retRes) {
  std::vector<Res> res(m.numValues(), Res::Any);
  for (auto [v, x] : seed) res[v] = x;
  auto nameOf = [&](ValueId v) { return "%" + (m.nameOf(v).empty() ? std::to_string(v) : m.nameOf(v)); };
  auto deviceAttr = [&](const Op& op, Res& out) -> Status {
    const AttrValue* a = op.attr("device");
    if (!a) return Status();
    const std::string* s = std::get_if<std::string>(a);
    if (!s || (*s != "cpu" && *s != "gpu")) return Status::error("verify: device must be \"cpu\" or \"gpu\"");
    out = *s == "gpu" ? Res::Gpu : Res::Cpu;
    return Status();
  };
  for (const Op& op : r.ops) {
    switch (op.kind) {
      case OpKind::Kernel: {
        const Res dev = isGpuKernelName(op.name) ? Res::Gpu : Res::Cpu;
        for (ValueId v : op.operands)
          if (res[v] != Res::Any && res[v] != dev)
            return Status::error(std::string("verify: devices (") + name + "): kernel '" + op.name + "' runs on " +
                                 (dev == Res::Gpu ? "gpu" : "cpu") + " but operand " + nameOf(v) +
                                 " is resident on " + (res[v] == Res::Gpu ? "gpu" : "cpu"));
        for (ValueId v : op.outs) res[v] = dev;
        for (ValueId v : op.results) res[v] = dev;
        if (const AttrValue* io = op.attr("inout"))
          if (const Ints* idx = std::get_if<Ints>(io))
            for (int64_t j : *idx)
              if (j >= 0 && static_cast<size_t>(j) < op.operands.size()) res[op.operands[static_cast<size_t>(j)]] = dev;
        break;
      }
      case OpKind::BufferAlloc:
      case OpKind::ConstInline:
      case OpKind::ConstInternal:
      case OpKind::ConstExternal:
        LKRT_TRY(deviceAttr(op, res[op.results[0]]));
        break;
      case OpKind::View:
        res[op.results[0]] = res[op.operands[0]];
        break;
      case OpKind::Sync:
        if (!op.results.empty()) res[op.results[0]] = op.ints[0] == kGpuToCpu ? Res::Cpu : Res::Gpu;
        break;
      case OpKind::DimRead:
        if (res[op.operands[0]] == Res::Gpu)
          return Status::error(std::string("verify: devices (") + name + "): dim.read of " + nameOf(op.operands[0]) +
                               " which is resident on gpu");
        break;
      case OpKind::Return:
        if (retRes)
          for (ValueId v : op.operands) retRes->push_back(res[v]);
        break;
      default:
        break;
    }
  }
  return Status();
}

}  // namespace

Status verifyModel(const Model& m) {
  LKRT_TRY(Checker(m).run());
  std::vector<Res> initRes;
  LKRT_TRY(residency(m, m.init, "init", {}, &initRes));
  std::vector<std::pair<ValueId, Res>> seed;
  for (size_t i = 0; i < m.exec.state.size() && i < initRes.size(); ++i)
    if (initRes[i] != Res::Any) seed.emplace_back(m.exec.state[i], initRes[i]);
  return residency(m, m.exec, "exec", seed, nullptr);
}

}  // namespace lkrt
