// Model verifier. The rules are the reference's (lariaus/lokinfer docs/verifier.md: structure, device residency
// across explicit syncs, in-place writes); the checks are organised here as three independent analyses over the
// model, each a forward walk with its own state:
//   1. structure: definitions before uses, symbols bound before use, and a per-op-kind rule table (operand / result
//      counts plus a shape check function per kind);
//   2. residency: which device each value lives on, so that no kernel reads the other device's value and no host
//      read (dim.read) touches a GPU value;
//   3. write rights: in-place (`inout`) writes only into a mutable input or persistent state, neither returned.
// The verifier never changes the model.
#include <algorithm>

#include "ir.h"

namespace lkrt {

namespace {

Status bad(const std::string& msg) { return Status::error("verify: " + msg); }
Status badOp(const Op& op, const std::string& msg) { return bad(std::string(opKindName(op.kind)) + " " + op.name + ": " + msg); }

// bytes of a statically shaped type, -1 when a dim is symbolic
int64_t fixedBytes(Type t) {
  int64_t n = static_cast<int64_t>(dtypeSize(t->dtype));
  for (Dim d : t->shape) {
    if (!d->isConst() || d->value < 0) return -1;
    n *= d->value;
  }
  return n;
}

// ---- 1. structure --------------------------------------------------------------------------------------------------

// per-kind shape checks (operand / result counts are checked from the table first)
using KindCheck = Status (*)(const Model&, const Op&);

Status kernelShape(const Model& m, const Op& op) {
  if (op.name.empty()) return badOp(op, "missing kernel name");
  for (ValueId v : op.outs)
    if (!m.typeOf(v)->isBuffer()) return badOp(op, "outs must be buffers");
  return Status();
}
Status inlineShape(const Model& m, const Op& op) {
  const int64_t need = fixedBytes(m.typeOf(op.results[0]));
  if (need < 0) return badOp(op, "an inline constant needs a static shape");
  if (static_cast<int64_t>(op.data.size()) != need)
    return badOp(op, "data has " + std::to_string(op.data.size()) + " bytes, its type " + std::to_string(need));
  return Status();
}
Status internalShape(const Model& m, const Op& op) {
  return m.findConstant(op.name) ? Status() : badOp(op, "unknown internal constant");
}
Status noShape(const Model&, const Op&) { return Status(); }
Status viewShape(const Model& m, const Op& op) {
  if (op.dims.size() != 1) return badOp(op, "missing offset");
  const Type from = m.typeOf(op.operands[0]), to = m.typeOf(op.results[0]);
  if (from->isScalar() || from->kind != to->kind) return badOp(op, "a view maps tensor to tensor or buffer to buffer");
  const int64_t fromBytes = fixedBytes(from), toBytes = fixedBytes(to);
  if (fromBytes >= 0 && toBytes >= 0 && op.dims[0]->isConst()) {
    const int64_t first = op.dims[0]->value * static_cast<int64_t>(dtypeSize(to->dtype));
    if (op.dims[0]->value < 0 || first + toBytes > fromBytes) return badOp(op, "view out of bounds of its source");
  }
  return Status();
}
Status allocShape(const Model& m, const Op& op) {
  return m.typeOf(op.results[0])->isBuffer() ? Status() : badOp(op, "result must be a buffer");
}
Status freeShape(const Model& m, const Op& op) {
  return m.typeOf(op.operands[0])->isBuffer() ? Status() : badOp(op, "operand must be a buffer");
}
Status planShape(const Model& m, const Op& op) {
  if (op.ints.size() != 2 * op.dims.size() + 1) return badOp(op, "live list must have 2 entries per size");
  if (op.symbols.size() != op.dims.size() + 1) return badOp(op, "must define arena size + one offset per size");
  if (!m.typeOf(op.results[0])->isBuffer()) return badOp(op, "result must be a buffer");
  if (const AttrValue* e = op.attr("elem")) {
    const Ints* sizes = std::get_if<Ints>(e);
    if (!sizes || sizes->size() != op.dims.size()) return badOp(op, "elem must list one element size per buffer");
    for (int64_t b : *sizes)
      if (b <= 0 || op.ints.back() % b) return badOp(op, "elem sizes must be positive divisors of align");
  }
  return Status();
}
Status dimReadShape(const Model& m, const Op& op) {
  const Type t = m.typeOf(op.operands[0]);
  if (t->isScalar() || (t->dtype != DType::I32 && t->dtype != DType::I64))
    return badOp(op, "operand must be an i32/i64 tensor or buffer");
  if (op.symbols.size() != 1 || op.ints.size() != 1) return badOp(op, "malformed");
  if (op.ints[0] < 0) return badOp(op, "negative index");
  const int64_t bytes = fixedBytes(t);
  if (bytes >= 0 && op.ints[0] * static_cast<int64_t>(dtypeSize(t->dtype)) >= bytes)
    return badOp(op, "index out of bounds");
  return Status();
}
Status syncShape(const Model& m, const Op& op) {
  if (op.ints.size() != 1 || (op.ints[0] != kGpuToCpu && op.ints[0] != kCpuToGpu)) return badOp(op, "malformed");
  const size_t n = op.operands.empty() ? 0 : 1;  // a bare sync, or one value moved to the other device
  if (op.operands.size() != n || op.results.size() != n)
    return badOp(op, "expected " + std::to_string(n) + " operands and " + std::to_string(n) + " results");
  if (n && m.typeOf(op.operands[0]) != m.typeOf(op.results[0])) return badOp(op, "result type must equal operand type");
  return Status();
}
Status returnShape(const Model&, const Op& op) {
  return op.results.empty() ? Status() : badOp(op, "return has no results");
}

struct KindRule {
  int operands, results;  // -1: any number (the check function decides)
  KindCheck check;
};
// indexed by OpKind
const KindRule kKindRules[] = {
    {-1, -1, kernelShape},   // kernel
    {0, 1, inlineShape},     // const.inline
    {0, 1, internalShape},   // const.internal
    {0, 1, noShape},         // const.external
    {1, 1, viewShape},       // view
    {0, 1, allocShape},      // buffer.alloc
    {1, 0, freeShape},       // buffer.free
    {0, 1, planShape},       // mem.plan
    {1, 0, dimReadShape},    // dim.read
    {-1, -1, syncShape},     // sync
    {-1, -1, returnShape},   // return
};

class Structure {
 public:
  explicit Structure(const Model& m)
      : m_(m), seen_(m.numValues(), 0), bound_(m.dims().numSymbols(), 0), bufferForm_(isBufferForm(m)) {}

  Status check() {
    if (!m_.init.args.empty() || !m_.init.state.empty()) return bad("init must not have arguments");
    LKRT_TRY(walk(m_.init, "init"));
    const std::vector<ValueId>& initOut = m_.init.ops.back().operands;
    if (initOut.size() != m_.exec.state.size())
      return bad("exec state count (" + std::to_string(m_.exec.state.size()) + ") != init results (" +
                 std::to_string(initOut.size()) + ")");
    for (size_t i = 0; i < initOut.size(); ++i)
      if (m_.typeOf(initOut[i]) != m_.typeOf(m_.exec.state[i]))
        return bad("exec state #" + std::to_string(i) + " type differs from init result");
    // the exec inputs' shapes bind their symbols; exec then sees only its own values
    for (ValueId v : m_.exec.args) markBound(m_.typeOf(v));
    std::fill(seen_.begin(), seen_.end(), 0);
    for (ValueId v : m_.exec.args) LKRT_TRY(introduce(v, "exec argument"));
    for (ValueId v : m_.exec.state) LKRT_TRY(introduce(v, "exec state"));
    return walk(m_.exec, "exec");
  }

 private:
  static bool isBufferForm(const Model& m) {
    for (const Region* r : {&m.init, &m.exec})
      for (const Op& op : r->ops)
        if ((op.kind == OpKind::Kernel && !op.outs.empty()) || op.kind == OpKind::BufferFree ||
            op.kind == OpKind::MemPlan)
          return true;
    return false;
  }
  void markBound(Type t) {
    std::vector<int64_t> syms;
    for (Dim d : t->shape) collectSymbols(d, syms);
    for (int64_t s : syms)
      if (s >= 0 && static_cast<size_t>(s) < bound_.size()) bound_[static_cast<size_t>(s)] = 1;
  }
  // the first symbol of d nothing has bound yet, or -1
  int64_t firstUnbound(Dim d) const {
    std::vector<int64_t> syms;
    collectSymbols(d, syms);
    for (int64_t s : syms)
      if (s < 0 || static_cast<size_t>(s) >= bound_.size() || !bound_[static_cast<size_t>(s)]) return s;
    return -1;
  }
  Status introduce(ValueId v, const std::string& what) {
    if (v >= m_.numValues()) return bad(what + ": invalid value id");
    if (seen_[v]) return bad(what + ": value defined twice");
    seen_[v] = 1;
    const Type t = m_.typeOf(v);
    if (bufferForm_ && t->isTensor()) return bad(what + " has tensor type after bufferization");
    for (Dim d : t->shape)
      if (const int64_t s = firstUnbound(d); s >= 0) return bad(what + " uses unbound symbol " + m_.dims().symbolName(s));
    return Status();
  }
  Status walk(const Region& r, const char* region) {
    if (r.ops.empty() || r.ops.back().kind != OpKind::Return) return bad(std::string(region) + " must end with return");
    for (size_t k = 0; k < r.ops.size(); ++k) {
      const Op& op = r.ops[k];
      if (op.kind == OpKind::Return && k + 1 < r.ops.size()) return bad(std::string(region) + ": return not last");
      for (const std::vector<ValueId>* used : {&op.operands, &op.outs})
        for (ValueId v : *used)
          if (v >= m_.numValues() || !seen_[v]) return badOp(op, "use of a value not defined before it in this region");
      const KindRule& rule = kKindRules[static_cast<int>(op.kind)];
      if ((rule.operands >= 0 && op.operands.size() != static_cast<size_t>(rule.operands)) ||
          (rule.results >= 0 && op.results.size() != static_cast<size_t>(rule.results)))
        return badOp(op, "expected " + std::to_string(rule.operands) + " operands and " + std::to_string(rule.results) +
                             " results");
      LKRT_TRY(rule.check(m_, op));
      for (int64_t s : op.symbols) {
        if (s < 0 || static_cast<size_t>(s) >= bound_.size()) return badOp(op, "invalid symbol id");
        bound_[static_cast<size_t>(s)] = 1;
      }
      for (Dim d : op.dims)
        if (const int64_t s = firstUnbound(d); s >= 0) return badOp(op, "uses unbound symbol " + m_.dims().symbolName(s));
      for (ValueId v : op.results) LKRT_TRY(introduce(v, opKindName(op.kind)));
    }
    return Status();
  }

  const Model& m_;
  std::vector<uint8_t> seen_, bound_;
  bool bufferForm_;
};

// ---- 2. residency ----------------------------------------------------------------------------------------------------
// Constants and allocations sit on their `device` attr (either device without one); kernel results, outs and inout
// operands on the kernel's device; a view on its source's; a sync's result on its target.
enum class Where : uint8_t { Either, Cpu, Gpu };

const char* whereName(Where w) { return w == Where::Gpu ? "gpu" : "cpu"; }

class Residency {
 public:
  explicit Residency(const Model& m) : m_(m), at_(m.numValues(), Where::Either) {}

  // walks a region; returns where its returned values live
  Status walk(const Region& r, const char* region, std::vector<Where>* returned) {
    region_ = region;
    for (const Op& op : r.ops) LKRT_TRY(step(op, returned));
    return Status();
  }
  void place(ValueId v, Where w) { at_[v] = w; }

 private:
  std::string label(ValueId v) const { return "%" + (m_.nameOf(v).empty() ? std::to_string(v) : m_.nameOf(v)); }
  Status step(const Op& op, std::vector<Where>* returned) {
    switch (op.kind) {
      case OpKind::Kernel: {
        const Where dev = isGpuKernelName(op.name) ? Where::Gpu : Where::Cpu;
        for (ValueId v : op.operands)
          if (at_[v] != Where::Either && at_[v] != dev)
            return bad(std::string("devices (") + region_ + "): kernel '" + op.name + "' runs on " + whereName(dev) +
                       " but operand " + label(v) + " is resident on " + whereName(at_[v]));
        for (const std::vector<ValueId>* written : {&op.outs, &op.results})
          for (ValueId v : *written) at_[v] = dev;
        if (const AttrValue* io = op.attr("inout"))
          if (const Ints* idx = std::get_if<Ints>(io))
            for (int64_t j : *idx)
              if (j >= 0 && static_cast<size_t>(j) < op.operands.size()) at_[op.operands[static_cast<size_t>(j)]] = dev;
        return Status();
      }
      case OpKind::BufferAlloc:
      case OpKind::ConstInline:
      case OpKind::ConstInternal:
      case OpKind::ConstExternal: {
        const AttrValue* a = op.attr("device");
        if (!a) return Status();
        const std::string* s = std::get_if<std::string>(a);
        if (!s || (*s != "cpu" && *s != "gpu")) return bad("device must be \"cpu\" or \"gpu\"");
        at_[op.results[0]] = *s == "gpu" ? Where::Gpu : Where::Cpu;
        return Status();
      }
      case OpKind::View: at_[op.results[0]] = at_[op.operands[0]]; return Status();
      case OpKind::Sync:
        if (!op.results.empty()) at_[op.results[0]] = op.ints[0] == kGpuToCpu ? Where::Cpu : Where::Gpu;
        return Status();
      case OpKind::DimRead:
        if (at_[op.operands[0]] == Where::Gpu)
          return bad(std::string("devices (") + region_ + "): dim.read of " + label(op.operands[0]) +
                     " which is resident on gpu");
        return Status();
      case OpKind::Return:
        if (returned)
          for (ValueId v : op.operands) returned->push_back(at_[v]);
        return Status();
      default: return Status();
    }
  }

  const Model& m_;
  std::vector<Where> at_;
  const char* region_ = "";
};

// ---- 3. write rights ---------------------------------------------------------------------------------------------------
enum Right : uint8_t { kNoRight = 0, kMutableInput = 1, kPersistent = 2 };

Status writeRights(const Model& m) {
  const Region& ex = m.exec;
  if (!ex.mutableArgs.empty() && ex.mutableArgs.size() != ex.args.size()) return bad("exec: mutable flags != args");
  const size_t nv = m.numValues();
  // the storage a value is a window on (through views and syncs), per region
  auto origins = [&](const Region& r) {
    std::vector<ValueId> o(nv);
    for (size_t v = 0; v < nv; ++v) o[v] = static_cast<ValueId>(v);
    for (const Op& op : r.ops)
      if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
        o[op.results[0]] = o[op.operands[0]];
    return o;
  };
  std::vector<uint8_t> right(nv, kNoRight);
  {  // exec state that init made from a persistent allocation
    const std::vector<ValueId> io = origins(m.init);
    std::vector<uint8_t> persistent(nv, 0);
    for (const Op& op : m.init.ops)
      if (op.kind == OpKind::BufferAlloc && op.flag("persistent")) persistent[op.results[0]] = 1;
    const std::vector<ValueId>& out = m.init.ops.back().operands;
    for (size_t i = 0; i < ex.state.size() && i < out.size(); ++i)
      if (persistent[io[out[i]]]) right[ex.state[i]] = kPersistent;
  }
  for (size_t i = 0; i < ex.args.size(); ++i) {
    if (!ex.isMutable(i)) continue;
    if (!m.typeOf(ex.args[i])->isBuffer()) return bad("exec argument #" + std::to_string(i) + " is mutable but not a buffer");
    right[ex.args[i]] = kMutableInput;
  }
  const std::vector<ValueId> origin = origins(ex);
  for (const Op& op : ex.ops) {
    if (op.kind == OpKind::BufferAlloc && op.flag("persistent")) right[op.results[0]] = kPersistent;
    if (op.kind == OpKind::Kernel)
      if (const AttrValue* io = op.attr("inout")) {
        const Ints* idx = std::get_if<Ints>(io);
        if (!idx) return badOp(op, "inout must be an int list");
        for (int64_t j : *idx) {
          if (j < 0 || static_cast<size_t>(j) >= op.operands.size()) return badOp(op, "inout index out of range");
          if (right[origin[op.operands[static_cast<size_t>(j)]]] == kNoRight)
            return badOp(op, "writes operand #" + std::to_string(j) +
                                 " in place, but it is neither a mutable input nor persistent state: declare the input "
                                 "mutable");
        }
      }
    if (op.kind == OpKind::Return)
      for (ValueId v : op.operands)
        if (const uint8_t r = right[origin[v]])
          return badOp(op, std::string("returns ") + (r == kMutableInput ? "a mutable input" : "persistent state") +
                               " (or a view of it); return a copy");
  }
  return Status();
}

}  // namespace

Status verifyModel(const Model& m) {
  LKRT_TRY(Structure(m).check());
  LKRT_TRY(writeRights(m));
  Residency initRes(m);
  std::vector<Where> initOut;
  LKRT_TRY(initRes.walk(m.init, "init", &initOut));
  Residency execRes(m);
  for (size_t i = 0; i < m.exec.state.size() && i < initOut.size(); ++i) execRes.place(m.exec.state[i], initOut[i]);
  return execRes.walk(m.exec, "exec", nullptr);
}

}  // namespace lkrt
