// Compiler passes over the runtime IR: dce, bufferize, plan-memory, hoist-init (the default pipeline, in that order)
// and internalize. The contracts are the reference's (lariaus/lokinfer docs/impl-notes/design-compiler-passes.md),
// so a model compiled here prints and saves as the reference's compiler writes it:
//   dce          drops ops whose results nothing live uses (kept: return, dim.read, inout / result-less kernels)
//   bufferize    tensor values become buffers: each kernel result gets a buffer.alloc before the kernel and moves
//                to `outs` (or reuses a dying operand named by `inplace = [out, in, ...]`); a buffer.free follows
//                every alloc's last use (for buffers a CPU op also touches: not before the next gpu_to_cpu sync);
//                returned exec allocs are marked `output`, allocs only GPU kernels touch `gpu_only`
//   plan-memory  frees + non-output allocs become views into arenas: one static arena (constant offsets) for
//                statically sized buffers, else a mem.plan whose offsets are symbols evaluated per call, placed at
//                the region start or right after the dim.read their sizes depend on; gpu_only buffers never share
//                an arena with the others
//   hoist-init   moves what does not depend on exec inputs (constants, static allocs, kernels over constants) into
//                init; the values exec still uses become state
//
// Structure: the passes share a few analyses over a region's op list (value origins through views and syncs, last
// touch per origin, device touches, the init-able subset as a greatest fixpoint), and none edits its op list in
// place: each fills an EditList (ops to insert before / after an op, ops to drop, a prologue) that one routine
// applies.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <numeric>

#include "ir.h"

namespace lkrt {

namespace {

constexpr size_t kNever = ~size_t(0);
constexpr int64_t kArenaAlign = 256;

bool shapeIsStatic(Type t) {
  for (Dim d : t->shape)
    if (!d->isConst()) return false;
  return true;
}
bool isCopyOf(const Op& op) { return (op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty(); }

// ---- analyses ------------------------------------------------------------------------------------------------------

// origin[v]: the value whose memory v is (through views and syncs); itself for everything else
std::vector<ValueId> originsOf(const std::vector<Op>& ops, size_t nv) {
  std::vector<ValueId> o(nv);
  std::iota(o.begin(), o.end(), ValueId{0});
  for (const Op& op : ops)
    if (isCopyOf(op)) o[op.results[0]] = o[op.operands[0]];
  return o;
}

// calls f(value) for every operand and out of op
template <class F>
void forTouched(const Op& op, F&& f) {
  for (ValueId v : op.operands) f(v);
  for (ValueId v : op.outs) f(v);
}

// last op index touching each origin (kNever: untouched)
std::vector<size_t> lastTouchOf(const std::vector<Op>& ops, const std::vector<ValueId>& origin) {
  std::vector<size_t> last(origin.size(), kNever);
  for (size_t i = 0; i < ops.size(); ++i) forTouched(ops[i], [&](ValueId v) { last[origin[v]] = i; });
  return last;
}

// The part of a buffer-form region that can run once, in init (shared by plan-memory and hoist-init):
//  - memory: constants, static non-output allocs, constant-offset static views of that memory;
//  - kernels: the greatest set of candidates (not `nohoist`, with outs, static results and dim attrs, every out
//    init-able memory) in which each member reads only constant contents (a constant, or init-able memory whose
//    every writer is a member) and writes only memory whose every writer is a member.
struct InitPart {
  std::vector<uint8_t> op;           // per op index
  std::vector<uint8_t> value;        // per value: available in init
  std::vector<uint8_t> initWritten;  // per origin: written by init kernels only
};

InitPart initPart(const Model& m, const Region& r) {
  const size_t nv = m.numValues(), n = r.ops.size();
  const std::vector<ValueId> origin = originsOf(r.ops, nv);
  InitPart part{std::vector<uint8_t>(n, 0), std::vector<uint8_t>(nv, 0), std::vector<uint8_t>(nv, 0)};
  std::vector<uint8_t> constant(nv, 0);
  for (size_t i = 0; i < n; ++i) {
    const Op& op = r.ops[i];
    bool movable = false;
    switch (op.kind) {
      case OpKind::ConstInline:
      case OpKind::ConstInternal:
      case OpKind::ConstExternal:
        movable = true;
        constant[op.results[0]] = 1;
        break;
      case OpKind::BufferAlloc: movable = !op.flag("output") && shapeIsStatic(m.typeOf(op.results[0])); break;
      case OpKind::View:
        movable = part.value[op.operands[0]] && op.dims[0]->isConst() && shapeIsStatic(m.typeOf(op.results[0]));
        break;
      default: break;
    }
    if (movable) {
      part.op[i] = 1;
      part.value[op.results[0]] = 1;
    }
  }
  // candidate kernels
  std::vector<uint8_t> member(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const Op& op = r.ops[i];
    if (op.kind != OpKind::Kernel || op.flag("nohoist") || op.outs.empty()) continue;
    bool ok = true;
    for (const NamedAttr& a : op.attrs)
      if (const Dim* d = std::get_if<Dim>(&a.value)) ok = ok && (*d)->isConst();
    for (ValueId v : op.results) ok = ok && shapeIsStatic(m.typeOf(v));
    for (ValueId v : op.outs) ok = ok && part.value[v];
    member[i] = ok;
  }
  // shrink to the greatest fixpoint (the condition is monotone in the member set, so any removal order ends there)
  std::vector<uint8_t> allWritersIn(nv);
  auto recount = [&] {
    std::vector<uint8_t> written(nv, 0), outsider(nv, 0);
    for (size_t i = 0; i < n; ++i)
      if (r.ops[i].kind == OpKind::Kernel)
        for (ValueId v : r.ops[i].outs) {
          written[origin[v]] = 1;
          if (!member[i]) outsider[origin[v]] = 1;
        }
    for (size_t v = 0; v < nv; ++v) allWritersIn[v] = written[v] && !outsider[v];
  };
  for (bool changed = true; changed;) {
    recount();
    changed = false;
    for (size_t i = 0; i < n; ++i) {
      if (!member[i]) continue;
      const Op& op = r.ops[i];
      bool keep = true;
      for (ValueId v : op.operands) {
        const ValueId o = origin[v];
        keep = keep && (constant[o] || (allWritersIn[o] && part.value[o]));
      }
      for (ValueId v : op.outs) keep = keep && allWritersIn[origin[v]];
      if (!keep) {
        member[i] = 0;
        changed = true;
      }
    }
  }
  recount();
  part.initWritten = allWritersIn;
  for (size_t i = 0; i < n; ++i)
    if (member[i]) {
      part.op[i] = 1;
      for (ValueId v : r.ops[i].results) part.value[v] = 1;
    }
  return part;
}

// ---- edits ---------------------------------------------------------------------------------------------------------
struct EditList {
  explicit EditList(size_t n) : before(n), after(n), drop(n, 0) {}
  std::vector<Op> prologue;
  std::vector<std::vector<Op>> before, after;
  std::vector<uint8_t> drop;
};

void applyEdits(Region& r, EditList& e) {
  std::vector<Op> out;
  for (Op& p : e.prologue) out.push_back(std::move(p));
  for (size_t i = 0; i < r.ops.size(); ++i) {
    for (Op& b : e.before[i]) out.push_back(std::move(b));
    if (!e.drop[i]) out.push_back(std::move(r.ops[i]));
    for (Op& a : e.after[i]) out.push_back(std::move(a));
  }
  r.ops = std::move(out);
}

Op allocOp(ValueId v) {
  Op op;
  op.kind = OpKind::BufferAlloc;
  op.results.push_back(v);
  return op;
}
Op freeOp(ValueId v) {
  Op op;
  op.kind = OpKind::BufferFree;
  op.operands.push_back(v);
  return op;
}

// ---- dce -----------------------------------------------------------------------------------------------------------
Status deadCode(Model& m) {
  Region& r = m.exec;
  std::vector<uint8_t> needed(m.numValues(), 0);
  EditList e(r.ops.size());
  for (size_t i = r.ops.size(); i-- > 0;) {
    const Op& op = r.ops[i];
    const bool effect = op.kind == OpKind::Return || op.kind == OpKind::DimRead ||
                        (op.kind == OpKind::Kernel && (op.attr("inout") || (op.results.empty() && op.outs.empty())));
    bool live = effect;
    for (ValueId v : op.results) live = live || needed[v];
    for (ValueId v : op.outs) live = live || needed[v];
    if (!live) {
      e.drop[i] = 1;
      continue;
    }
    forTouched(op, [&](ValueId v) { needed[v] = 1; });
  }
  applyEdits(r, e);
  return Status();
}

// ---- bufferize -----------------------------------------------------------------------------------------------------
class Bufferizer {
 public:
  Bufferizer(Model& m, Region& r, bool isExec, const std::vector<uint8_t>& wasTensor)
      : m_(m), r_(r), exec_(isExec), wasTensor_(wasTensor), nv_(m.numValues()) {}

  Status run() {
    EditList e(r_.ops.size());
    LKRT_TRY(assignStorage(e));
    return placeFrees(e);
  }

 private:
  // Every tensor result of a kernel becomes an out: a fresh alloc just before the kernel, or the operand an
  // `inplace` pair names when that operand is an alloc of this region, used once by the kernel and dead after it.
  Status assignStorage(EditList& e) {
    const std::vector<ValueId> origin = originsOf(r_.ops, nv_);
    std::vector<uint8_t> ownsMemory(nv_, 0);  // allocs, and tensor kernel results (future allocs)
    persistent_.assign(nv_, 0);
    for (const Op& op : r_.ops) {
      if (op.kind == OpKind::BufferAlloc) {
        ownsMemory[op.results[0]] = 1;
        if (op.flag("persistent")) persistent_[op.results[0]] = 1;
      }
      if (op.kind == OpKind::Kernel)
        for (ValueId v : op.results)
          if (wasTensor_[v]) ownsMemory[v] = 1;
    }
    std::vector<size_t> dies = lastTouchOf(r_.ops, origin);
    std::vector<ValueId> alias(nv_);  // a result renamed to the operand it reuses
    std::iota(alias.begin(), alias.end(), ValueId{0});
    fresh_.assign(nv_, 0);
    for (size_t i = 0; i < r_.ops.size(); ++i) {
      Op& op = r_.ops[i];
      for (ValueId& v : op.operands) v = alias[v];
      for (ValueId& v : op.outs) v = alias[v];
      if (op.kind != OpKind::Kernel) continue;
      std::vector<std::pair<size_t, size_t>> pairs;  // (result k, operand j)
      if (const AttrValue* a = op.attr("inplace")) {
        const Ints* list = std::get_if<Ints>(a);
        if (!list) return Status::error("bufferize: inplace must be an int list");
        for (size_t q = 0; q + 1 < list->size(); q += 2)
          pairs.emplace_back(static_cast<size_t>((*list)[q]), static_cast<size_t>((*list)[q + 1]));
      }
      std::vector<ValueId> keptResults, taken;
      for (size_t k = 0; k < op.results.size(); ++k) {
        const ValueId res = op.results[k];
        if (!wasTensor_[res]) {
          keptResults.push_back(res);
          continue;
        }
        ValueId reuse = kNoValue;
        for (auto [outK, inJ] : pairs) {
          if (outK != k || inJ >= op.operands.size()) continue;
          const ValueId in = op.operands[inJ];
          const ValueId o = origin[in];
          const bool dying = ownsMemory[o] && o == in && !persistent_[o] && dies[o] == i;
          if (!dying || std::count(taken.begin(), taken.end(), o) || m_.typeOf(in) != m_.typeOf(res)) continue;
          const auto once = std::count_if(op.operands.begin(), op.operands.end(), [&](ValueId x) { return origin[x] == o; });
          if (once != 1) continue;
          reuse = in;
          break;
        }
        if (reuse != kNoValue) {
          alias[res] = reuse;
          if (dies[res] != kNever) dies[origin[reuse]] = dies[res];  // the buffer now lives as long as the result
          taken.push_back(origin[reuse]);
          op.outs.push_back(reuse);
        } else {
          e.before[i].push_back(allocOp(res));
          fresh_[res] = 1;
          op.outs.push_back(res);
        }
      }
      op.results = keptResults;
    }
    return Status();
  }

  // Frees after last uses, and the output / gpu_only marks, from the rewritten ops.
  Status placeFrees(EditList& e) {
    const std::vector<Op>& ops = r_.ops;
    const size_t n = ops.size();
    const std::vector<ValueId> origin = originsOf(ops, nv_);
    const std::vector<size_t> last = lastTouchOf(ops, origin);
    std::vector<uint8_t> isAlloc(fresh_), returned(nv_, 0);
    for (const Op& op : ops)
      if (op.kind == OpKind::BufferAlloc) isAlloc[op.results[0]] = 1;
    for (ValueId v : ops.back().operands) {
      returned[origin[v]] = 1;
      if (exec_ && persistent_[origin[v]])
        return Status::error("exec returns persistent state %" + std::to_string(v) +
                             " (or a view of it); persistent buffers can't be graph outputs: return a copy");
    }
    // device touches: the last GPU kernel use; any host use (CPU kernel, dim.read, return)
    std::vector<size_t> lastGpu(nv_, kNever);
    std::vector<uint8_t> host(nv_, 0);
    for (size_t i = 0; i < n; ++i) {
      const Op& op = ops[i];
      const bool gpu = op.kind == OpKind::Kernel && isGpuKernelName(op.name);
      const bool cpu = !gpu && (op.kind == OpKind::Kernel || op.kind == OpKind::DimRead || op.kind == OpKind::Return);
      if (gpu) forTouched(op, [&](ValueId v) { lastGpu[origin[v]] = i; });
      if (cpu) forTouched(op, [&](ValueId v) { host[origin[v]] = 1; });
    }
    // first gpu_to_cpu sync at or after each index (the return when none)
    std::vector<size_t> syncFrom(n + 1, n - 1);
    for (size_t i = n; i-- > 0;)
      syncFrom[i] = ops[i].kind == OpKind::Sync && ops[i].ints[0] == kGpuToCpu ? i : syncFrom[i + 1];
    // A buffer both devices touch is freed no earlier than the first gpu_to_cpu sync after its last GPU use (the
    // op before the return when there is none): until then the GPU may still read it.
    std::vector<std::pair<size_t, ValueId>> frees;
    for (ValueId v = 0; v < nv_; ++v) {
      if (!isAlloc[v] || origin[v] != v || returned[v] || persistent_[v] || last[v] == kNever) continue;
      size_t at = last[v];
      if (lastGpu[v] != kNever && host[v]) {
        const size_t s = syncFrom[lastGpu[v]];
        at = std::max(at, s >= n - 1 ? n - 2 : s);
      }
      frees.emplace_back(at, v);
    }
    std::sort(frees.begin(), frees.end());
    for (auto [at, v] : frees) e.after[at].push_back(freeOp(v));
    auto mark = [&](Op& alloc) {
      const ValueId v = alloc.results[0];
      if (exec_ && returned[v]) alloc.setAttr("output", true);
      if (lastGpu[v] != kNever && !host[v] && !persistent_[v]) alloc.setAttr("gpu_only", true);
    };
    for (auto& list : e.before)
      for (Op& a : list) mark(a);
    for (Op& op : r_.ops)
      if (op.kind == OpKind::BufferAlloc) mark(op);
    applyEdits(r_, e);
    return Status();
  }

  Model& m_;
  Region& r_;
  bool exec_;
  const std::vector<uint8_t>& wasTensor_;
  size_t nv_;
  std::vector<uint8_t> persistent_, fresh_;
};

Status bufferize(Model& m) {
  std::vector<uint8_t> wasTensor(m.numValues(), 0);
  for (ValueId v = 0; v < m.numValues(); ++v)
    if (const Type t = m.typeOf(v); t->isTensor()) {
      wasTensor[v] = 1;
      m.setType(v, m.types().withKind(t, TypeKind::Buffer));
    }
  LKRT_TRY(Bufferizer(m, m.init, false, wasTensor).run());
  return Bufferizer(m, m.exec, true, wasTensor).run();
}

// ---- plan-memory ---------------------------------------------------------------------------------------------------
Status planMemory(Model& m) {
  Region& r = m.exec;
  DimPool& dims = m.dims();
  const InitPart init = initPart(m, r);
  const size_t n = r.ops.size();
  // where each dim.read symbol is defined, and where each buffer is freed
  std::vector<int64_t> definedAt(dims.numSymbols(), -1);
  bool reads = false;
  std::vector<size_t> freedAt(m.numValues(), kNever);
  for (size_t i = 0; i < n; ++i) {
    const Op& op = r.ops[i];
    if (op.kind == OpKind::DimRead) {
      definedAt[static_cast<size_t>(op.symbols[0])] = static_cast<int64_t>(i);
      reads = true;
    }
    if (op.kind == OpKind::BufferFree) freedAt[op.operands[0]] = i;
  }
  // candidates: per-call allocs with a free (not outputs, not arenas, not written by init)
  struct Slot {
    size_t alloc, free;
    ValueId v;
    Dim bytes;
  };
  // (the dim.read after which the sizes are known, or -1; gpu_only) -> slots, in op order
  std::map<std::pair<int64_t, bool>, std::vector<Slot>> pools;
  for (size_t i = 0; i < n; ++i) {
    const Op& op = r.ops[i];
    if (op.kind != OpKind::BufferAlloc) continue;
    const ValueId v = op.results[0];
    if (init.initWritten[v] || freedAt[v] == kNever || op.flag("output") || op.flag("arena")) continue;
    const Dim bytes = m.types().numBytes(m.typeOf(v));
    int64_t after = -1;
    if (reads && !bytes->isConst()) {
      std::vector<int64_t> syms;
      collectSymbols(bytes, syms);
      for (int64_t s : syms) after = std::max(after, definedAt[static_cast<size_t>(s)]);
    }
    pools[{after, op.flag("gpu_only")}].push_back({i, freedAt[v], v, bytes});
  }
  if (pools.empty()) return Status();

  EditList e(n);
  auto elemSize = [&](ValueId v) { return static_cast<int64_t>(dtypeSize(m.typeOf(v)->dtype)); };
  int planNo = 0;
  for (auto& [key, slots] : pools) {
    const int64_t after = key.first;
    const bool sizesKnown = std::all_of(slots.begin(), slots.end(), [](const Slot& s) { return s.bytes->isConst(); });
    Op arenaOp;
    ValueId arena;
    std::vector<Dim> where;  // each slot's offset in its own elements
    if (sizesKnown && after < 0) {
      std::vector<PlanItem> items;
      for (const Slot& s : slots)
        items.push_back({s.bytes->value, static_cast<int64_t>(s.alloc), static_cast<int64_t>(s.free)});
      std::vector<int64_t> byteOff;
      const int64_t total = planOffsets(items, kArenaAlign, byteOff);
      arena = m.newValue(m.types().buffer(DType::U8, {dims.constant(total)}), "arena");
      arenaOp = allocOp(arena);
      arenaOp.setAttr("arena", true);
      for (size_t k = 0; k < slots.size(); ++k) where.push_back(dims.constant(byteOff[k] / elemSize(slots[k].v)));
    } else {
      while (dims.findSymbol("M" + std::to_string(planNo) + "_size") >= 0) ++planNo;
      const std::string base = "M" + std::to_string(planNo++);
      arenaOp.kind = OpKind::MemPlan;
      const Dim size = dims.sym(base + "_size");
      arenaOp.symbols.push_back(size->value);
      Ints elem;
      for (size_t k = 0; k < slots.size(); ++k) {
        const Dim off = dims.sym(base + "_o" + std::to_string(k));
        arenaOp.dims.push_back(slots[k].bytes);
        arenaOp.ints.push_back(static_cast<int64_t>(slots[k].alloc));
        arenaOp.ints.push_back(static_cast<int64_t>(slots[k].free));
        arenaOp.symbols.push_back(off->value);
        elem.push_back(elemSize(slots[k].v));
        where.push_back(off);
      }
      arenaOp.ints.push_back(kArenaAlign);
      arenaOp.setAttr("elem", elem);
      if (key.second) arenaOp.setAttr("gpu_only", true);
      arena = m.newValue(m.types().buffer(DType::U8, {size}), "arena");
      arenaOp.results.push_back(arena);
    }
    for (size_t k = 0; k < slots.size(); ++k) {  // the alloc becomes a view of the arena (same result value)
      Op& op = r.ops[slots[k].alloc];
      op.kind = OpKind::View;
      op.attrs.clear();
      op.operands = {arena};
      op.dims = {where[k]};
      e.drop[slots[k].free] = 1;
    }
    if (after < 0) e.prologue.push_back(std::move(arenaOp));
    else e.after[static_cast<size_t>(after)].push_back(std::move(arenaOp));
  }
  applyEdits(r, e);
  return Status();
}

// ---- hoist-init ----------------------------------------------------------------------------------------------------
Status hoistInit(Model& m) {
  Region& ex = m.exec;
  const InitPart part = initPart(m, ex);
  const size_t n = ex.ops.size();
  std::vector<uint8_t> execUses(m.numValues(), 0);  // touched by an op that stays per call
  for (size_t i = 0; i < n; ++i)
    if (!part.op[i] && ex.ops[i].kind != OpKind::BufferFree) forTouched(ex.ops[i], [&](ValueId v) { execUses[v] = 1; });
  Op initRet = std::move(m.init.ops.back());
  m.init.ops.pop_back();
  EditList stays(n);
  for (size_t i = 0; i < n; ++i) {
    Op& op = ex.ops[i];
    const bool freesInitMemory = op.kind == OpKind::BufferFree && part.value[op.operands[0]];
    if (part.op[i]) {
      m.init.ops.push_back(std::move(op));
      stays.drop[i] = 1;
    } else if (freesInitMemory) {
      // an init-only temporary is freed in init; memory exec still uses lives as long as the model
      if (!execUses[op.operands[0]]) m.init.ops.push_back(std::move(op));
      stays.drop[i] = 1;
    }
  }
  applyEdits(ex, stays);
  // init values exec still refers to become state, in order of first reference
  std::vector<ValueId> asState(m.numValues(), kNoValue);
  auto stateFor = [&](ValueId& v) {
    if (v >= part.value.size() || !part.value[v]) return;
    if (asState[v] == kNoValue) {
      asState[v] = m.newValue(m.typeOf(v), m.nameOf(v));
      initRet.operands.push_back(v);
      ex.state.push_back(asState[v]);
    }
    v = asState[v];
  };
  for (Op& op : ex.ops) {
    for (ValueId& v : op.operands) stateFor(v);
    for (ValueId& v : op.outs) stateFor(v);
  }
  m.init.ops.push_back(std::move(initRet));
  return Status();
}

// ---- pass table ----------------------------------------------------------------------------------------------------
struct PassEntry {
  const char* name;
  Status (*run)(Model&);
};
const PassEntry kPasses[] = {
    {"dce", deadCode}, {"bufferize", bufferize}, {"plan-memory", planMemory}, {"hoist-init", hoistInit}};

}  // namespace

// Greedy by size (largest first, ties by index); each buffer goes to the smallest gap between the placed buffers
// whose [start, end] lifetimes overlap its own that holds it, else past all of them.
int64_t planOffsets(const std::vector<PlanItem>& items, int64_t align, std::vector<int64_t>& offsets) {
  offsets.assign(items.size(), 0);
  std::vector<size_t> order(items.size());
  std::iota(order.begin(), order.end(), size_t{0});
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return items[a].bytes > items[b].bytes; });
  struct Span {
    int64_t lo, hi;  // [lo, hi) bytes
    size_t item;
  };
  std::vector<Span> spans;  // by lo
  int64_t total = 0;
  for (size_t i : order) {
    const PlanItem& it = items[i];
    const int64_t size = (std::max<int64_t>(it.bytes, 1) + align - 1) / align * align;
    int64_t at = -1, tightest = INT64_MAX, frontier = 0;
    for (const Span& s : spans) {
      const PlanItem& other = items[s.item];
      if (other.end < it.start || it.end < other.start) continue;  // never live together
      if (s.lo >= frontier && s.lo - frontier >= size && s.lo - frontier < tightest) {
        at = frontier;
        tightest = s.lo - frontier;
      }
      frontier = std::max(frontier, s.hi);
    }
    if (at < 0) at = frontier;
    offsets[i] = at;
    total = std::max(total, at + size);
    const Span mine{at, at + size, i};
    spans.insert(std::upper_bound(spans.begin(), spans.end(), mine, [](const Span& a, const Span& b) { return a.lo < b.lo; }),
                 mine);
  }
  return total;
}

const std::vector<std::string>& defaultPipeline() {
  static const std::vector<std::string> p = {"dce", "bufferize", "plan-memory", "hoist-init"};
  return p;
}

Status runPass(Model& m, std::string_view name) {
  const PassEntry* pass = nullptr;
  for (const PassEntry& p : kPasses)
    if (name == p.name) pass = &p;
  if (!pass) return Status::error("unknown pass '" + std::string(name) + "'");
  if (Status s = pass->run(m); !s) return Status::error(std::string(name) + ": " + s.message());
  if (Status v = verifyModel(m); !v) return Status::error("IR invalid after pass '" + std::string(name) + "': " + v.message());
  return Status();
}

// const.external -> const.internal for every external whose bytes are given; with `copy` the model keeps its own
// page-aligned copy, else it refers to the caller's bytes (kept alive through `owner`).
Status internalize(Model& m, const std::vector<ExternalBytes>& data, bool copy) {
  auto bytesFor = [&](const std::string& name) -> const ExternalBytes* {
    for (const ExternalBytes& e : data)
      if (e.name == name) return &e;
    return nullptr;
  };
  for (Region* r : {&m.init, &m.exec})
    for (Op& op : r->ops) {
      if (op.kind != OpKind::ConstExternal) continue;
      const ExternalBytes* d = bytesFor(op.name);
      if (!d) return Status::error("internalize: no data for external constant '" + op.name + "'");
      if (!m.findConstant(op.name)) {
        const Type t = m.typeOf(op.results[0]);
        size_t need = dtypeSize(t->dtype);
        for (Dim dim : t->shape) {
          if (!dim->isConst() || dim->value < 0)
            return Status::error("internalize: external constant '" + op.name + "' has a symbolic shape");
          need *= static_cast<size_t>(dim->value);
        }
        if (d->size != need)
          return Status::error("internalize: '" + op.name + "' has " + std::to_string(d->size) + " bytes, its type " +
                               std::to_string(need));
        Constant c{op.name, t, d->owner, d->bytes, need};
        if (copy) {
          constexpr size_t kPage = 16384;
          const size_t cap = (std::max<size_t>(need, 1) + kPage - 1) / kPage * kPage;
          void* mem = std::aligned_alloc(kPage, cap);
          if (!mem) return Status::error("internalize: out of memory");
          if (need) std::memcpy(mem, d->bytes, need);
          c.owner = std::shared_ptr<const void>(mem, [](const void* q) { std::free(const_cast<void*>(q)); });
          c.bytes = static_cast<const uint8_t*>(mem);
        }
        m.addConstant(std::move(c));
      }
      op.kind = OpKind::ConstInternal;
    }
  return Status();
}

}  // namespace lkrt
