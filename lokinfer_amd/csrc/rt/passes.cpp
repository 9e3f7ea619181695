// Compiler passes over the runtime IR: dce, bufferize, plan-memory, hoist-init (the reference's default pipeline,
// in that order) and internalize. Their contracts are the reference's (lariaus/lokinfer src/compiler/*.cpp,
// docs/impl-notes/design-compiler-passes.md), so a model compiled here prints and saves as the reference's
// compiler would write it:
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
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <numeric>

#include "ir.h"

namespace lkrt {

namespace {

constexpr size_t kNone = ~size_t(0);
constexpr int64_t kArenaAlign = 256;

bool staticType(Type t) {
  return std::all_of(t->shape.begin(), t->shape.end(), [](Dim d) { return d->isConst(); });
}

// view / sync result -> the value whose memory it is
struct Roots {
  std::vector<ValueId> up;
  explicit Roots(size_t n) : up(n, kNoValue) {}
  ValueId of(ValueId v) const { return up[v] == kNoValue ? v : up[v]; }
  void scan(const std::vector<Op>& ops) {
    for (const Op& op : ops)
      if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
        up[op.results[0]] = of(op.operands[0]);
  }
};

// Which ops of a buffer-form region can run once, in init:
//  - memory: constants, static non-output allocs, constant-offset static views of those;
//  - kernels (fixpoint): not `nohoist`, with outs, static results and dim attrs, every operand's contents constant
//    (a constant, or a buffer all of whose writers are hoisted) and every out hoistable memory no per-call kernel
//    writes.
struct Hoist {
  std::vector<uint8_t> op, value, initWritten;
};

Hoist hoistable(const Model& m, const Region& r) {
  const size_t nv = m.numValues(), no = r.ops.size();
  Roots roots(nv);
  roots.scan(r.ops);
  Hoist h{std::vector<uint8_t>(no, 0), std::vector<uint8_t>(nv, 0), std::vector<uint8_t>(nv, 0)};
  std::vector<uint8_t> isConst(nv, 0);
  for (size_t i = 0; i < no; ++i) {
    const Op& op = r.ops[i];
    bool ok = false;
    if (op.kind == OpKind::ConstInline || op.kind == OpKind::ConstInternal || op.kind == OpKind::ConstExternal) {
      ok = true;
      isConst[op.results[0]] = 1;
    } else if (op.kind == OpKind::BufferAlloc) {
      ok = !op.flag("output") && staticType(m.typeOf(op.results[0]));
    } else if (op.kind == OpKind::View) {
      ok = h.value[op.operands[0]] && op.dims[0]->isConst() && staticType(m.typeOf(op.results[0]));
    }
    h.op[i] = ok;
    if (ok) h.value[op.results[0]] = 1;
  }
  std::vector<uint8_t> cand(no, 0);
  for (size_t i = 0; i < no; ++i) {
    const Op& op = r.ops[i];
    if (op.kind != OpKind::Kernel) continue;
    bool ok = !op.flag("nohoist") && !op.outs.empty();
    for (const NamedAttr& a : op.attrs)
      if (a.value.index() == 6) ok = ok && std::get<Dim>(a.value)->isConst();
    for (ValueId v : op.results) ok = ok && staticType(m.typeOf(v));
    for (ValueId v : op.outs) ok = ok && h.value[v];
    cand[i] = ok;
  }
  std::vector<int8_t> writersOk(nv);  // per root: -1 unwritten, 0 a writer stays per-call, 1 all writers hoisted
  while (true) {
    std::fill(writersOk.begin(), writersOk.end(), int8_t(-1));
    for (size_t i = 0; i < no; ++i) {
      if (r.ops[i].kind != OpKind::Kernel) continue;
      for (ValueId v : r.ops[i].outs) {
        int8_t& w = writersOk[roots.of(v)];
        w = (w != 0 && cand[i]) ? 1 : 0;
      }
    }
    auto constContents = [&](ValueId v) {
      const ValueId root = roots.of(v);
      return isConst[root] || (writersOk[root] == 1 && h.value[root]);
    };
    bool changed = false;
    for (size_t i = 0; i < no; ++i) {
      if (!cand[i]) continue;
      const Op& op = r.ops[i];
      bool ok = std::all_of(op.operands.begin(), op.operands.end(), constContents);
      for (ValueId v : op.outs) ok = ok && writersOk[roots.of(v)] == 1;
      if (!ok) {
        cand[i] = 0;
        changed = true;
        for (ValueId v : op.outs) writersOk[roots.of(v)] = 0;
      }
    }
    if (!changed) break;
  }
  for (size_t v = 0; v < nv; ++v) h.initWritten[v] = writersOk[v] == 1;
  for (size_t i = 0; i < no; ++i)
    if (cand[i]) {
      h.op[i] = 1;
      for (ValueId v : r.ops[i].results) h.value[v] = 1;
    }
  return h;
}

// ---- dce -------------------------------------------------------------------------------------------------------
Status dce(Model& m) {
  Region& r = m.exec;
  std::vector<uint8_t> live(m.numValues(), 0);
  std::vector<uint8_t> keep(r.ops.size(), 0);
  for (size_t i = r.ops.size(); i-- > 0;) {
    const Op& op = r.ops[i];
    bool k = op.kind == OpKind::Return || op.kind == OpKind::DimRead ||
             (op.kind == OpKind::Kernel && (op.attr("inout") || (op.results.empty() && op.outs.empty())));
    for (ValueId v : op.results) k = k || live[v];
    for (ValueId v : op.outs) k = k || live[v];
    if (!k) continue;
    keep[i] = 1;
    for (ValueId v : op.operands) live[v] = 1;
    for (ValueId v : op.outs) live[v] = 1;
  }
  std::vector<Op> out;
  for (size_t i = 0; i < r.ops.size(); ++i)
    if (keep[i]) out.push_back(std::move(r.ops[i]));
  r.ops = std::move(out);
  return Status();
}

// ---- bufferize -------------------------------------------------------------------------------------------------
Status bufferizeRegion(Model& m, Region& r, bool exec, const std::vector<uint8_t>& wasTensor) {
  const size_t nv = m.numValues();
  // Liveness before rewriting: a tensor kernel result is its own (future alloc) root.
  Roots pre(nv);
  pre.scan(r.ops);
  std::vector<uint8_t> allocRoot(nv, 0);
  for (const Op& op : r.ops) {
    if (op.kind == OpKind::BufferAlloc) allocRoot[op.results[0]] = 1;
    if (op.kind == OpKind::Kernel)
      for (ValueId v : op.results)
        if (wasTensor[v]) allocRoot[v] = 1;
  }
  auto lastUse = [&](const std::vector<Op>& ops, const Roots& roots) {
    std::vector<size_t> last(nv, kNone);
    for (size_t i = 0; i < ops.size(); ++i) {
      for (ValueId v : ops[i].operands) last[roots.of(v)] = i;
      for (ValueId v : ops[i].outs) last[roots.of(v)] = i;
    }
    return last;
  };
  std::vector<size_t> preLast = lastUse(r.ops, pre);
  std::vector<uint8_t> persistent(nv, 0);
  for (const Op& op : r.ops)
    if (op.kind == OpKind::BufferAlloc && op.flag("persistent")) persistent[op.results[0]] = 1;

  std::vector<ValueId> renamed(nv, kNoValue);
  auto ren = [&](ValueId v) { return renamed[v] == kNoValue ? v : renamed[v]; };
  std::vector<std::pair<size_t, ValueId>> newAllocs;  // (before op index, value)
  for (size_t i = 0; i < r.ops.size(); ++i) {
    Op& op = r.ops[i];
    for (ValueId& v : op.operands) v = ren(v);
    for (ValueId& v : op.outs) v = ren(v);
    if (op.kind != OpKind::Kernel) continue;
    std::vector<std::pair<size_t, size_t>> inplace;  // (result k, operand j)
    if (const AttrValue* a = op.attr("inplace")) {
      const Ints* v = std::get_if<Ints>(a);
      if (!v) return Status::error("bufferize: inplace must be an int list");
      for (size_t k = 0; k + 1 < v->size(); k += 2)
        inplace.emplace_back(static_cast<size_t>((*v)[k]), static_cast<size_t>((*v)[k + 1]));
    }
    std::vector<ValueId> reusedHere;
    std::vector<ValueId> scalarResults;
    for (size_t k = 0; k < op.results.size(); ++k) {
      const ValueId res = op.results[k];
      if (!wasTensor[res]) {
        scalarResults.push_back(res);
        continue;
      }
      bool reused = false;
      for (auto [outK, inJ] : inplace) {
        if (outK != k || inJ >= op.operands.size()) continue;
        const ValueId in = op.operands[inJ];
        const ValueId inRoot = pre.of(in);
        // the operand must be an in-region alloc root that dies at this kernel, used once by it
        if (!allocRoot[inRoot] || inRoot != in || persistent[inRoot] || preLast[inRoot] != i) continue;
        if (std::find(reusedHere.begin(), reusedHere.end(), inRoot) != reusedHere.end()) continue;
        if (m.typeOf(in) != m.typeOf(res)) continue;
        size_t uses = 0;
        for (ValueId o : op.operands) uses += pre.of(o) == inRoot;
        if (uses != 1) continue;
        renamed[res] = in;
        if (preLast[res] != kNone) preLast[inRoot] = preLast[res];  // the buffer now lives as long as the result
        reusedHere.push_back(inRoot);
        op.outs.push_back(in);
        reused = true;
        break;
      }
      if (reused) continue;
      newAllocs.emplace_back(i, res);
      op.outs.push_back(res);
    }
    op.results = scalarResults;
  }
  std::vector<Op>& ops = r.ops;

  Roots post(nv);
  post.scan(ops);
  std::vector<uint8_t> postAlloc(nv, 0);
  for (const Op& op : ops)
    if (op.kind == OpKind::BufferAlloc) postAlloc[op.results[0]] = 1;
  for (const auto& a : newAllocs) postAlloc[a.second] = 1;
  const std::vector<size_t> last = lastUse(ops, post);
  std::vector<uint8_t> returned(nv, 0);
  for (ValueId v : ops.back().operands) returned[post.of(v)] = 1;
  if (exec)
    for (ValueId v : ops.back().operands)
      if (persistent[post.of(v)])
        return Status::error("exec returns persistent state %" + std::to_string(v) +
                             " (or a view of it); persistent buffers can't be graph outputs: return a copy");
  // A buffer both a GPU kernel and a CPU op touch is freed no earlier than the next gpu_to_cpu sync after its last
  // GPU use (else the end of the region): until then the GPU may still read it.
  std::vector<size_t> lastGpu(nv, kNone);
  std::vector<uint8_t> cpuTouched(nv, 0);
  for (size_t i = 0; i < ops.size(); ++i) {
    const Op& o = ops[i];
    if (o.kind == OpKind::Kernel && isGpuKernelName(o.name)) {
      for (ValueId v : o.operands) lastGpu[post.of(v)] = i;
      for (ValueId v : o.outs) lastGpu[post.of(v)] = i;
    } else if (o.kind == OpKind::Kernel || o.kind == OpKind::DimRead || o.kind == OpKind::Return) {
      for (ValueId v : o.operands) cpuTouched[post.of(v)] = 1;
      for (ValueId v : o.outs) cpuTouched[post.of(v)] = 1;
    }
  }
  std::vector<size_t> nextSync(ops.size() + 1, ops.size() - 1);
  for (size_t i = ops.size(); i-- > 0;) {
    nextSync[i] = nextSync[i + 1];
    if (ops[i].kind == OpKind::Sync && ops[i].ints[0] == kGpuToCpu) nextSync[i] = i;
  }
  std::vector<std::pair<size_t, ValueId>> frees;
  for (ValueId root = 0; root < nv; ++root) {
    if (!postAlloc[root] || post.of(root) != root || returned[root] || persistent[root] || last[root] == kNone)
      continue;
    size_t at = last[root];
    if (lastGpu[root] != kNone && cpuTouched[root]) {
      const size_t s = nextSync[lastGpu[root]];
      at = std::max(at, s >= ops.size() - 1 ? ops.size() - 2 : s);
    }
    frees.emplace_back(at, root);
  }
  std::sort(frees.begin(), frees.end());
  auto mark = [&](Op& alloc) {
    const ValueId v = alloc.results[0];
    if (exec && returned[v]) alloc.setAttr("output", true);
    if (lastGpu[v] != kNone && !cpuTouched[v] && !persistent[v]) alloc.setAttr("gpu_only", true);
  };
  std::vector<Op> out;
  out.reserve(ops.size() + newAllocs.size() + frees.size());
  size_t f = 0, a = 0;
  for (size_t i = 0; i < ops.size(); ++i) {
    for (; a < newAllocs.size() && newAllocs[a].first == i; ++a) {
      Op alloc;
      alloc.kind = OpKind::BufferAlloc;
      alloc.results.push_back(newAllocs[a].second);
      mark(alloc);
      out.push_back(std::move(alloc));
    }
    if (ops[i].kind == OpKind::BufferAlloc) mark(ops[i]);
    out.push_back(std::move(ops[i]));
    for (; f < frees.size() && frees[f].first == i; ++f) {
      Op fr;
      fr.kind = OpKind::BufferFree;
      fr.operands.push_back(frees[f].second);
      out.push_back(std::move(fr));
    }
  }
  r.ops = std::move(out);
  return Status();
}

Status bufferize(Model& m) {
  std::vector<uint8_t> wasTensor(m.numValues(), 0);
  for (ValueId v = 0; v < m.numValues(); ++v) {
    Type t = m.typeOf(v);
    if (t->isTensor()) {
      wasTensor[v] = 1;
      m.setType(v, m.types().withKind(t, TypeKind::Buffer));
    }
  }
  LKRT_TRY(bufferizeRegion(m, m.init, false, wasTensor));
  return bufferizeRegion(m, m.exec, true, wasTensor);
}

// ---- plan-memory -----------------------------------------------------------------------------------------------
Status planMemory(Model& m) {
  Region& r = m.exec;
  const Hoist hoist = hoistable(m, r);
  DimPool& dp = m.dims();
  std::vector<int64_t> readAt(dp.numSymbols(), -1);  // symbol -> index of the dim.read defining it
  bool anyRead = false;
  for (size_t i = 0; i < r.ops.size(); ++i)
    if (r.ops[i].kind == OpKind::DimRead) {
      readAt[static_cast<size_t>(r.ops[i].symbols[0])] = static_cast<int64_t>(i);
      anyRead = true;
    }
  std::vector<size_t> freeAt(m.numValues(), kNone);
  for (size_t i = 0; i < r.ops.size(); ++i)
    if (r.ops[i].kind == OpKind::BufferFree) freeAt[r.ops[i].operands[0]] = i;

  struct Cand {
    size_t alloc, free;
    ValueId v;
    Dim bytes;
    int64_t group;
    bool gpuOnly;
  };
  std::vector<Cand> cands;
  std::unordered_map<Type, Dim> bytesOf;
  for (size_t i = 0; i < r.ops.size(); ++i) {
    const Op& op = r.ops[i];
    if (op.kind != OpKind::BufferAlloc) continue;
    const ValueId v = op.results[0];
    if (hoist.initWritten[v] || freeAt[v] == kNone || op.flag("output") || op.flag("arena")) continue;
    Type t = m.typeOf(v);
    auto it = bytesOf.find(t);
    Dim bytes = it != bytesOf.end() ? it->second : (bytesOf[t] = m.types().numBytes(t));
    Cand c{i, freeAt[v], v, bytes, -1, op.flag("gpu_only")};
    if (anyRead && !bytes->isConst()) {
      std::vector<int64_t> syms;
      collectSymbols(bytes, syms);
      for (int64_t s : syms)
        if (readAt[static_cast<size_t>(s)] >= 0) c.group = std::max(c.group, readAt[static_cast<size_t>(s)]);
    }
    cands.push_back(c);
  }
  if (cands.empty()) return Status();
  std::map<std::pair<int64_t, bool>, std::vector<size_t>> groups;
  for (size_t i = 0; i < cands.size(); ++i) groups[{cands[i].group, cands[i].gpuOnly}].push_back(i);

  std::vector<uint8_t> drop(r.ops.size(), 0);
  std::vector<Op> prologue;
  std::vector<std::pair<size_t, Op>> after;
  auto elemBytes = [&](ValueId v) { return static_cast<int64_t>(dtypeSize(m.typeOf(v)->dtype)); };
  int planNo = 0;
  for (auto& [key, idx] : groups) {
    const int64_t group = key.first;
    const bool allStatic = std::all_of(idx.begin(), idx.end(), [&](size_t i) { return cands[i].bytes->isConst(); });
    Op plan;
    ValueId arena;
    std::vector<Dim> offsets;
    if (allStatic && group < 0) {
      std::vector<PlanItem> items;
      for (size_t i : idx)
        items.push_back({cands[i].bytes->value, static_cast<int64_t>(cands[i].alloc), static_cast<int64_t>(cands[i].free)});
      std::vector<int64_t> offs;
      const int64_t total = planOffsets(items, kArenaAlign, offs);
      arena = m.newValue(m.types().buffer(DType::U8, {dp.constant(total)}), "arena");
      plan.kind = OpKind::BufferAlloc;
      plan.setAttr("arena", true);
      plan.results.push_back(arena);
      for (size_t k = 0; k < idx.size(); ++k) offsets.push_back(dp.constant(offs[k] / elemBytes(cands[idx[k]].v)));
    } else {
      while (dp.findSymbol("M" + std::to_string(planNo) + "_size") >= 0) ++planNo;
      const std::string base = "M" + std::to_string(planNo++);
      plan.kind = OpKind::MemPlan;
      plan.symbols.push_back(dp.sym(base + "_size")->value);
      Ints elems;
      for (size_t k = 0; k < idx.size(); ++k) {
        const Cand& c = cands[idx[k]];
        Dim off = dp.sym(base + "_o" + std::to_string(k));  // in elements of buffer k (attr `elem`)
        plan.dims.push_back(c.bytes);
        plan.ints.push_back(static_cast<int64_t>(c.alloc));
        plan.ints.push_back(static_cast<int64_t>(c.free));
        plan.symbols.push_back(off->value);
        elems.push_back(elemBytes(c.v));
        offsets.push_back(off);
      }
      plan.ints.push_back(kArenaAlign);
      plan.setAttr("elem", elems);
      if (key.second) plan.setAttr("gpu_only", true);
      arena = m.newValue(m.types().buffer(DType::U8, {dp.sym(base + "_size")}), "arena");
      plan.results.push_back(arena);
    }
    for (size_t k = 0; k < idx.size(); ++k) {
      const Cand& c = cands[idx[k]];
      Op& view = r.ops[c.alloc];  // the alloc becomes a view of the arena, same result
      view.kind = OpKind::View;
      view.attrs.clear();
      view.operands.assign(1, arena);
      view.dims.assign(1, offsets[k]);
      drop[c.free] = 1;
    }
    if (group < 0) prologue.push_back(std::move(plan));
    else after.emplace_back(static_cast<size_t>(group), std::move(plan));
  }
  std::stable_sort(after.begin(), after.end(), [](const auto& a, const auto& b) { return a.first < b.first; });
  std::vector<Op> out;
  out.reserve(r.ops.size() + prologue.size() + after.size());
  for (Op& p : prologue) out.push_back(std::move(p));
  size_t a = 0;
  for (size_t i = 0; i < r.ops.size(); ++i) {
    if (!drop[i]) out.push_back(std::move(r.ops[i]));
    for (; a < after.size() && after[a].first == i; ++a) out.push_back(std::move(after[a].second));
  }
  r.ops = std::move(out);
  return Status();
}

// ---- hoist-init ------------------------------------------------------------------------------------------------
Status hoistInit(Model& m) {
  Region& ex = m.exec;
  const Hoist h = hoistable(m, ex);
  std::vector<uint8_t> usedByExec(m.numValues(), 0);
  for (size_t i = 0; i < ex.ops.size(); ++i) {
    const Op& op = ex.ops[i];
    if (h.op[i] || op.kind == OpKind::BufferFree) continue;
    for (ValueId v : op.operands) usedByExec[v] = 1;
    for (ValueId v : op.outs) usedByExec[v] = 1;
  }
  Op initReturn = std::move(m.init.ops.back());
  m.init.ops.pop_back();
  std::vector<Op> stay;
  for (size_t i = 0; i < ex.ops.size(); ++i) {
    Op& op = ex.ops[i];
    if (h.op[i]) {
      m.init.ops.push_back(std::move(op));
    } else if (op.kind == OpKind::BufferFree && h.value[op.operands[0]]) {
      if (!usedByExec[op.operands[0]]) m.init.ops.push_back(std::move(op));  // an init-only temporary
      // else dropped: the buffer lives as long as the model
    } else {
      stay.push_back(std::move(op));
    }
  }
  ex.ops = std::move(stay);
  std::vector<ValueId> stateOf(m.numValues(), kNoValue);
  auto toState = [&](ValueId& v) {
    if (v >= h.value.size() || !h.value[v]) return;
    if (stateOf[v] == kNoValue) {
      stateOf[v] = m.newValue(m.typeOf(v), m.nameOf(v));
      initReturn.operands.push_back(v);
      ex.state.push_back(stateOf[v]);
    }
    v = stateOf[v];
  };
  for (Op& op : ex.ops) {
    for (ValueId& v : op.operands) toState(v);
    for (ValueId& v : op.outs) toState(v);
  }
  m.init.ops.push_back(std::move(initReturn));
  return Status();
}

}  // namespace

int64_t planOffsets(const std::vector<PlanItem>& items, int64_t align, std::vector<int64_t>& offsets) {
  const size_t n = items.size();
  offsets.assign(n, 0);
  std::vector<size_t> order(n);
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) {
    return items[a].bytes != items[b].bytes ? items[a].bytes > items[b].bytes : a < b;
  });
  struct Placed {
    int64_t off, size, start, end;
  };
  std::vector<Placed> placed;  // by offset
  int64_t total = 0;
  for (size_t i : order) {
    const PlanItem& b = items[i];
    const int64_t size = (std::max<int64_t>(b.bytes, 1) + align - 1) / align * align;
    // best fit: the smallest gap between lifetime-overlapping placed buffers that holds it, else past them all
    int64_t best = -1, bestGap = INT64_MAX, cursor = 0;
    for (const Placed& p : placed) {
      if (p.end < b.start || b.end < p.start) continue;
      if (p.off >= cursor) {
        const int64_t gap = p.off - cursor;
        if (gap >= size && gap < bestGap) {
          best = cursor;
          bestGap = gap;
        }
      }
      cursor = std::max(cursor, p.off + p.size);
    }
    if (best < 0) best = cursor;
    offsets[i] = best;
    total = std::max(total, best + size);
    const Placed np{best, size, b.start, b.end};
    placed.insert(std::upper_bound(placed.begin(), placed.end(), np,
                                   [](const Placed& x, const Placed& y) { return x.off < y.off; }),
                  np);
  }
  return total;
}

const std::vector<std::string>& defaultPipeline() {
  static const std::vector<std::string> p = {"dce", "bufferize", "plan-memory", "hoist-init"};
  return p;
}

Status runPass(Model& m, std::string_view name) {
  Status s;
  if (name == "dce") s = dce(m);
  else if (name == "bufferize") s = bufferize(m);
  else if (name == "plan-memory") s = planMemory(m);
  else if (name == "hoist-init") s = hoistInit(m);
  else return Status::error("unknown pass '" + std::string(name) + "'");
  if (!s) return Status::error(std::string(name) + ": " + s.message());
  if (Status v = verifyModel(m); !v) return Status::error("IR invalid after pass '" + std::string(name) + "': " + v.message());
  return Status();
}

Status internalize(Model& m, const std::vector<ExternalBytes>& data, bool copy) {
  for (Region* r : {&m.init, &m.exec})
    for (Op& op : r->ops) {
      if (op.kind != OpKind::ConstExternal) continue;
      const ExternalBytes* d = nullptr;
      for (const ExternalBytes& e : data)
        if (e.name == op.name) d = &e;
      if (!d) return Status::error("internalize: no data for external constant '" + op.name + "'");
      if (!m.findConstant(op.name)) {
        Type t = m.typeOf(op.results[0]);
        size_t bytes = dtypeSize(t->dtype);
        for (Dim dim : t->shape) {
          if (!dim->isConst() || dim->value < 0)
            return Status::error("internalize: external constant '" + op.name + "' has a symbolic shape");
          bytes *= static_cast<size_t>(dim->value);
        }
        if (d->size != bytes)
          return Status::error("internalize: '" + op.name + "' has " + std::to_string(d->size) + " bytes, its type " +
                               std::to_string(bytes));
        Constant c{op.name, t, d->owner, d->bytes, bytes};
        if (copy) {
          constexpr size_t kPage = 16384;
          void* p = std::aligned_alloc(kPage, (std::max<size_t>(bytes, 1) + kPage - 1) / kPage * kPage);
          if (!p) return Status::error("internalize: out of memory");
          if (bytes) std::memcpy(p, d->bytes, bytes);
          c.owner = std::shared_ptr<const void>(p, [](const void* q) { std::free(const_cast<void*>(q)); });
          c.bytes = static_cast<const uint8_t*>(p);
        }
        m.addConstant(std::move(c));
      }
      op.kind = OpKind::ConstInternal;
    }
  return Status();
}

}  // namespace lkrt
