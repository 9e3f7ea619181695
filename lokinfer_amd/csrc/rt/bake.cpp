// bake-init: run a model's init once and store its computed results as constants (the reference's
// runtime/bake_init.h:19-27, src/runtime/bake_init.cpp in lariaus/lokinfer; the same selection rules, so a baked
// model from either runtime holds the same constants). Lives beside the executable because it runs init.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "executable.h"
#include "ir.h"

namespace lkrt {

namespace {

constexpr size_t kPage = 16384;  // baked constants are page-aligned host copies (the .lkm data alignment)

// An exact copy: the text form round-trips the IR; the constants' bytes are shared with the original.
std::unique_ptr<Model> cloneModel(const Model& m, Status& st) {
  std::unique_ptr<Model> c = parseModel(printModel(m), st);
  if (!c) return nullptr;
  for (Constant& k : c->constants)
    if (const Constant* o = m.findConstant(k.name)) {
      k.owner = o->owner;
      k.bytes = o->bytes;
      k.size = o->size;
    }
  return c;
}

// Keeps the init ops something still needs, walking backwards from the return: a kernel is needed when it writes
// in place, writes nothing, or writes / returns a needed value (views share their root buffer's liveness); a
// buffer.free goes with its buffer.
void pruneInit(Model& m) {
  Region& r = m.init;
  const size_t nv = m.numValues();
  std::vector<ValueId> root(nv, kNoValue);
  auto rootOf = [&](ValueId v) { return root[v] == kNoValue ? v : root[v]; };
  for (const Op& op : r.ops)
    if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
      root[op.results[0]] = rootOf(op.operands[0]);
  std::vector<uint8_t> liveVal(nv, 0), liveRoot(nv, 0), keep(r.ops.size(), 0);
  auto use = [&](ValueId v) {
    liveVal[v] = 1;
    liveRoot[rootOf(v)] = 1;
  };
  for (size_t i = r.ops.size(); i-- > 0;) {
    const Op& op = r.ops[i];
    bool k = false;
    switch (op.kind) {
      case OpKind::Return:
      case OpKind::DimRead:
        k = true;
        break;
      case OpKind::Kernel:
        k = op.attr("inout") || (op.outs.empty() && op.results.empty());
        for (ValueId v : op.outs) k = k || liveRoot[rootOf(v)];
        for (ValueId v : op.results) k = k || liveVal[v];
        if (k)
          for (ValueId v : op.outs) use(v);
        break;
      case OpKind::BufferFree:
        break;  // decided below, from its buffer
      case OpKind::BufferAlloc:
        k = liveRoot[op.results[0]] || liveVal[op.results[0]];
        break;
      default:
        for (ValueId v : op.results) k = k || liveVal[v] || liveRoot[v];
        break;
    }
    if (!k) continue;
    keep[i] = 1;
    for (ValueId v : op.operands) use(v);
  }
  for (size_t i = 0; i < r.ops.size(); ++i)
    if (r.ops[i].kind == OpKind::BufferFree) keep[i] = liveRoot[rootOf(r.ops[i].operands[0])];
  std::vector<Op> kept;
  for (size_t i = 0; i < r.ops.size(); ++i)
    if (keep[i]) kept.push_back(std::move(r.ops[i]));
  r.ops = std::move(kept);
}

}  // namespace

std::unique_ptr<Model> bakeInit(std::shared_ptr<const Model> model, const std::vector<ExternalPtr>& ext,
                                hipStream_t stream, BakeStats* stats, Status& st) {
  BakeStats bs;
  std::unique_ptr<Model> c = cloneModel(*model, st);
  if (!c) return nullptr;
  bs.initOpsBefore = bs.initOpsAfter = c->init.ops.size();
  for (const Op& op : c->init.ops)
    if (op.kind == OpKind::DimRead || op.kind == OpKind::MemPlan) {  // init defines symbols: left as it is
      if (stats) *stats = bs;
      st = Status();
      return c;
    }
  std::unique_ptr<Executable> exe = Executable::create(model, ext, stream, false, st);
  if (!exe) return nullptr;

  Region& init = c->init;
  const size_t nv = c->numValues();
  std::vector<ValueId> root(nv, kNoValue);
  auto rootOf = [&](ValueId v) { return root[v] == kNoValue ? v : root[v]; };
  std::vector<int> allocAt(nv, -1);
  std::vector<int8_t> writerGpu(nv, -1);  // root -> device of its last init writer (-1: none)
  for (size_t i = 0; i < init.ops.size(); ++i) {
    const Op& op = init.ops[i];
    if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
      root[op.results[0]] = rootOf(op.operands[0]);
    if (op.kind == OpKind::BufferAlloc) allocAt[op.results[0]] = static_cast<int>(i);
    if (op.kind == OpKind::Kernel)
      for (ValueId v : op.outs) writerGpu[rootOf(v)] = isGpuKernelName(op.name) ? 1 : 0;
  }
  if (init.ops.empty() || init.ops.back().kind != OpKind::Return) {
    st = Status::error("bake-init: init does not end with a return");
    return nullptr;
  }
  std::vector<Op> consts;
  Op& ret = init.ops.back();
  for (size_t i = 0; i < ret.operands.size(); ++i) {
    const ValueId v = ret.operands[i];
    const ValueId rv = rootOf(v);
    if (allocAt[rv] < 0 || writerGpu[rv] < 0) continue;  // not a computed buffer (a constant, an arena view, ...)
    const Op& alloc = init.ops[static_cast<size_t>(allocAt[rv])];
    if (alloc.flag("arena") || alloc.flag("persistent") || alloc.flag("output")) continue;
    const Type t = c->typeOf(v);
    size_t bytes = dtypeSize(t->dtype);
    bool isStatic = true;
    for (Dim d : t->shape) {
      isStatic = isStatic && d->isConst() && d->value >= 0;
      if (isStatic) bytes *= static_cast<size_t>(d->value);
    }
    const void* src = exe->stateData(i);
    if (!isStatic || !src) continue;
    void* p = std::aligned_alloc(kPage, (std::max<size_t>(bytes, 1) + kPage - 1) / kPage * kPage);
    if (!p) {
      st = Status::error("bake-init: out of host memory");
      return nullptr;
    }
    std::shared_ptr<const void> owner(p, [](const void* q) { std::free(const_cast<void*>(q)); });
    if (bytes && hipMemcpy(p, src, bytes, hipMemcpyDefault) != hipSuccess) {
      (void)hipGetLastError();
      st = Status::error("bake-init: copying init result " + std::to_string(i) + " failed");
      return nullptr;
    }
    std::string name = "baked" + std::to_string(i);
    while (c->findConstant(name)) name += "_";
    c->addConstant(Constant{name, t, owner, static_cast<const uint8_t*>(p), bytes});
    Op k;
    k.kind = OpKind::ConstInternal;
    k.name = name;
    k.setAttr("device", AttrValue{std::string(writerGpu[rv] ? "gpu" : "cpu")});
    const ValueId nid = c->newValue(t, c->nameOf(v).empty() ? name : c->nameOf(v) + "_baked");
    k.results.push_back(nid);
    ret.operands[i] = nid;
    consts.push_back(std::move(k));
    ++bs.baked;
    bs.bakedBytes += bytes;
  }
  init.ops.insert(init.ops.end() - 1, std::make_move_iterator(consts.begin()), std::make_move_iterator(consts.end()));
  pruneInit(*c);
  bs.initOpsAfter = c->init.ops.size();
  if (Status v = verifyModel(*c); !v) {
    st = v;
    return nullptr;
  }
  if (stats) *stats = bs;
  st = Status();
  return c;
}

}  // namespace lkrt
