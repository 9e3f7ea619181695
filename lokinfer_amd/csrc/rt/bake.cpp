// bake-init: runs a model's init once and stores its computed results as constants, so loading the baked model
// does no init work (the reference's runtime/bake_init.h:19-27 contract in lariaus/lokinfer: the same selection,
// names and pruning, so a baked model holds the same constants whichever runtime baked it). It lives beside the
// executable because it runs init.
//
// Steps (class Baker): copy the model; pick the init results that are computed data (storage a plain buffer.alloc
// that an init kernel writes, with a static shape); run init through an executable and copy each picked result to a
// page-aligned host block; make each a const.internal on its writer's device in place of the result; drop the init
// ops nothing needs any more.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <numeric>

#include "executable.h"
#include "ir.h"

namespace lkrt {

namespace {

constexpr size_t kHostPage = 16384;  // baked constants are page-aligned host blocks (the .lkm data alignment)

// What one init result becomes.
struct Pick {
  size_t slot;   // index among init's results
  ValueId value;
  size_t bytes;
  bool onGpu;
};

class Baker {
 public:
  Baker(std::shared_ptr<const Model> original, const std::vector<ExternalPtr>& ext, hipStream_t s)
      : orig_(std::move(original)), ext_(ext), stream_(s) {}

  std::unique_ptr<Model> run(BakeStats& stats, Status& st) {
    if (!(model_ = copyOf(*orig_, st))) return nullptr;
    stats.initOpsBefore = stats.initOpsAfter = model_->init.ops.size();
    for (const Op& op : model_->init.ops)
      if (op.kind == OpKind::DimRead || op.kind == OpKind::MemPlan) {  // init defines symbols: left alone
        st = Status();
        return std::move(model_);
      }
    if (model_->init.ops.empty() || model_->init.ops.back().kind != OpKind::Return) {
      st = Status::error("bake-init: init does not end with a return");
      return nullptr;
    }
    const std::vector<Pick> picks = choose();
    std::unique_ptr<Executable> exe = Executable::create(orig_, ext_, stream_, false, st);
    if (!exe) return nullptr;
    std::vector<Op> consts;
    for (const Pick& p : picks) {
      const void* src = exe->stateData(p.slot);
      if (!src) continue;
      Op k;
      if (st = bakeOne(p, src, k, stats); !st) return nullptr;
      consts.push_back(std::move(k));
    }
    Region& init = model_->init;
    init.ops.insert(init.ops.end() - 1, std::make_move_iterator(consts.begin()), std::make_move_iterator(consts.end()));
    prune();
    stats.initOpsAfter = init.ops.size();
    if (st = verifyModel(*model_); !st) return nullptr;
    st = Status();
    return std::move(model_);
  }

 private:
  // The copy shares the constants' bytes; everything else round-trips through the model text.
  static std::unique_ptr<Model> copyOf(const Model& m, Status& st) {
    std::unique_ptr<Model> copy = parseModel(printModel(m), st);
    if (!copy) return nullptr;
    for (Constant& c : copy->constants) {
      const Constant* src = m.findConstant(c.name);
      if (!src) continue;
      c.owner = src->owner;
      c.bytes = src->bytes;
      c.size = src->size;
    }
    return copy;
  }

  std::vector<ValueId> originsIn(const Region& r) const {
    std::vector<ValueId> o(model_->numValues());
    std::iota(o.begin(), o.end(), ValueId{0});
    for (const Op& op : r.ops)
      if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty()) o[op.results[0]] = o[op.operands[0]];
    return o;
  }

  std::vector<Pick> choose() {
    const Region& init = model_->init;
    const std::vector<ValueId> origin = originsIn(init);
    std::vector<const Op*> allocOf(model_->numValues(), nullptr);
    std::vector<int8_t> writer(model_->numValues(), -1);  // device of the last init kernel writing an origin
    for (const Op& op : init.ops) {
      if (op.kind == OpKind::BufferAlloc) allocOf[op.results[0]] = &op;
      if (op.kind == OpKind::Kernel)
        for (ValueId v : op.outs) writer[origin[v]] = isGpuKernelName(op.name) ? 1 : 0;
    }
    std::vector<Pick> picks;
    const std::vector<ValueId>& results = init.ops.back().operands;
    for (size_t i = 0; i < results.size(); ++i) {
      const ValueId v = results[i], o = origin[v];
      const Op* alloc = allocOf[o];
      if (!alloc || writer[o] < 0) continue;  // a constant, a view of an arena, an unwritten buffer, ...
      if (alloc->flag("arena") || alloc->flag("persistent") || alloc->flag("output")) continue;
      const Type t = model_->typeOf(v);
      size_t bytes = dtypeSize(t->dtype);
      bool fixed = true;
      for (Dim d : t->shape) {
        fixed = fixed && d->isConst() && d->value >= 0;
        if (fixed) bytes *= static_cast<size_t>(d->value);
      }
      if (fixed) picks.push_back({i, v, bytes, writer[o] == 1});
    }
    return picks;
  }

  Status bakeOne(const Pick& p, const void* src, Op& k, BakeStats& stats) {
    const size_t cap = (std::max<size_t>(p.bytes, 1) + kHostPage - 1) / kHostPage * kHostPage;
    void* host = std::aligned_alloc(kHostPage, cap);
    if (!host) return Status::error("bake-init: out of host memory");
    std::shared_ptr<const void> owner(host, [](const void* q) { std::free(const_cast<void*>(q)); });
    if (p.bytes && hipMemcpy(host, src, p.bytes, hipMemcpyDefault) != hipSuccess) {
      (void)hipGetLastError();
      return Status::error("bake-init: copying init result " + std::to_string(p.slot) + " failed");
    }
    std::string name = "baked" + std::to_string(p.slot);
    while (model_->findConstant(name)) name.push_back('_');
    const Type t = model_->typeOf(p.value);
    model_->addConstant(Constant{name, t, owner, static_cast<const uint8_t*>(host), p.bytes});
    const std::string& hint = model_->nameOf(p.value);
    const ValueId baked = model_->newValue(t, hint.empty() ? name : hint + "_baked");
    k.kind = OpKind::ConstInternal;
    k.name = name;
    k.setAttr("device", AttrValue{std::string(p.onGpu ? "gpu" : "cpu")});
    k.results.push_back(baked);
    model_->init.ops.back().operands[p.slot] = baked;
    ++stats.baked;
    stats.bakedBytes += p.bytes;
    return Status();
  }

  // Backward over init: a value is wanted when a kept op reads it (its storage is wanted with it). Kept: return and
  // dim.read; kernels with an effect of their own (an in-place write, or no outputs at all) or writing wanted
  // storage or producing a wanted result; allocs whose storage or value is wanted; other ops whose result is; a
  // buffer.free when its buffer's storage is wanted.
  void prune() {
    Region& init = model_->init;
    const size_t nv = model_->numValues(), n = init.ops.size();
    const std::vector<ValueId> origin = originsIn(init);
    std::vector<uint8_t> wantValue(nv, 0), wantStorage(nv, 0), keep(n, 0);
    auto want = [&](ValueId v) {
      wantValue[v] = 1;
      wantStorage[origin[v]] = 1;
    };
    for (size_t i = n; i-- > 0;) {
      const Op& op = init.ops[i];
      bool kept = false;
      if (op.kind == OpKind::Return || op.kind == OpKind::DimRead) {
        kept = true;
      } else if (op.kind == OpKind::Kernel) {
        kept = op.attr("inout") || (op.outs.empty() && op.results.empty()) ||
               std::any_of(op.outs.begin(), op.outs.end(), [&](ValueId v) { return wantStorage[origin[v]]; }) ||
               std::any_of(op.results.begin(), op.results.end(), [&](ValueId v) { return wantValue[v]; });
        if (kept)
          for (ValueId v : op.outs) want(v);
      } else if (op.kind == OpKind::BufferAlloc) {
        kept = wantStorage[op.results[0]] || wantValue[op.results[0]];
      } else if (op.kind != OpKind::BufferFree) {
        kept = std::any_of(op.results.begin(), op.results.end(), [&](ValueId v) { return wantValue[v] || wantStorage[v]; });
      }
      if (!kept) continue;
      keep[i] = 1;
      for (ValueId v : op.operands) want(v);
    }
    std::vector<Op> kept;
    for (size_t i = 0; i < n; ++i) {
      Op& op = init.ops[i];
      if (keep[i] || (op.kind == OpKind::BufferFree && wantStorage[origin[op.operands[0]]])) kept.push_back(std::move(op));
    }
    init.ops = std::move(kept);
  }

  std::shared_ptr<const Model> orig_;
  const std::vector<ExternalPtr>& ext_;
  hipStream_t stream_;
  std::unique_ptr<Model> model_;
};

}  // namespace

std::unique_ptr<Model> bakeInit(std::shared_ptr<const Model> model, const std::vector<ExternalPtr>& ext,
                                hipStream_t stream, BakeStats* stats, Status& st) {
  BakeStats bs;
  std::unique_ptr<Model> baked = Baker(std::move(model), ext, stream).run(bs, st);
  if (baked && stats) *stats = bs;
  return baked;
}

}  // namespace lkrt
