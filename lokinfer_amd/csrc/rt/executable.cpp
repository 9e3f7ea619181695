// The MI355X executable (see executable.h). Instruction lowering follows the reference's argument convention
// (include/lokinfer/runtime/kernel.h:3-11, src/runtime/executable.cpp:406-447): a kernel gets its operands then
// its outs as pointers; ints = every operand's dims, every out's dims, then the non-structural int / bool /
// int-list / dim attrs in name order; floats = the float attrs in name order.
#include "executable.h"

#include <algorithm>
#include <array>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "lokinfer_hip.h"

namespace lkrt {

namespace {

constexpr int64_t kUnbound = INT64_MIN;
constexpr size_t kAlign = 256;
constexpr size_t kWorkspaceBytes = size_t(64) << 20;
constexpr size_t kMaxInts = 256, kMaxFloats = 32;  // the registry's argument maxima (lk_run_kernel)

size_t alignUp(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

Status hipStatus(hipError_t e, const char* what) {
  if (e == hipSuccess) return Status();
  (void)hipGetLastError();
  return Status::error(std::string(what) + ": " + hipGetErrorString(e));
}

Status deviceErrors() {
  int64_t detail = 0;
  const int code = lk_take_device_error(&detail);
  if (code == 0) return Status();
  if (code < 0) return Status::error("could not read the device error record");
  return Status::error("device error " + std::to_string(code) + ": " + lk_device_error_message(code) + " (detail " +
                       std::to_string(detail) + ")");
}

}  // namespace

struct Executable::Instr {
  OpKind kind;
  const Op* op;
  const lkh::KernelEntry* kernel = nullptr;
  std::vector<ValueId> args;  // kernel: operands then outs
  std::vector<int64_t> ints;  // static ints; dynInts patch the symbolic ones per call
  std::vector<std::pair<uint32_t, Dim>> dynInts;
  std::vector<double> floats;
  std::vector<double> floatBuf;  // floats, zero-padded to kMaxFloats
  mutable std::vector<void*> ptrBuf;
  mutable std::vector<int64_t> intBuf;  // ints (symbolic ones patched per call), zero-padded to kMaxInts
  int lane = 0;            // concurrency lane of a captured call (its workspace; kernels of a lane are ordered)
  std::vector<int> waits;  // kernels of other lanes this one depends on (not already implied by its lane's order)
};

// One kernel instruction's nodes in a graph captured on one stream: a chain from `first` to `tail` (both null when
// the kernel enqueued nothing); `before` is the capture's tail node before the kernel.
struct Executable::Segment {
  hipGraphNode_t before = nullptr, first = nullptr, tail = nullptr;
};

Executable::Memory::~Memory() {
  if (p) (void)hipFree(p);
}

Executable::~Executable() {
  for (auto& [k, g] : graphs_) {
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
  }
  if (captureStream_) (void)hipStreamDestroy(captureStream_);
  for (size_t k = 1; k < laneStreams_.size(); ++k) (void)hipStreamDestroy(laneStreams_[k]);
  for (hipEvent_t e : laneEvents_)
    if (e) (void)hipEventDestroy(e);
  if (pinned_) (void)hipHostFree(pinned_);
}

char* Executable::Bump::alloc(size_t bytes, Status& st) {
  bytes = alignUp(std::max<size_t>(bytes, 1));
  if (!blocks.empty() && used + bytes <= blocks.back()->n) {
    char* p = static_cast<char*>(blocks.back()->p) + used;
    used += bytes;
    return p;
  }
  auto m = std::make_unique<Memory>();
  m->n = std::max({bytes, 2 * capacity(), size_t(1) << 20});
  if (hipError_t e = hipMalloc(&m->p, m->n); e != hipSuccess) {
    st = hipStatus(e, "hipMalloc (call arena)");
    return nullptr;
  }
  blocks.push_back(std::move(m));
  used = bytes;
  return static_cast<char*>(blocks.back()->p);
}

size_t Executable::Bump::capacity() const {
  size_t n = 0;
  for (const auto& b : blocks) n += b->n;
  return n;
}

size_t Executable::callArenaBytes() const {
  size_t n = eager_.capacity();
  for (const auto& [k, g] : graphs_) n += g->mem ? g->mem->n : 0;
  return n;
}

std::string Executable::strategy() const {
  if (dynamic_) return "eager (data-dependent shapes or host scalar inputs)";
  return graphs_on_ ? "hipGraph per input-shape binding" : "eager";
}

Status Executable::lower(const Region& r, std::vector<Instr>& out) {
  const Model& m = *model_;
  for (const Op& op : r.ops) {
    Instr in;
    in.kind = op.kind;
    in.op = &op;
    if (op.kind == OpKind::Kernel) {
      if (!op.results.empty()) return Status::error("kernel '" + op.name + "' still has results (run bufferize)");
      in.kernel = lkh::findKernel(op.name);
      if (!in.kernel) {
        return Status::error(isGpuKernelName(op.name)
                                 ? "unknown kernel '" + op.name + "'"
                                 : "kernel '" + op.name + "' is a host kernel: this runtime runs GPU kernels only");
      }
      if ((in.kernel->device == lkh::Device::Gpu) != isGpuKernelName(op.name))
        return Status::error("kernel '" + op.name + "' is registered on a device its name doesn't say");
      in.args = op.operands;
      in.args.insert(in.args.end(), op.outs.begin(), op.outs.end());
      if (in.kernel->numOperands >= 0 &&
          (op.operands.size() != static_cast<size_t>(in.kernel->numOperands) ||
           op.outs.size() != static_cast<size_t>(in.kernel->numOuts)))
        return Status::error("kernel '" + op.name + "' takes " + std::to_string(in.kernel->numOperands) +
                             " operands and " + std::to_string(in.kernel->numOuts) + " outs");
      auto addDim = [&](Dim d) {
        if (!d->isConst()) in.dynInts.emplace_back(static_cast<uint32_t>(in.ints.size()), d);
        in.ints.push_back(d->isConst() ? d->value : 0);
      };
      for (ValueId v : in.args)
        for (Dim d : m.typeOf(v)->shape) addDim(d);
      for (const NamedAttr& a : op.attrs) {
        if (isStructuralAttr(a.name)) continue;
        switch (a.value.index()) {
          case 0: in.ints.push_back(std::get<bool>(a.value) ? 1 : 0); break;
          case 1: in.ints.push_back(std::get<int64_t>(a.value)); break;
          case 2: in.floats.push_back(std::get<double>(a.value)); break;
          case 3: break;  // string attrs carry no kernel argument
          case 4: {
            const Ints& v = std::get<Ints>(a.value);
            in.ints.insert(in.ints.end(), v.begin(), v.end());
            break;
          }
          case 5: {
            const Floats& v = std::get<Floats>(a.value);
            in.floats.insert(in.floats.end(), v.begin(), v.end());
            break;
          }
          default: addDim(std::get<Dim>(a.value));
        }
      }
      if (in.ints.size() > kMaxInts || in.floats.size() > kMaxFloats)
        return Status::error("kernel '" + op.name + "': too many int / float arguments");
      in.ptrBuf.resize(in.args.size());
      // Runners index ints and floats by position: the arrays a call passes are zero-padded to the registry's
      // maxima (as lk_run_kernel pads a caller's arrays), so a dim or attribute the op does not carry reads as 0,
      // which every runner's shape checks reject, instead of reading past the array.
      in.intBuf = in.ints;
      in.intBuf.resize(kMaxInts, 0);
      in.floatBuf = in.floats;
      in.floatBuf.resize(kMaxFloats, 0.0);
    } else if (op.kind == OpKind::MemPlan && r.args.empty() && &r == &model_->init) {
      return Status::error("mem.plan in init is not supported");
    }
    out.push_back(std::move(in));
  }
  return Status();
}

// Binds every symbol the exec inputs' shapes define: a dim that is (a sum of bound terms plus) k * S with S the
// one unbound symbol binds S; every other dim is checked against the input's extent.
Status Executable::bindInputs(const std::vector<TensorIn>& in, std::vector<int64_t>& sv) const {
  const Model& m = *model_;
  const Region& ex = m.exec;
  if (in.size() != ex.args.size())
    return Status::error("expected " + std::to_string(ex.args.size()) + " inputs, got " + std::to_string(in.size()));
  sv.assign(m.dims().numSymbols(), kUnbound);
  for (size_t i = 0; i < in.size(); ++i) {
    Type t = m.typeOf(ex.args[i]);
    if (in[i].dtype != t->dtype)
      return Status::error("input " + std::to_string(i) + ": expected dtype " + dtypeName(t->dtype) + ", got " +
                           dtypeName(in[i].dtype));
    if (in[i].shape.size() != t->shape.size())
      return Status::error("input " + std::to_string(i) + ": expected rank " + std::to_string(t->shape.size()) +
                           ", got " + std::to_string(in[i].shape.size()));
    if (!in[i].data && !t->isScalar()) return Status::error("input " + std::to_string(i) + " has no data");
  }
  const DimPool& dp = m.dims();
  // linear form k * S + b of d in one unbound symbol S (b evaluable now)
  auto linear = [&](Dim d, int64_t& sym, int64_t& k, int64_t& b) {
    auto term = [&](Dim t, int64_t& s, int64_t& c) {
      if (t->kind == DimKind::Sym && sv[static_cast<size_t>(t->value)] == kUnbound) {
        s = t->value;
        c = 1;
        return true;
      }
      if (t->kind == DimKind::Mul && t->args.size() == 2 && t->args[0]->isConst() && t->args[1]->kind == DimKind::Sym &&
          sv[static_cast<size_t>(t->args[1]->value)] == kUnbound) {
        s = t->args[1]->value;
        c = t->args[0]->value;
        return true;
      }
      return false;
    };
    if (term(d, sym, k)) {
      b = 0;
      return true;
    }
    if (d->kind != DimKind::Add) return false;
    bool found = false;
    b = 0;
    for (Dim t : d->args) {
      int64_t s, c;
      if (auto v = dp.eval(t, sv, kUnbound)) {
        b += *v;
      } else if (!found && term(t, s, c)) {
        found = true;
        sym = s;
        k = c;
      } else {
        return false;
      }
    }
    return found;
  };
  for (int pass = 0;; ++pass) {
    bool progress = false, pending = false;
    for (size_t i = 0; i < in.size(); ++i) {
      Type t = m.typeOf(ex.args[i]);
      for (size_t j = 0; j < t->shape.size(); ++j) {
        const int64_t actual = in[i].shape[j];
        if (dp.eval(t->shape[j], sv, kUnbound)) continue;
        int64_t sym = 0, k = 0, b = 0;
        if (linear(t->shape[j], sym, k, b) && k != 0 && (actual - b) % k == 0) {
          sv[static_cast<size_t>(sym)] = (actual - b) / k;
          progress = true;
        } else {
          pending = true;
        }
      }
    }
    if (!pending) break;
    if (!progress) return Status::error("cannot bind the symbols of the input shapes");
  }
  for (size_t i = 0; i < in.size(); ++i) {
    Type t = m.typeOf(ex.args[i]);
    for (size_t j = 0; j < t->shape.size(); ++j) {
      const int64_t want = *dp.eval(t->shape[j], sv, kUnbound);
      if (want != in[i].shape[j] || want < 0)
        return Status::error("input " + std::to_string(i) + " dim " + std::to_string(j) + " is " +
                             std::to_string(in[i].shape[j]) + ", the model's shape " + m.types().str(t) + " needs " +
                             std::to_string(want));
    }
  }
  return Status();
}

Status Executable::interpret(const std::vector<Instr>& code, std::vector<char*>& slot, std::vector<int64_t>& sv,
                             Bump& mem, hipStream_t s, std::vector<TensorOut>* outs, std::vector<Segment>* segs,
                             bool laneStreams) {
  const Model& m = *model_;
  const DimPool& dp = m.dims();
  // A captured call records the graph nodes each kernel instruction enqueued (the capture runs on one stream, so
  // they form a chain); the graph's edges are re-wired from the lanes afterwards (rewire).
  auto captureTail = [&](hipGraphNode_t& tail) -> Status {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipGraphNode_t* deps = nullptr;
    size_t nd = 0;
    LKRT_TRY(hipStatus(hipStreamGetCaptureInfo_v2(s, &cs, nullptr, nullptr, &deps, &nd), "capture info"));
    if (cs != hipStreamCaptureStatusActive || nd > 1) return Status::error("capture: not a single-stream capture");
    tail = nd ? deps[0] : nullptr;
    return Status();
  };
  auto eval = [&](Dim d, int64_t& v) -> bool {
    auto r = dp.eval(d, sv, kUnbound);
    if (!r) return false;
    v = *r;
    return true;
  };
  auto bytesOf = [&](Type t, int64_t& n) -> bool {
    n = static_cast<int64_t>(dtypeSize(t->dtype));
    for (Dim d : t->shape) {
      int64_t v;
      if (!eval(d, v) || v < 0) return false;
      n *= v;
    }
    return true;
  };
  for (const Instr& in : code) {
    const Op& op = *in.op;
    switch (in.kind) {
      case OpKind::Kernel: {
        for (size_t k = 0; k < in.args.size(); ++k) {
          const ValueId v = in.args[k];
          if (m.typeOf(v)->isScalar()) {
            in.ptrBuf[k] = &scalars_[v];
          } else {
            if (!slot[v]) return Status::error("kernel '" + op.name + "': an argument has no memory");
            in.ptrBuf[k] = slot[v];
          }
        }
        for (const auto& [idx, d] : in.dynInts)
          if (!eval(d, in.intBuf[idx])) return Status::error("kernel '" + op.name + "': unbound symbol in its shapes");
        lkh::KernelArgs a{in.ptrBuf.data(), nullptr, in.intBuf.data(), in.floatBuf.data(), nullptr,
                          static_cast<uint32_t>(in.ptrBuf.size()), static_cast<uint32_t>(in.ints.size()),
                          static_cast<uint32_t>(in.floats.size())};
        Segment* seg = segs ? &(*segs)[static_cast<size_t>(&in - code.data())] : nullptr;
        if (seg) LKRT_TRY(captureTail(seg->before));
        lkh::ExecCtx ctx;
        ctx.stream = s;
        const size_t ji = static_cast<size_t>(&in - code.data());
        if (laneStreams) {
          ctx.stream = laneStreams_[static_cast<size_t>(in.lane)];
          for (int w : in.waits)
            LKRT_TRY(hipStatus(hipStreamWaitEvent(ctx.stream, laneEvents_[static_cast<size_t>(w)], 0), "lane wait"));
        }
        ctx.workspace = workspace_[&code == &exec_ ? static_cast<size_t>(in.lane) : 0];
        ctx.workspaceBytes = workspaceBytes_;
        in.kernel->run(ctx, a);
        if (ctx.error) return Status::error("kernel '" + op.name + "': " + ctx.error);
        if (laneStreams && laneEvents_[ji])
          LKRT_TRY(hipStatus(hipEventRecord(laneEvents_[ji], ctx.stream), "lane event"));
        if (seg) {
          LKRT_TRY(captureTail(seg->tail));
          if (seg->tail == seg->before) {
            seg->tail = nullptr;  // enqueued nothing
          } else {  // walk the chain back to the kernel's first node
            hipGraphNode_t n = seg->tail;
            for (;;) {
              size_t nd = 0;
              LKRT_TRY(hipStatus(hipGraphNodeGetDependencies(n, nullptr, &nd), "graph node"));
              if (nd > 1) return Status::error("capture: a kernel's nodes are not a chain");
              hipGraphNode_t dep = nullptr;
              if (nd) LKRT_TRY(hipStatus(hipGraphNodeGetDependencies(n, &dep, &nd), "graph node"));
              if (dep == seg->before) break;
              if (!dep) return Status::error("capture: a kernel's nodes do not follow the previous kernel's");
              n = dep;
            }
            seg->first = n;
          }
        }
        break;
      }
      case OpKind::View: {
        int64_t off;
        if (!eval(op.dims[0], off)) return Status::error("view: unbound symbol in its offset");
        Type src = m.typeOf(op.operands[0]), dst = m.typeOf(op.results[0]);
        const int64_t es = static_cast<int64_t>(dtypeSize(dst->dtype));
        int64_t sb, db;
        if (bytesOf(src, sb) && bytesOf(dst, db) && (off < 0 || off * es + db > sb))
          return Status::error("view out of bounds of its source (" + std::to_string(off * es + db) + " > " +
                               std::to_string(sb) + " bytes)");
        slot[op.results[0]] = slot[op.operands[0]] ? slot[op.operands[0]] + off * es : nullptr;
        break;
      }
      case OpKind::BufferAlloc: {
        const ValueId v = op.results[0];
        if (fixed_[v] || skipAlloc_[v]) {  // model memory, or an arena whose temporaries were re-placed
          slot[v] = fixed_[v];
          break;
        }
        int64_t n;
        if (!bytesOf(m.typeOf(v), n)) return Status::error("buffer.alloc: unbound symbol in its shape");
        Status st;
        slot[v] = mem.alloc(static_cast<size_t>(n), st);
        if (!slot[v]) return st;
        break;
      }
      case OpKind::MemPlan: {
        std::vector<PlanItem> items;
        for (size_t k = 0; k < op.dims.size(); ++k) {
          int64_t n;
          if (!eval(op.dims[k], n)) return Status::error("mem.plan: unbound symbol in a size");
          items.push_back({n, op.ints[2 * k], op.ints[2 * k + 1]});
        }
        std::vector<int64_t> offs;
        const int64_t total = planOffsets(items, op.ints.back(), offs);
        const Ints* elem = op.attr("elem") ? std::get_if<Ints>(op.attr("elem")) : nullptr;
        sv[static_cast<size_t>(op.symbols[0])] = total;
        for (size_t k = 0; k < offs.size(); ++k)
          sv[static_cast<size_t>(op.symbols[k + 1])] = offs[k] / (elem ? (*elem)[k] : 1);
        Status st;
        slot[op.results[0]] = mem.alloc(static_cast<size_t>(total), st);
        if (!slot[op.results[0]]) return st;
        break;
      }
      case OpKind::DimRead: {
        const ValueId v = op.operands[0];
        const size_t es = dtypeSize(m.typeOf(v)->dtype);
        int64_t have;  // the index against the operand's extent (the verifier checks it only for static shapes)
        if (!bytesOf(m.typeOf(v), have) || op.ints[0] < 0 || (op.ints[0] + 1) * static_cast<int64_t>(es) > have)
          return Status::error("dim.read: index " + std::to_string(op.ints[0]) + " is outside its operand");
        if (!slot[v]) return Status::error("dim.read: its operand has no memory");
        LKRT_TRY(hipStatus(hipMemcpyAsync(pinned_, slot[v] + op.ints[0] * static_cast<int64_t>(es), es,
                                          hipMemcpyDeviceToHost, s),
                           "dim.read"));
        LKRT_TRY(hipStatus(hipStreamSynchronize(s), "dim.read"));
        int64_t val;
        if (es == 8) {
          val = *pinned_;
        } else {
          int32_t x;
          std::memcpy(&x, pinned_, 4);
          val = x;
        }
        if (val < 0) return Status::error("dim.read: negative value " + std::to_string(val));
        sv[static_cast<size_t>(op.symbols[0])] = val;
        break;
      }
      case OpKind::Sync:
        if (!op.results.empty()) slot[op.results[0]] = slot[op.operands[0]];  // one address space on the device
        break;
      case OpKind::ConstInline:
      case OpKind::ConstInternal:
      case OpKind::ConstExternal:
        slot[op.results[0]] = fixed_[op.results[0]];
        break;
      case OpKind::BufferFree:
        break;
      case OpKind::Return:
        if (outs) {
          outs->clear();
          for (ValueId v : op.operands) {
            TensorOut o{slot[v], {}, m.typeOf(v)->dtype};
            for (Dim d : m.typeOf(v)->shape) {
              int64_t x;
              if (!eval(d, x)) return Status::error("return: unbound symbol in an output shape");
              o.shape.push_back(x);
            }
            outs->push_back(std::move(o));
          }
        }
        break;
    }
  }
  return Status();
}

Status Executable::callBytes(std::vector<int64_t> sv, size_t& bytes) const {
  const Model& m = *model_;
  bytes = 0;
  for (const Instr& in : exec_) {
    const Op& op = *in.op;
    if (in.kind == OpKind::BufferAlloc && !fixed_[op.results[0]]) {
      int64_t n = static_cast<int64_t>(dtypeSize(m.typeOf(op.results[0])->dtype));
      for (Dim d : m.typeOf(op.results[0])->shape) {
        auto v = m.dims().eval(d, sv, kUnbound);
        if (!v) return Status::error("buffer.alloc: unbound symbol");
        n *= *v;
      }
      bytes += alignUp(static_cast<size_t>(std::max<int64_t>(n, 1)));
    } else if (in.kind == OpKind::MemPlan) {
      std::vector<PlanItem> items;
      for (size_t k = 0; k < op.dims.size(); ++k) {
        auto v = m.dims().eval(op.dims[k], sv, kUnbound);
        if (!v) return Status::error("mem.plan: unbound symbol");
        items.push_back({*v, op.ints[2 * k], op.ints[2 * k + 1]});
      }
      std::vector<int64_t> offs;
      const int64_t total = planOffsets(items, op.ints.back(), offs);
      const Ints* elem = op.attr("elem") ? std::get_if<Ints>(op.attr("elem")) : nullptr;
      sv[static_cast<size_t>(op.symbols[0])] = total;
      for (size_t k = 0; k < offs.size(); ++k)
        sv[static_cast<size_t>(op.symbols[k + 1])] = offs[k] / (elem ? (*elem)[k] : 1);
      bytes += alignUp(static_cast<size_t>(std::max<int64_t>(total, 1)));
    }
  }
  return Status();
}

// Lane schedule of a statically shaped exec region, and the re-placement of its per-call temporaries.
//
// Dependencies are per memory root (a value, seen through views and syncs): a kernel depends on the last writer of
// every root it reads or writes and, for the roots it writes, on their readers since that write. In program order,
// a kernel continues the lane whose last kernel is its latest predecessor; if no predecessor ends a lane it takes
// an unused lane, else the lane whose last kernel is oldest. Kernels of one lane are ordered (they share the lane's
// workspace); a dependency on another lane is kept as a wait unless the vector clock of the waiting lane already
// covers it; the vector clocks then give happens-before between any two kernels. The lanes become edges of the
// call's captured graph (rewire), so concurrent branches run concurrently on replay without side streams.
//
// The temporaries plan-memory put in a static arena (hoisted to init, reaching exec as state) were placed for one
// lane. They are placed again here, largest first at the lowest fitting offset, where two of them conflict unless
// every kernel touching one happens before the first kernel touching the other: concurrent branches never share
// bytes, and the schedule needs no extra edges.
Status Executable::schedule(int maxLanes) {
  const Model& m = *model_;
  const Region& ex = m.exec;
  const size_t nv = m.numValues();
  const int S = std::max(1, std::min(maxLanes, 8));
  relocOffset_.assign(nv, -1);
  skipAlloc_.assign(nv, 0);

  // relocatable temporaries: exec state whose init value is a view of an init arena no init kernel touches
  std::vector<ValueId> iroot(nv, kNoValue);
  auto irootOf = [&](ValueId v) { return iroot[v] == kNoValue ? v : iroot[v]; };
  std::vector<uint8_t> arena(nv, 0);
  for (const Op& op : m.init.ops) {
    if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty())
      iroot[op.results[0]] = irootOf(op.operands[0]);
    if (op.kind == OpKind::BufferAlloc && op.flag("arena")) arena[op.results[0]] = 1;
  }
  for (const Op& op : m.init.ops)
    if (op.kind == OpKind::Kernel)
      for (const auto* vs : {&op.operands, &op.outs})
        for (ValueId v : *vs) arena[irootOf(v)] = 0;
  const Op& initRet = m.init.ops.back();
  // Exec state can alias other exec state: init may return a view and a view of that view (a slice of a style-bank
  // projection), which exec receives as two values. Each state value is resolved to its outermost state ancestor
  // (`outer`, at byte offset `outerOff`): only those are re-placed, a nested one keeps its offset inside its
  // ancestor, and in exec every access to it is an access to the ancestor.
  std::vector<ValueId> iparent(nv, kNoValue);
  std::vector<int64_t> ioff(nv, 0);
  bool staticViews = true;
  for (const Op& op : m.init.ops)
    if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty()) {
      iparent[op.results[0]] = op.operands[0];
      if (op.kind == OpKind::View) {
        if (!op.dims[0]->isConst()) staticViews = false;
        ioff[op.results[0]] = op.dims[0]->value * static_cast<int64_t>(dtypeSize(m.typeOf(op.results[0])->dtype));
      }
    }
  std::vector<ValueId> stateOfInit(nv, kNoValue);  // init value -> the first exec state value it becomes
  for (size_t i = 0; i < ex.state.size(); ++i)
    if (stateOfInit[initRet.operands[i]] == kNoValue) stateOfInit[initRet.operands[i]] = ex.state[i];
  std::vector<ValueId> outer(nv, kNoValue);
  std::vector<int64_t> outerOff(nv, 0);
  for (size_t i = 0; i < ex.state.size(); ++i) {
    const ValueId sv = ex.state[i];
    ValueId best = sv;
    int64_t off = 0, acc = 0;
    for (ValueId iv = initRet.operands[i]; iv != kNoValue; iv = iparent[iv]) {
      const ValueId s = stateOfInit[iv];
      if (s != kNoValue && s != sv) {
        best = s;
        off = acc;
      }
      acc += ioff[iv];
    }
    outer[sv] = best;
    outerOff[sv] = off;
  }
  // a state value that is its own outermost ancestor is re-placed when it lives in a relocatable arena and every
  // dim is static
  bool relocOk = staticViews;
  std::vector<uint8_t> reloc(nv, 0);
  for (size_t i = 0; i < ex.state.size(); ++i) {
    const ValueId sv = ex.state[i];
    if (!arena[irootOf(initRet.operands[i])]) continue;
    for (Dim d : m.typeOf(sv)->shape) relocOk = relocOk && d->isConst();
    if (outer[sv] == sv) reloc[sv] = 1;
  }
  if (!relocOk) {  // symbolic temporaries: keep one lane and the compiler's placement
    numLanes_ = 1;
    return Status();
  }
  for (const Op& op : m.init.ops)
    if (op.kind == OpKind::BufferAlloc && arena[op.results[0]]) skipAlloc_[op.results[0]] = 1;

  // dependencies between exec kernels
  std::vector<ValueId> root(nv, kNoValue);
  for (ValueId sv : ex.state)
    if (outer[sv] != sv) root[sv] = outer[sv];
  auto rootOf = [&](ValueId v) { return root[v] == kNoValue ? v : root[v]; };
  std::vector<int> lastWriter(nv, -1);
  std::vector<std::vector<int>> readers(nv);
  std::vector<std::vector<int>> preds(exec_.size());
  std::vector<std::vector<int>> touching(nv);  // kernels touching each root
  for (size_t j = 0; j < exec_.size(); ++j) {
    const Op& op = *exec_[j].op;
    if ((op.kind == OpKind::View || op.kind == OpKind::Sync) && !op.results.empty()) {
      root[op.results[0]] = rootOf(op.operands[0]);
      continue;
    }
    if (op.kind != OpKind::Kernel) continue;
    std::vector<uint8_t> isInout(op.operands.size(), 0);
    if (const AttrValue* io = op.attr("inout"))
      if (const Ints* idx = std::get_if<Ints>(io))
        for (int64_t k : *idx)
          if (k >= 0 && static_cast<size_t>(k) < isInout.size()) isInout[static_cast<size_t>(k)] = 1;
    std::vector<ValueId> rd, wr;
    for (size_t k = 0; k < op.operands.size(); ++k) {
      if (m.typeOf(op.operands[k])->isScalar()) continue;
      (isInout[k] ? wr : rd).push_back(rootOf(op.operands[k]));
    }
    for (ValueId v : op.outs) wr.push_back(rootOf(v));
    std::vector<int>& P = preds[j];
    for (ValueId r : rd)
      if (lastWriter[r] >= 0) P.push_back(lastWriter[r]);
    for (ValueId w : wr) {
      if (lastWriter[w] >= 0) P.push_back(lastWriter[w]);
      P.insert(P.end(), readers[w].begin(), readers[w].end());
    }
    std::sort(P.begin(), P.end());
    P.erase(std::unique(P.begin(), P.end()), P.end());
    P.erase(std::remove(P.begin(), P.end(), static_cast<int>(j)), P.end());
    for (ValueId r : rd) {
      readers[r].push_back(static_cast<int>(j));
      touching[r].push_back(static_cast<int>(j));
    }
    for (ValueId w : wr) {
      lastWriter[w] = static_cast<int>(j);
      readers[w].clear();
      touching[w].push_back(static_cast<int>(j));
    }
  }

  // Stream structure from the trace: a function that issues its branches on side streams leaves on every kernel
  // its lane, its trace sequence number and the points its lane waits for (lane:seq, the waited lane's kernels up
  // to that number: a fork, a join or an event). Such a model keeps those lanes (mod the lane count) and those
  // waits, which order a branch after everything issued before its fork, as a stream capture of the function
  // would; the data-dependency waits below are added to them.
  auto strAttr = [](const Op& op, const char* n) -> const std::string* {
    const AttrValue* a = op.attr(n);
    return a ? std::get_if<std::string>(a) : nullptr;
  };
  bool hinted = false;
  for (const Instr& in : exec_)
    if (in.kind == OpKind::Kernel && strAttr(*in.op, "lane") && strAttr(*in.op, "seq")) hinted = true;
  std::vector<int> hLane(exec_.size(), 0);
  std::vector<int64_t> hSeq(exec_.size(), -1);
  std::vector<std::vector<std::pair<int, int64_t>>> hAfter(exec_.size());
  if (hinted)
    for (size_t j = 0; j < exec_.size(); ++j) {
      if (exec_[j].kind != OpKind::Kernel) continue;
      const Op& op = *exec_[j].op;
      if (const std::string* v = strAttr(op, "lane")) hLane[j] = std::max(0, std::atoi(v->c_str()));
      if (const std::string* v = strAttr(op, "seq")) hSeq[j] = std::atoll(v->c_str());
      if (const std::string* v = strAttr(op, "after")) {
        size_t at = 0;
        while (at < v->size()) {
          size_t end = v->find(',', at);
          if (end == std::string::npos) end = v->size();
          const std::string item = v->substr(at, end - at);
          const size_t colon = item.find(':');
          if (colon != std::string::npos)
            hAfter[j].emplace_back(std::atoi(item.substr(0, colon).c_str()), std::atoll(item.substr(colon + 1).c_str()));
          at = end + 1;
        }
      }
    }
  std::vector<std::vector<std::pair<int64_t, int>>> issued;  // per traced lane: (seq, kernel) in exec order

  // streams and vector clocks
  std::vector<std::array<int, 8>> vc(exec_.size());
  std::vector<int> pos(exec_.size(), 0), tail(static_cast<size_t>(S), -1), count(static_cast<size_t>(S), 0);
  for (size_t j = 0; j < exec_.size(); ++j) {
    Instr& in = exec_[j];
    if (in.kind != OpKind::Kernel) continue;
    std::vector<int> P = preds[j];
    if (hinted) {
      for (const auto& [l, q] : hAfter[j]) {  // the latest kernel of lane l traced at or before q
        if (static_cast<size_t>(l) >= issued.size()) continue;
        const auto& v = issued[static_cast<size_t>(l)];
        auto it = std::upper_bound(v.begin(), v.end(), std::make_pair(q, INT32_MAX));
        if (it != v.begin()) P.push_back(std::prev(it)->second);
      }
      std::sort(P.begin(), P.end());
      P.erase(std::unique(P.begin(), P.end()), P.end());
      if (issued.size() <= static_cast<size_t>(hLane[j])) issued.resize(static_cast<size_t>(hLane[j]) + 1);
      issued[static_cast<size_t>(hLane[j])].emplace_back(hSeq[j], static_cast<int>(j));
    }
    int best = -1;
    for (int p : P)
      if (tail[static_cast<size_t>(exec_[p].lane)] == p && p > best) best = p;
    int st = 0;
    if (hinted) {
      st = hLane[j] % S;
    } else if (best >= 0) {
      st = exec_[best].lane;
    } else {
      int unused = -1, oldest = 0;
      for (int k = 0; k < S; ++k) {
        if (count[static_cast<size_t>(k)] == 0) {
          unused = k;
          break;
        }
        if (tail[static_cast<size_t>(k)] < tail[static_cast<size_t>(oldest)]) oldest = k;
      }
      st = j == 0 || tail[0] < 0 ? 0 : unused >= 0 ? unused : oldest;
    }
    std::array<int, 8> cur{};
    if (tail[static_cast<size_t>(st)] >= 0) cur = vc[static_cast<size_t>(tail[static_cast<size_t>(st)])];
    for (auto it = P.rbegin(); it != P.rend(); ++it) {  // latest first: its clock may cover the older ones
      const int p = *it, sp = exec_[p].lane;
      if (sp == st || cur[static_cast<size_t>(sp)] >= pos[static_cast<size_t>(p)]) continue;
      in.waits.push_back(p);
      for (int k = 0; k < 8; ++k) cur[static_cast<size_t>(k)] = std::max(cur[static_cast<size_t>(k)], vc[static_cast<size_t>(p)][static_cast<size_t>(k)]);
    }
    in.lane = st;
    pos[j] = ++count[static_cast<size_t>(st)];
    cur[static_cast<size_t>(st)] = pos[j];
    vc[j] = cur;
    tail[static_cast<size_t>(st)] = static_cast<int>(j);
  }
  numLanes_ = 1;
  for (int k = 0; k < S; ++k)
    if (count[static_cast<size_t>(k)] > 0) numLanes_ = std::max(numLanes_, k + 1);
  tracedLanes_ = hinted;
  auto hb = [&](int a, int b) {  // kernel a happens before kernel b
    return a == b || vc[static_cast<size_t>(b)][static_cast<size_t>(exec_[a].lane)] >= pos[static_cast<size_t>(a)];
  };

  // re-place the temporaries
  struct Tmp {
    ValueId v;
    size_t bytes;
    const std::vector<int>* users;
  };
  std::vector<Tmp> tmps;
  for (ValueId v = 0; v < nv; ++v) {
    if (!reloc[v]) continue;
    size_t n = dtypeSize(m.typeOf(v)->dtype);
    for (Dim d : m.typeOf(v)->shape) n *= static_cast<size_t>(d->value);
    tmps.push_back({v, alignUp(std::max<size_t>(n, 1)), &touching[v]});
  }
  std::stable_sort(tmps.begin(), tmps.end(), [](const Tmp& a, const Tmp& b) { return a.bytes > b.bytes; });
  auto before = [&](const Tmp& a, const Tmp& b) {  // every use of a happens before b's first use
    if (a.users->empty() || b.users->empty()) return true;
    const int first = b.users->front();
    for (int u : *a.users)
      if (!hb(u, first) || u == first) return false;
    return true;
  };
  struct Placed {
    size_t off, size, idx;
  };
  std::vector<Placed> placed;  // by offset
  size_t total = 0;
  for (size_t i = 0; i < tmps.size(); ++i) {
    size_t best = SIZE_MAX, bestGap = SIZE_MAX, cursor = 0;
    for (const Placed& p : placed) {
      if (before(tmps[p.idx], tmps[i]) || before(tmps[i], tmps[p.idx])) continue;
      if (p.off >= cursor) {
        const size_t gap = p.off - cursor;
        if (gap >= tmps[i].bytes && gap < bestGap) {
          best = cursor;
          bestGap = gap;
        }
      }
      cursor = std::max(cursor, p.off + p.size);
    }
    if (best == SIZE_MAX) best = cursor;
    relocOffset_[tmps[i].v] = static_cast<int64_t>(best);
    total = std::max(total, best + tmps[i].bytes);
    const Placed np{best, tmps[i].bytes, i};
    placed.insert(std::upper_bound(placed.begin(), placed.end(), np,
                                   [](const Placed& x, const Placed& y) { return x.off < y.off; }),
                  np);
  }
  tempsBytes_ = total;
  for (ValueId sv : ex.state)
    if (outer[sv] != sv && relocOffset_[outer[sv]] >= 0) relocOffset_[sv] = relocOffset_[outer[sv]] + outerOff[sv];
  return Status();
}

// Turns a call captured on one stream (a chain of the kernels' node segments in program order) into the lanes'
// graph: each kernel's first node depends on the tail of the previous kernel of its lane and on the tails of the
// kernels it waits for, instead of on the kernel just before it. A kernel that enqueued nothing stands for its own
// dependencies. Every node still completes before the graph does.
Status Executable::rewire(hipGraph_t graph, const std::vector<Segment>& segs) const {
  // what depending on kernel j means: its tail node, or (a kernel that enqueued nothing) its own dependencies
  std::vector<std::vector<hipGraphNode_t>> eff(exec_.size());
  std::vector<std::vector<hipGraphNode_t>> laneDeps(exec_.size()), waitDeps(exec_.size());
  std::vector<int> laneLast(static_cast<size_t>(numLanes_), -1);
  for (size_t j = 0; j < exec_.size(); ++j) {
    const Instr& in = exec_[j];
    if (in.kind != OpKind::Kernel) continue;
    const int prev = laneLast[static_cast<size_t>(in.lane)];
    if (prev >= 0) laneDeps[j] = eff[static_cast<size_t>(prev)];
    for (int w : in.waits)
      for (hipGraphNode_t d : eff[static_cast<size_t>(w)])
        if (std::find(laneDeps[j].begin(), laneDeps[j].end(), d) == laneDeps[j].end() &&
            std::find(waitDeps[j].begin(), waitDeps[j].end(), d) == waitDeps[j].end())
          waitDeps[j].push_back(d);
    laneLast[static_cast<size_t>(in.lane)] = static_cast<int>(j);
    if (segs[j].tail) {
      eff[j] = {segs[j].tail};
    } else {
      eff[j] = laneDeps[j];
      eff[j].insert(eff[j].end(), waitDeps[j].begin(), waitDeps[j].end());
    }
  }
  // the capture's chain edges go first, then every lane's own chain, then the waits across lanes: a node's first
  // successor is then the next kernel of its lane, so a runtime that follows first successors to form its
  // streams follows the lanes
  for (size_t j = 0; j < exec_.size(); ++j)
    if (exec_[j].kind == OpKind::Kernel && segs[j].tail && segs[j].before)
      LKRT_TRY(hipStatus(hipGraphRemoveDependencies(graph, &segs[j].before, &segs[j].first, 1), "rewire"));
  for (const auto* deps : {&laneDeps, &waitDeps})
    for (size_t j = 0; j < exec_.size(); ++j)
      if (exec_[j].kind == OpKind::Kernel && segs[j].tail)
        for (hipGraphNode_t d : (*deps)[j])
          LKRT_TRY(hipStatus(hipGraphAddDependencies(graph, &d, &segs[j].first, 1), "rewire"));
  return Status();
}

std::unique_ptr<Executable> Executable::create(std::shared_ptr<const Model> model, const std::vector<ExternalPtr>& ext,
                                               hipStream_t stream, bool useGraphs, Status& st, int maxStreams) {
  std::unique_ptr<Executable> x(new Executable());
  x->model_ = std::move(model);
  const Model& m = *x->model_;
  auto fail = [&](Status s) {
    st = std::move(s);
    return nullptr;
  };
  if (Status v = verifyModel(m); !v) return fail(v);
  for (ValueId v = 0; v < m.numValues(); ++v)
    if (m.typeOf(v)->isTensor()) return fail(Status::error("the model is not in buffer form (run bufferize)"));
  if (Status s = x->lower(m.init, x->init_); !s) return fail(s);
  if (Status s = x->lower(m.exec, x->exec_); !s) return fail(s);
  for (const Op& op : m.exec.ops) x->dynamic_ = x->dynamic_ || op.kind == OpKind::DimRead;
  for (ValueId v : m.exec.args) x->dynamic_ = x->dynamic_ || m.typeOf(v)->isScalar();
  x->graphs_on_ = useGraphs;
  x->relocOffset_.assign(m.numValues(), -1);
  x->skipAlloc_.assign(m.numValues(), 0);
  // Exec-region arenas (a mem.plan, an unhoisted static arena) were planned for one stream: such models keep one.
  bool planned = false;
  for (const Op& op : m.exec.ops)
    planned = planned || op.kind == OpKind::MemPlan || (op.kind == OpKind::BufferAlloc && op.flag("arena"));
  if (!x->dynamic_ && !planned && useGraphs && maxStreams > 1)
    if (Status s = x->schedule(maxStreams); !s) return fail(s);

  // Model arena: every constant, init allocation, persistent buffer, then the workspace.
  const size_t nv = m.numValues();
  std::vector<int64_t> offset(nv, -1);
  struct Upload {
    ValueId v;
    const void* src;
    size_t bytes;
  };
  std::vector<Upload> uploads;
  std::vector<std::pair<ValueId, void*>> deviceExternals;
  size_t off = 0;
  auto take = [&](ValueId v, size_t bytes) {
    offset[v] = static_cast<int64_t>(off);
    off += alignUp(std::max<size_t>(bytes, 1));
  };
  auto staticBytes = [&](Type t, size_t& n) {
    n = dtypeSize(t->dtype);
    for (Dim d : t->shape) {
      if (!d->isConst() || d->value < 0) return false;
      n *= static_cast<size_t>(d->value);
    }
    return true;
  };
  for (const Region* r : {&m.init, &m.exec}) {
    const bool init = r == &m.init;
    for (const Op& op : r->ops) {
      switch (op.kind) {
        case OpKind::ConstInline:
          take(op.results[0], op.data.size());
          uploads.push_back({op.results[0], op.data.data(), op.data.size()});
          break;
        case OpKind::ConstInternal: {
          const Constant* c = m.findConstant(op.name);
          size_t n;
          if (!staticBytes(m.typeOf(op.results[0]), n)) return fail(Status::error("constant '" + op.name + "' has a symbolic shape"));
          if (!c || (!c->bytes && n)) return fail(Status::error("constant '" + op.name + "' has no data"));
          if (c->size != n) return fail(Status::error("constant '" + op.name + "' size doesn't match its type"));
          take(op.results[0], n);
          uploads.push_back({op.results[0], c->bytes, n});
          break;
        }
        case OpKind::ConstExternal: {
          const ExternalPtr* e = nullptr;
          for (const ExternalPtr& q : ext)
            if (q.name == op.name) e = &q;
          size_t n;
          if (!staticBytes(m.typeOf(op.results[0]), n)) return fail(Status::error("external '" + op.name + "' has a symbolic shape"));
          if (!e) return fail(Status::error("no data bound for external constant '" + op.name + "'"));
          if (e->bytes != n) return fail(Status::error("external '" + op.name + "' has " + std::to_string(e->bytes) +
                                                       " bytes, its type " + std::to_string(n)));
          if (e->onDevice) {
            deviceExternals.emplace_back(op.results[0], e->ptr);
          } else {
            take(op.results[0], n);
            uploads.push_back({op.results[0], e->ptr, n});
          }
          break;
        }
        case OpKind::BufferAlloc: {
          if (!init && !op.flag("persistent")) break;  // per-call memory
          if (x->skipAlloc_[op.results[0]]) break;      // its temporaries were re-placed
          size_t n;
          if (!staticBytes(m.typeOf(op.results[0]), n))
            return fail(Status::error("a model-lifetime buffer has a symbolic shape"));
          take(op.results[0], n);
          break;
        }
        case OpKind::DimRead:
          if (init) return fail(Status::error("dim.read in init is not supported"));
          break;
        default:
          break;
      }
    }
  }
  const size_t wsOff = off;
  off += kWorkspaceBytes * static_cast<size_t>(x->numLanes_);
  x->modelArena_ = std::make_unique<Memory>();
  x->modelArena_->n = off;
  if (Status s = hipStatus(hipMalloc(&x->modelArena_->p, off), "hipMalloc (model arena)"); !s) return fail(s);
  x->modelBytes_ = off;
  char* base = static_cast<char*>(x->modelArena_->p);
  if (Status s = hipStatus(hipMemsetAsync(base, 0, off, stream), "hipMemsetAsync"); !s) return fail(s);
  for (int k = 0; k < x->numLanes_; ++k) x->workspace_.push_back(base + wsOff + kWorkspaceBytes * static_cast<size_t>(k));
  x->workspaceBytes_ = kWorkspaceBytes;
  x->fixed_.assign(nv, nullptr);
  for (ValueId v = 0; v < nv; ++v)
    if (offset[v] >= 0) x->fixed_[v] = base + offset[v];
  for (auto& [v, p] : deviceExternals) x->fixed_[v] = static_cast<char*>(p);
  for (const Upload& u : uploads)
    if (u.bytes)
      if (Status s = hipStatus(hipMemcpyAsync(x->fixed_[u.v], u.src, u.bytes, hipMemcpyHostToDevice, stream),
                               "upload");
          !s)
        return fail(s);
  x->scalars_.assign(nv, 0);
  if (Status s = hipStatus(hipHostMalloc(reinterpret_cast<void**>(&x->pinned_), 8), "hipHostMalloc"); !s) return fail(s);
  if (Status s = hipStatus(hipStreamCreateWithFlags(&x->captureStream_, hipStreamNonBlocking), "hipStreamCreate"); !s)
    return fail(s);
  // Multi-stream capture for a model with traced lanes (its stream structure, replayed as the function issued
  // it: 5.65 -> 5.38 ms at 59 tokens, 26.92 -> 26.70 ms at 487, the capture runtime's times). Lanes the scheduler
  // assigns itself keep the single-stream capture and its re-wired edges: captured over lane streams, that
  // schedule's Kokoro-59 call ended its process without a message once, cause not found.
  if (x->numLanes_ > 1 && x->tracedLanes_) {
    x->laneStreams_.push_back(x->captureStream_);
    for (int k = 1; k < x->numLanes_; ++k) {
      hipStream_t ls = nullptr;
      if (Status s = hipStatus(hipStreamCreateWithFlags(&ls, hipStreamNonBlocking), "hipStreamCreate"); !s)
        return fail(s);
      x->laneStreams_.push_back(ls);
    }
    // an event after every kernel another lane waits for, then one fork event and one join event per lane
    x->laneEvents_.assign(x->exec_.size() + 1 + static_cast<size_t>(x->numLanes_), nullptr);
    std::vector<uint8_t> waited(x->exec_.size(), 0);
    for (const Instr& in : x->exec_)
      for (int w : in.waits) waited[static_cast<size_t>(w)] = 1;
    for (size_t j = 0; j < x->laneEvents_.size(); ++j)
      if (j >= x->exec_.size() || waited[j])
        if (Status s = hipStatus(hipEventCreateWithFlags(&x->laneEvents_[j], hipEventDisableTiming), "hipEventCreate");
            !s)
          return fail(s);
  }

  // The device error record is one per GPU, not per call: an error some earlier work recorded and nobody read is
  // cleared here (after that work has finished), so that it is not reported as a failure of this init.
  if (Status s = hipStatus(hipStreamSynchronize(stream), "init"); !s) return fail(s);
  (void)deviceErrors();
  // init: model-lifetime results become the exec state
  std::vector<char*> slot(x->fixed_);
  std::vector<int64_t> sv(m.dims().numSymbols(), kUnbound);
  std::vector<TensorOut> initOut;
  Bump none;
  if (Status s = x->interpret(x->init_, slot, sv, none, stream, &initOut); !s) return fail(Status::error("init: " + s.message()));
  if (!none.blocks.empty()) return fail(Status::error("init allocated per-call memory"));
  for (size_t i = 0; i < m.exec.state.size(); ++i) x->fixed_[m.exec.state[i]] = static_cast<char*>(initOut[i].data);
  for (const TensorOut& o : initOut) x->state_.push_back(static_cast<char*>(o.data));
  if (x->tempsBytes_) {
    x->temps_ = std::make_unique<Memory>();
    x->temps_->n = x->tempsBytes_;
    if (Status s = hipStatus(hipMalloc(&x->temps_->p, x->tempsBytes_), "hipMalloc (temporaries)"); !s) return fail(s);
    x->modelBytes_ += x->tempsBytes_;
  }
  for (ValueId v = 0; v < nv; ++v)
    if (x->relocOffset_[v] >= 0) x->fixed_[v] = static_cast<char*>(x->temps_->p) + x->relocOffset_[v];
  if (Status s = hipStatus(hipStreamSynchronize(stream), "init"); !s) return fail(s);
  if (Status s = deviceErrors(); !s) return fail(Status::error("init: " + s.message()));
  st = Status();
  return x;
}

Status Executable::run(const std::vector<TensorIn>& inputs, std::vector<TensorOut>& outputs, hipStream_t stream,
                       bool sync) {
  const Model& m = *model_;
  const Region& ex = m.exec;
  std::vector<int64_t> sv;
  LKRT_TRY(bindInputs(inputs, sv));
  std::vector<char*> slot(fixed_);
  for (size_t i = 0; i < inputs.size(); ++i) {
    const ValueId v = ex.args[i];
    if (m.typeOf(v)->isScalar()) std::memcpy(&scalars_[v], inputs[i].data, 8);
    else slot[v] = static_cast<char*>(inputs[i].data);
  }
  bool eager = !graphs_on_ || dynamic_;
  std::vector<int64_t> key;
  if (!eager) {
    key = sv;
    for (size_t i = 0; i < inputs.size(); ++i)
      if (ex.isMutable(i)) key.push_back(reinterpret_cast<int64_t>(inputs[i].data));
    auto it = graphs_.find(key);
    eager = it != graphs_.end() && !it->second->exec;  // a binding whose capture failed runs eagerly
  }
  if (eager) {
    if (eager_.blocks.size() > 1) {  // coalesce last call's overflow blocks into one
      LKRT_TRY(hipStatus(hipDeviceSynchronize(), "call arena"));
      const size_t cap = eager_.capacity();
      eager_.blocks.clear();
      Status st;
      if (!eager_.alloc(cap, st)) return st;
    }
    eager_.used = 0;
    LKRT_TRY(interpret(exec_, slot, sv, eager_, stream, &outputs));
  } else {
    auto it = graphs_.find(key);
    if (it == graphs_.end()) {
      auto g = std::make_unique<Graph>();
      size_t callB = 0, inB = 0;
      LKRT_TRY(callBytes(sv, callB));
      std::vector<size_t> inSize(inputs.size(), 0);
      for (size_t i = 0; i < inputs.size(); ++i) {
        if (ex.isMutable(i)) continue;
        size_t n = dtypeSize(inputs[i].dtype);
        for (int64_t d : inputs[i].shape) n *= static_cast<size_t>(d);
        inSize[i] = n;
        inB += alignUp(std::max<size_t>(n, 1));
      }
      g->mem = std::make_unique<Memory>();
      g->mem->n = inB + callB;
      LKRT_TRY(hipStatus(hipMalloc(&g->mem->p, std::max<size_t>(g->mem->n, 1)), "hipMalloc (call block)"));
      char* p = static_cast<char*>(g->mem->p);
      g->inputs.assign(inputs.size(), nullptr);
      for (size_t i = 0; i < inputs.size(); ++i) {
        if (ex.isMutable(i)) continue;
        g->inputs[i] = p;
        slot[ex.args[i]] = p;
        if (inSize[i])
          LKRT_TRY(hipStatus(hipMemcpyAsync(p, inputs[i].data, inSize[i], hipMemcpyDeviceToDevice, stream), "input copy"));
        p += alignUp(std::max<size_t>(inSize[i], 1));
      }
      // A non-owning view of the block's call region: the warm-up run and the capture walk allocate the same
      // addresses.
      Bump view;
      auto region = std::make_unique<Memory>();
      region->p = p;
      region->n = callB;
      view.blocks.push_back(std::move(region));
      std::vector<char*> warmSlot(slot);
      std::vector<int64_t> warmSv(sv);
      Status ws = interpret(exec_, warmSlot, warmSv, view, stream, &g->outputs);
      if (ws && view.blocks.size() == 1) {
        view.used = 0;
        std::vector<char*> capSlot(slot);
        std::vector<int64_t> capSv(sv);
        std::vector<TensorOut> capOut;
        const bool multi = !laneStreams_.empty();
        std::vector<Segment> segs(numLanes_ > 1 && !multi ? exec_.size() : 0);
        LKRT_TRY(hipStatus(hipStreamBeginCapture(captureStream_, hipStreamCaptureModeThreadLocal), "capture"));
        Status cs;
        const size_t fork = exec_.size();
        if (multi) {  // every lane joins the capture at its start
          cs = hipStatus(hipEventRecord(laneEvents_[fork], captureStream_), "capture fork");
          for (size_t k = 1; cs && k < laneStreams_.size(); ++k)
            cs = hipStatus(hipStreamWaitEvent(laneStreams_[k], laneEvents_[fork], 0), "capture fork");
        }
        if (cs)
          cs = interpret(exec_, capSlot, capSv, view, captureStream_, &capOut, segs.empty() ? nullptr : &segs, multi);
        if (multi)  // and rejoins it at its end
          for (size_t k = 1; k < laneStreams_.size(); ++k) {
            if (cs) cs = hipStatus(hipEventRecord(laneEvents_[fork + k], laneStreams_[k]), "capture join");
            if (cs) cs = hipStatus(hipStreamWaitEvent(captureStream_, laneEvents_[fork + k], 0), "capture join");
          }
        hipGraph_t graph = nullptr;
        const hipError_t ee = hipStreamEndCapture(captureStream_, &graph);
        if (cs && ee == hipSuccess && !segs.empty()) cs = rewire(graph, segs);
        if (cs && ee == hipSuccess) {
          g->graph = graph;
          LKRT_TRY(hipStatus(hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate"));
        } else {
          if (graph) (void)hipGraphDestroy(graph);
          (void)hipGetLastError();
          if (!cs) ws = cs;
        }
      }
      view.blocks[0]->p = nullptr;  // not owned
      LKRT_TRY(ws);
      outputs = g->outputs;
      graphs_[key] = std::move(g);
    } else {
      Graph& g = *it->second;
      for (size_t i = 0; i < inputs.size(); ++i) {
        if (!g.inputs[i]) continue;
        size_t n = dtypeSize(inputs[i].dtype);
        for (int64_t d : inputs[i].shape) n *= static_cast<size_t>(d);
        if (n)
          LKRT_TRY(hipStatus(hipMemcpyAsync(g.inputs[i], inputs[i].data, n, hipMemcpyDeviceToDevice, stream),
                             "input copy"));
      }
      LKRT_TRY(hipStatus(hipGraphLaunch(g.exec, stream), "hipGraphLaunch"));
      outputs = g.outputs;
    }
  }
  if (sync) {
    LKRT_TRY(hipStatus(hipStreamSynchronize(stream), "run"));
    LKRT_TRY(deviceErrors());
  }
  return Status();
}

}  // namespace lkrt
