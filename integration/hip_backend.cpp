// The binding a lokinfer maintainer adds to the reference's tree (e.g. src/runtime/hip_backend.cpp in
// lariaus/lokinfer) to run its compiled GPU path on the MI355X kernels: every kernel of liblokinfer_hip.so
// (include/lokinfer_hip.h) is registered under its own name in the reference's registry
// (include/lokinfer/runtime/kernel.h:56-72), with the reference's KernelEntry lifecycle:
//   prepare  looks the kernel up once and counts the op's float attributes (the reference's KernelArgs carries no
//            float count; the executable fills `floats` with the op's non-structural float attrs in name order,
//            src/runtime/executable.cpp:406-447), kept as the kernel's state;
//   run      calls lk_run_kernel with device pointers (BufRef {buffer, offset} from the HIP context) and the HIP
//            stream and workspace of the context;
//   destroy  frees the state.
// The HIP context (one stream, a zeroed workspace) replaces the Metal GpuContext; the runtime owns it and hands it
// out through hipContextOf. This file is compiled against the reference's headers by tests/test_integration.py.
#include <string>

#include "lokinfer/ir/ir.h"
#include "lokinfer/runtime/kernel.h"
#include "lokinfer_hip.h"

namespace lk::rt {

// The HIP counterpart of GpuContext the runtime would hold (its stream, and a device workspace whose first 64 KiB
// are zero, for kernels that merge partial results).
struct HipContext {
  void* stream;
  void* workspace;
  uint64_t workspaceBytes;
};
HipContext* hipContextOf(GpuContext* gpu);  // provided by the runtime's HIP context

namespace {

struct HipKernelState {
  const lk_kernel* kernel;
  uint32_t numFloats;
};

Status prepareHip(PrepareCtx&, const Op& op, void** state) {
  const lk_kernel* k = lk_find_kernel(op.name.c_str());
  if (!k) return Status::error("no MI355X kernel '" + op.name + "'");
  uint32_t floats = 0;
  for (const NamedAttr& a : op.attrs) {
    if (isStructuralAttr(a.name)) continue;
    if (std::holds_alternative<double>(a.attr.value)) floats += 1;
    else if (auto* v = std::get_if<Attr::Floats>(&a.attr.value)) floats += static_cast<uint32_t>(v->size());
  }
  *state = new HipKernelState{k, floats};
  return Status::ok();
}

void runHip(ExecCtx& ctx, const KernelArgs& a) {
  const auto* s = static_cast<const HipKernelState*>(a.state);
  HipContext* h = hipContextOf(ctx.gpu);
  // device pointers: the HIP context keeps the device address in BufRef::mtlBuffer (plus the slot's offset);
  // operands without a buffer (host scalars) pass their host slot, as the reference does
  void* ptrs[64];
  if (a.numPtrs > 64) {
    ctx.error = "MI355X kernel: too many operands";
    return;
  }
  for (uint32_t i = 0; i < a.numPtrs; ++i)
    ptrs[i] = a.bufs && a.bufs[i].mtlBuffer ? static_cast<char*>(a.bufs[i].mtlBuffer) + a.bufs[i].offset : a.ptrs[i];
  if (lk_run_kernel(s->kernel, ptrs, a.numPtrs, a.ints, a.numInts, a.floats, s->numFloats, h->workspace,
                    h->workspaceBytes, h->stream) != 0) {
    thread_local std::string message;  // ExecCtx::error must outlive the call
    message = lk_last_error();
    ctx.error = message.c_str();
  }
}

void destroyHip(void* state) { delete static_cast<HipKernelState*>(state); }

}  // namespace

// Called from registerBuiltinKernels() in place of the Metal kernels' registration.
void registerHipKernels() {
  lk_init();
  for (int i = 0; i < lk_num_kernels(); ++i) {
    const char* name = lk_kernel_name_at(i);
    registerKernel({name, lk_kernel_is_gpu(lk_find_kernel(name)) ? Device::Gpu : Device::Cpu, prepareHip, runHip,
                    destroyHip});
  }
}

}  // namespace lk::rt
