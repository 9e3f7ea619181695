// The MI355X executable: runs a compiled (buffer-form) model on one HIP stream.
//
// Replaces the reference's Executable (lariaus/lokinfer include/lokinfer/runtime/runtime.h:84-124,
// src/runtime/executable.cpp:567-1144) and its Metal GpuContext (src/runtime/gpu_internal.h:53-290):
//  - one hipMalloc'd model arena per executable holds every constant (internal constants uploaded once at create),
//    init's allocations, persistent state and the kernel workspace, zeroed once;
//  - per call, memory comes from a call arena that grows by whole hipMallocs and is reused: a statically shaped
//    call (no dim.read, no host scalar inputs) runs from one exactly sized block per input-shape binding, and after
//    its first (eager) run is captured into a hipGraph that later calls replay after copying the inputs into the
//    block's input buffers;
//  - kernels are the registry's (lkh::findKernel), called with the reference's argument convention;
//  - a statically shaped exec region's captured graph can run its independent branches concurrently: kernels are
//    assigned to up to 8 lanes from their data dependencies (a kernel continues the lane of its latest predecessor
//    when it can, else takes an idle one), the call is captured on one stream and its graph's edges are re-wired
//    from the lanes (each kernel after its lane's previous kernel and the kernels of other lanes it depends on),
//    and the per-call temporaries the compiler placed in a static arena are re-placed so that two buffers share
//    bytes only when every use of one happens before the other is written under that schedule. Every call still
//    enqueues on the caller's one stream;
//  - a kernel's ExecCtx::error becomes the call's Status, and so does a data error a kernel recorded on the device
//    (read at the call's synchronisation, the reference's takeGpuError).
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "ir.h"

namespace lkrt {

struct ExternalPtr {
  std::string name;
  void* ptr;
  size_t bytes;
  bool onDevice;  // false: host memory, uploaded into the model arena at create
};

struct TensorIn {
  void* data;  // device pointer (host pointer to 8 bytes for a scalar)
  std::vector<int64_t> shape;
  DType dtype;
};

struct TensorOut {
  void* data;  // device memory owned by the executable, valid until its next call
  std::vector<int64_t> shape;
  DType dtype;
};

class Executable {
 public:
  ~Executable();
  // `model` must be in buffer form (after bufferize). Uploads constants and runs init on `stream`.
  static std::unique_ptr<Executable> create(std::shared_ptr<const Model> model, const std::vector<ExternalPtr>& ext,
                                            hipStream_t stream, bool useGraphs, Status& st, int maxStreams = 1);
  // Enqueues one call on `stream`. With `sync`, waits for it and reports device-side data errors.
  Status run(const std::vector<TensorIn>& inputs, std::vector<TensorOut>& outputs, hipStream_t stream, bool sync);

  const Model& model() const { return *model_; }
  size_t modelArenaBytes() const { return modelBytes_; }
  size_t callArenaBytes() const;
  int graphsCaptured() const { return static_cast<int>(graphs_.size()); }
  // Address of init's i-th result (the exec state), in the model arena or an external's memory.
  const void* stateData(size_t i) const { return i < state_.size() ? state_[i] : nullptr; }
  int lanesUsed() const { return numLanes_; }
  std::string strategy() const;

  struct Instr;
  struct Segment;

 private:
  Executable() = default;
  struct Memory {
    void* p = nullptr;
    size_t n = 0;
    Memory() = default;
    Memory(const Memory&) = delete;
    Memory& operator=(const Memory&) = delete;
    ~Memory();
  };
  struct Bump {  // a bump allocator over one or more blocks; reset per call
    std::vector<std::unique_ptr<Memory>> blocks;
    size_t used = 0;
    char* alloc(size_t bytes, Status& st);
    size_t capacity() const;
  };
  struct Graph {
    std::unique_ptr<Memory> mem;  // inputs, then the call's memory
    std::vector<char*> inputs;    // staging buffer of each non-mutable input
    std::vector<TensorOut> outputs;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
  };

  Status lower(const Region& r, std::vector<Instr>& out);
  // lane assignment + temporaries re-placement for a statically shaped exec region
  Status schedule(int maxLanes);
  // the lanes as the edges of a graph captured on one stream
  Status rewire(hipGraph_t graph, const std::vector<Segment>& segs) const;
  Status bindInputs(const std::vector<TensorIn>& in, std::vector<int64_t>& sv) const;
  Status interpret(const std::vector<Instr>& code, std::vector<char*>& slot, std::vector<int64_t>& sv, Bump& mem,
                   hipStream_t s, std::vector<TensorOut>* outs, std::vector<Segment>* segs = nullptr,
                   bool laneStreams = false);
  // bytes the exec region allocates for a binding (statically shaped calls only)
  Status callBytes(std::vector<int64_t> sv, size_t& bytes) const;

  std::shared_ptr<const Model> model_;
  std::vector<Instr> init_, exec_;
  std::unique_ptr<Memory> modelArena_;
  size_t modelBytes_ = 0;
  std::vector<void*> workspace_;  // one per lane
  size_t workspaceBytes_ = 0;
  int numLanes_ = 1;
  bool tracedLanes_ = false;  // lanes taken from the trace's stream structure (lane / seq / after attributes)
  std::unique_ptr<Memory> temps_;   // re-placed per-call temporaries
  size_t tempsBytes_ = 0;
  std::vector<int64_t> relocOffset_;  // exec state value -> offset in temps_ (-1: not re-placed)
  std::vector<uint8_t> skipAlloc_;    // init arena allocs whose every byte was re-placed
  std::vector<char*> fixed_;          // value -> model-lifetime address (constants, state, persistent buffers)
  std::vector<char*> state_;          // init's results as init wrote them
  std::vector<int64_t> scalars_;      // host slots of scalar exec inputs
  bool graphs_on_ = false;
  bool dynamic_ = false;              // exec has dim.read or scalar inputs: always eager
  Bump eager_;
  std::map<std::vector<int64_t>, std::unique_ptr<Graph>> graphs_;
  hipStream_t captureStream_ = nullptr;
  // multi-stream capture: lane k's kernels are captured on laneStreams_[k] (0: captureStream_), a cross-lane wait
  // as an event recorded after the waited kernel (laneEvents_[kernel]) and waited for on the waiting lane
  std::vector<hipStream_t> laneStreams_;
  std::vector<hipEvent_t> laneEvents_;  // per exec instruction (null: nothing waits for it), then fork / joins
  int64_t* pinned_ = nullptr;         // dim.read landing slot
};

// bake-init (the reference's runtime/bake_init.h): runs `model`'s init once (externals bound) and returns a copy
// in which every init result that is computed data (a plain buffer.alloc written by init kernels, or a view of one)
// is a const.internal holding that data, on the device of the kernel that wrote it; init ops nothing needs any more
// are removed. Left alone: arena / persistent / output buffers, constants, and the whole model when init defines
// symbols (dim.read, mem.plan).
struct BakeStats {
  size_t baked = 0, bakedBytes = 0, initOpsBefore = 0, initOpsAfter = 0;
};
std::unique_ptr<Model> bakeInit(std::shared_ptr<const Model> model, const std::vector<ExternalPtr>& ext,
                                hipStream_t stream, BakeStats* stats, Status& st);

}  // namespace lkrt
