// Device-side error record: how a kernel that finds invalid data mid-graph reports it. The reference's host kernels
// set ExecCtx::error and the runtime turns GPU faults into an error at the next synchronisation (takeGpuError,
// lariaus/lokinfer src/runtime/executable.cpp:850-852, gpu.cpp:382-387). A device kernel cannot stop the graph, so
// it writes a neutral value (NaN, no cache row) and records the first error here: {code, detail} on each GPU,
// claimed with a compare-and-swap so the first error wins. lk_take_device_error reads and clears it at a
// synchronisation point; the Python layer raises it as LokinferError.
#include <mutex>

#include "common.h"
#include "lokinfer_hip.h"

namespace {

static __device__ __align__(16) unsigned long long gErrorWords[2];  // [code, detail]

constexpr int kMaxDevices = 64;
std::mutex gMu;
unsigned long long* gRecord[kMaxDevices] = {};

}  // namespace

namespace lkh {

unsigned long long* deviceErrorRecord() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(gMu);
  if (!gRecord[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(gErrorWords)) != hipSuccess) {
      (void)hipGetLastError();  // do not leave the failure for the caller's launch check
      return nullptr;
    }
    gRecord[dev] = static_cast<unsigned long long*>(p);
  }
  return gRecord[dev];
}

}  // namespace lkh

extern "C" {

int lk_take_device_error(int64_t* detail) {
  unsigned long long* rec = lkh::deviceErrorRecord();
  if (!rec) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  unsigned long long host[2] = {0, 0};
  if (hipMemcpy(host, rec, sizeof host, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  if (host[0] != 0) {
    const unsigned long long zero[2] = {0, 0};
    if (hipMemcpy(rec, zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess) return -1;
  }
  if (detail) *detail = static_cast<int64_t>(host[1]);
  return static_cast<int>(host[0]);
}

const char* lk_device_error_message(int code) {
  switch (code) {
    case 0: return "no error";
    case LK_DEVERR_EXCHANGE_TIMEOUT:
      return "a persistent kernel's cross-workgroup exchange timed out (peer workgroups made no progress); its "
             "outputs are NaN";
    case LK_DEVERR_POSITION: return "a position is outside the KV cache; no cache row was written and the output is NaN";
    case LK_DEVERR_INDEX: return "an index (token id) is out of range; its row is NaN";
    case LK_DEVERR_DURATIONS: return "the durations cover fewer frames than the frame count; the missing rows are NaN";
    case LK_DEVERR_AUDIO_ROWS: return "more audio-pad ids than audio embedding rows; the extra rows are NaN";
    default: return "unknown device error";
  }
}

}  // extern "C"
