// Kokoro token-rate front end and signal path on the GPU (the reference runs these as host CPU kernels inside
// its GPU graph; here they stay on the device so a forward needs no host round trips).
#include "common.h"

namespace lkh {

void registerFrontendKernels() {}

}  // namespace lkh
