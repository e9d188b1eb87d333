// prefill.hip -- block-scaled MFMA prefill on requantized activations.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

bool prefill_supported(uint32_t, uint32_t, uint32_t) { return false; }
hipError_t launch_prefill(const PrefillArgs&, int) { return hipErrorNotSupported; }

}  // namespace mx4
