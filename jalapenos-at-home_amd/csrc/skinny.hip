// skinny.hip -- exact skinny kernel (2 <= M <= 16) on bf16 MFMA.
#include "mx4_device.h"
#include "mx4_kernels.h"

namespace mx4 {

bool skinny_supported(uint32_t, uint32_t) { return false; }
hipError_t launch_skinny(const GemvArgs&, int) { return hipErrorNotSupported; }

}  // namespace mx4
