// Prefill attention on MFMA: not built yet. The C ABI reports it, and the
// step planner routes every run through the paged decode kernel meanwhile.
#include "device.hpp"
#include "kernels.hpp"

namespace ember::hip {

hipError_t launch_prefill(const EmberPrefillArgs &, hipStream_t) { return hipErrorNotSupported; }

}  // namespace ember::hip
