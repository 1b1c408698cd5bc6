// Chunked gated-delta prefill (placeholder until the MFMA kernel lands): refuses to run.
#include "ha_kernels.h"
namespace ha {
hipError_t launch_gdn_chunked(const GdnArgs&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace ha
