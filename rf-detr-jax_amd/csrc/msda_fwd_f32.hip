// Forward kernels for an f32 value map: the core (msda_fwd) and the fused-prologue variants
// (msda_fused_fwd). A translation unit of its own so the build compiles the variants in parallel.
#include "msda_launch.h"

namespace msda_host {
template int dispatch_fwd<float>(int, int, bool, const msda::SampleParams&, int, int, int, hipStream_t);
}  // namespace msda_host
