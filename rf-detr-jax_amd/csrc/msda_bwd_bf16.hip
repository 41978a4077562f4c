// Backward kernels for a bf16 value map (band kernel, partial sums, sorted gather). A translation
// unit of its own so the build compiles them in parallel.
#include "msda_launch.h"

namespace msda_host {
template int dispatch_bwd_band<msda::bf16_t>(int, const msda::BandParams&, int, int, int, hipStream_t, bool);
template int launch_part_sum<msda::bf16_t>(const float*, int, int64_t, int64_t, void*, int, int, hipStream_t, const float*, float*, int, int64_t);
template int dispatch_bwd_gather<msda::bf16_t>(int, bool, const msda::GatherParams&, int, int, int, hipStream_t);
}  // namespace msda_host
