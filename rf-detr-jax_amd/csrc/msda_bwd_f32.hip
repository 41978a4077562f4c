// Backward kernels for an f32 value map (band kernel, partial sums, sorted gather). A translation
// unit of its own so the build compiles them in parallel.
#include "msda_launch.h"

namespace msda_host {
template int dispatch_bwd_band<float>(int, const msda::BandParams&, int, int, int, hipStream_t, bool);
template int launch_part_sum<float>(const float*, int, int64_t, int64_t, void*, int, int, hipStream_t, const float*, float*, int, int64_t);
template int dispatch_bwd_gather<float>(int, bool, const msda::GatherParams&, int, int, int, hipStream_t);
}  // namespace msda_host
