// Instances of the one-tensor step (descriptor as a kernel argument) for storage class ST_S16.
#include "mdq_dispatch.h"

namespace mdq {
hipError_t launch_one_s16(const MdqDesc &d, long long tiles, int gt, int log2b, bool sr,
                         unsigned long long *prof, const StepArgs &sa, hipStream_t s)
{
    return launch_for_arg<ST_S16>(d, tiles, gt, log2b, sr, prof, sa, s);
}
}  // namespace mdq
