// Instances of the fused step for storage class ST_S32.
#include "mdq_dispatch.h"

namespace mdq {
hipError_t launch_s32(const MdqDesc *d, int n, long long tiles, int gt, int log2b, bool sr,
                      unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    return launch_for<ST_S32>(d, n, tiles, gt, log2b, sr, prof, sa, views, s);
}
}  // namespace mdq
