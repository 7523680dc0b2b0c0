// Instances of the storage-changing step with destination storage ST_S32.
#include "mdq_dispatch.h"

namespace mdq {
hipError_t launch_tr_s32(int src, const MdqDesc *d, int n, long long tiles, int gt, int log2b, bool sr,
                       unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    return launch_tr_to<ST_S32>(src, d, n, tiles, gt, log2b, sr, prof, sa, views, s);
}
}  // namespace mdq
