// mdq_dispatch.h -- run-time (grad dtype, block size, rounding) -> template
// instance dispatch.  Included by mdq_kernels_<storage>.hip (steps that keep
// their storage, every block size), mdq_kernels_one_<storage>.hip (the same
// for one tensor whose descriptor is a kernel argument) and
// mdq_kernels_tr_<storage>.hip (steps into that storage from another one,
// block sizes 64 / 128 / 256), so the instance sets compile in parallel.
#pragma once
#include "mdq_kernel.h"
#include "mdq_launch.h"

namespace mdq {

template <int SRC, int DST, int GT, int LOG2B, bool SR>
static hipError_t launch_one(const MdqDesc *d, int n, long long tiles, unsigned long long *prof,
                             const StepArgs &sa, bool views, hipStream_t s)
{
    // the compact tile_begin array follows the n descriptors in the same buffer
    const long long *tb = reinterpret_cast<const long long *>(d + n);
    if (views)
        hipLaunchKernelGGL((mdq_step_kernel<SRC, DST, GT, LOG2B, SR, true>), dim3((unsigned)tiles),
                           dim3(Cfg<LOG2B>::THREADS), 0, s, d, tb, n, prof, sa);
    else
        hipLaunchKernelGGL((mdq_step_kernel<SRC, DST, GT, LOG2B, SR, false>), dim3((unsigned)tiles),
                           dim3(Cfg<LOG2B>::THREADS), 0, s, d, tb, n, prof, sa);
    return hipGetLastError();
}

// Every block size 1 .. 1024 for a step that keeps its storage.
template <int ST, int GT, bool SR>
static hipError_t launch_b(int log2b, const MdqDesc *d, int n, long long tiles,
                           unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    switch (log2b) {
    case 0: return launch_one<ST, ST, GT, 0, SR>(d, n, tiles, prof, sa, views, s);
    case 1: return launch_one<ST, ST, GT, 1, SR>(d, n, tiles, prof, sa, views, s);
    case 2: return launch_one<ST, ST, GT, 2, SR>(d, n, tiles, prof, sa, views, s);
    case 3: return launch_one<ST, ST, GT, 3, SR>(d, n, tiles, prof, sa, views, s);
    case 4: return launch_one<ST, ST, GT, 4, SR>(d, n, tiles, prof, sa, views, s);
    case 5: return launch_one<ST, ST, GT, 5, SR>(d, n, tiles, prof, sa, views, s);
    case 6: return launch_one<ST, ST, GT, 6, SR>(d, n, tiles, prof, sa, views, s);
    case 7: return launch_one<ST, ST, GT, 7, SR>(d, n, tiles, prof, sa, views, s);
    case 8: return launch_one<ST, ST, GT, 8, SR>(d, n, tiles, prof, sa, views, s);
    case 9: return launch_one<ST, ST, GT, 9, SR>(d, n, tiles, prof, sa, views, s);
    case 10: return launch_one<ST, ST, GT, 10, SR>(d, n, tiles, prof, sa, views, s);
    default: return hipErrorInvalidValue;
    }
}

template <int ST>
static hipError_t launch_for(const MdqDesc *d, int n, long long tiles, int gt, int log2b, bool sr,
                             unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    switch (gt) {
    case GT_F32: return sr ? launch_b<ST, GT_F32, true>(log2b, d, n, tiles, prof, sa, views, s)
                           : launch_b<ST, GT_F32, false>(log2b, d, n, tiles, prof, sa, views, s);
    case GT_BF16: return sr ? launch_b<ST, GT_BF16, true>(log2b, d, n, tiles, prof, sa, views, s)
                            : launch_b<ST, GT_BF16, false>(log2b, d, n, tiles, prof, sa, views, s);
    case GT_F16: return sr ? launch_b<ST, GT_F16, true>(log2b, d, n, tiles, prof, sa, views, s)
                           : launch_b<ST, GT_F16, false>(log2b, d, n, tiles, prof, sa, views, s);
    default: return hipErrorInvalidValue;
    }
}

// One tensor, its descriptor a kernel argument (mdq_step_kernel_one), every block size.
template <int ST, int GT, int LOG2B, bool SR>
static hipError_t launch_arg(const MdqDesc &d, long long tiles, unsigned long long *prof, const StepArgs &sa,
                             hipStream_t s)
{
    hipLaunchKernelGGL((mdq_step_kernel_one<ST, GT, LOG2B, SR>), dim3((unsigned)tiles), dim3(Cfg<LOG2B>::THREADS),
                       0, s, d, prof, sa);
    return hipGetLastError();
}

template <int ST, int GT, bool SR>
static hipError_t launch_b_arg(int log2b, const MdqDesc &d, long long tiles, unsigned long long *prof,
                               const StepArgs &sa, hipStream_t s)
{
    switch (log2b) {
    case 0: return launch_arg<ST, GT, 0, SR>(d, tiles, prof, sa, s);
    case 1: return launch_arg<ST, GT, 1, SR>(d, tiles, prof, sa, s);
    case 2: return launch_arg<ST, GT, 2, SR>(d, tiles, prof, sa, s);
    case 3: return launch_arg<ST, GT, 3, SR>(d, tiles, prof, sa, s);
    case 4: return launch_arg<ST, GT, 4, SR>(d, tiles, prof, sa, s);
    case 5: return launch_arg<ST, GT, 5, SR>(d, tiles, prof, sa, s);
    case 6: return launch_arg<ST, GT, 6, SR>(d, tiles, prof, sa, s);
    case 7: return launch_arg<ST, GT, 7, SR>(d, tiles, prof, sa, s);
    case 8: return launch_arg<ST, GT, 8, SR>(d, tiles, prof, sa, s);
    case 9: return launch_arg<ST, GT, 9, SR>(d, tiles, prof, sa, s);
    case 10: return launch_arg<ST, GT, 10, SR>(d, tiles, prof, sa, s);
    default: return hipErrorInvalidValue;
    }
}

template <int ST>
static hipError_t launch_for_arg(const MdqDesc &d, long long tiles, int gt, int log2b, bool sr,
                                 unsigned long long *prof, const StepArgs &sa, hipStream_t s)
{
    switch (gt) {
    case GT_F32: return sr ? launch_b_arg<ST, GT_F32, true>(log2b, d, tiles, prof, sa, s)
                           : launch_b_arg<ST, GT_F32, false>(log2b, d, tiles, prof, sa, s);
    case GT_BF16: return sr ? launch_b_arg<ST, GT_BF16, true>(log2b, d, tiles, prof, sa, s)
                            : launch_b_arg<ST, GT_BF16, false>(log2b, d, tiles, prof, sa, s);
    case GT_F16: return sr ? launch_b_arg<ST, GT_F16, true>(log2b, d, tiles, prof, sa, s)
                           : launch_b_arg<ST, GT_F16, false>(log2b, d, tiles, prof, sa, s);
    default: return hipErrorInvalidValue;
    }
}

// Storage-changing steps: block sizes 64, 128 and 256 (TRANSITION_LOG2B_MIN .. MAX).
template <int SRC, int DST, int GT, bool SR>
static hipError_t launch_b_tr(int log2b, const MdqDesc *d, int n, long long tiles,
                              unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    static_assert(TRANSITION_LOG2B_MIN == 6 && TRANSITION_LOG2B_MAX == 8, "instances below");
    switch (log2b) {
    case 6: return launch_one<SRC, DST, GT, 6, SR>(d, n, tiles, prof, sa, views, s);
    case 7: return launch_one<SRC, DST, GT, 7, SR>(d, n, tiles, prof, sa, views, s);
    case 8: return launch_one<SRC, DST, GT, 8, SR>(d, n, tiles, prof, sa, views, s);
    default: return hipErrorInvalidValue;
    }
}

template <int SRC, int DST>
static hipError_t launch_tr_pair(const MdqDesc *d, int n, long long tiles, int gt, int log2b, bool sr,
                                 unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    switch (gt) {
    case GT_F32: return sr ? launch_b_tr<SRC, DST, GT_F32, true>(log2b, d, n, tiles, prof, sa, views, s)
                           : launch_b_tr<SRC, DST, GT_F32, false>(log2b, d, n, tiles, prof, sa, views, s);
    case GT_BF16: return sr ? launch_b_tr<SRC, DST, GT_BF16, true>(log2b, d, n, tiles, prof, sa, views, s)
                            : launch_b_tr<SRC, DST, GT_BF16, false>(log2b, d, n, tiles, prof, sa, views, s);
    case GT_F16: return sr ? launch_b_tr<SRC, DST, GT_F16, true>(log2b, d, n, tiles, prof, sa, views, s)
                           : launch_b_tr<SRC, DST, GT_F16, false>(log2b, d, n, tiles, prof, sa, views, s);
    default: return hipErrorInvalidValue;
    }
}

// All sources other than DST, for one destination storage.
template <int DST>
static hipError_t launch_tr_to(int src, const MdqDesc *d, int n, long long tiles, int gt, int log2b, bool sr,
                               unsigned long long *prof, const StepArgs &sa, bool views, hipStream_t s)
{
    switch (src) {
    case ST_P4:
        if constexpr (DST != ST_P4) return launch_tr_pair<ST_P4, DST>(d, n, tiles, gt, log2b, sr, prof, sa, views, s);
        break;
    case ST_S8:
        if constexpr (DST != ST_S8) return launch_tr_pair<ST_S8, DST>(d, n, tiles, gt, log2b, sr, prof, sa, views, s);
        break;
    case ST_S16:
        if constexpr (DST != ST_S16) return launch_tr_pair<ST_S16, DST>(d, n, tiles, gt, log2b, sr, prof, sa, views, s);
        break;
    case ST_S32:
        if constexpr (DST != ST_S32) return launch_tr_pair<ST_S32, DST>(d, n, tiles, gt, log2b, sr, prof, sa, views, s);
        break;
    default:
        break;
    }
    return hipErrorInvalidValue;
}

}  // namespace mdq
