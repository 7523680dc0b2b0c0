// mdq_launch.h -- host entry points of the kernel instances (one per storage
// class) and of the math self-check kernels.
#pragma once
#include <hip/hip_runtime.h>

#include "mdq_desc.h"

namespace mdq {

// views: some tensor of the launch has p or grads off their 128-byte lines (and aligned codes),
// so the launch takes the kernel variant with the staged tile modes.
hipError_t launch_p4(const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);
hipError_t launch_s8(const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);
hipError_t launch_s16(const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);
hipError_t launch_s32(const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);

// One tensor whose descriptor travels as a kernel argument (no table in device memory: the
// launch of a call on a stream that captures a HIP graph).
hipError_t launch_one_p4(const MdqDesc &, long long, int, int, bool, unsigned long long *, const StepArgs &, hipStream_t);
hipError_t launch_one_s8(const MdqDesc &, long long, int, int, bool, unsigned long long *, const StepArgs &, hipStream_t);
hipError_t launch_one_s16(const MdqDesc &, long long, int, int, bool, unsigned long long *, const StepArgs &, hipStream_t);
hipError_t launch_one_s32(const MdqDesc &, long long, int, int, bool, unsigned long long *, const StepArgs &, hipStream_t);

// Storage-changing steps (codes read in storage src, written in the destination
// storage of the function name): block sizes 2^TRANSITION_LOG2B_MIN ..
// 2^TRANSITION_LOG2B_MAX; src must differ from the destination.
constexpr int TRANSITION_LOG2B_MIN = 6, TRANSITION_LOG2B_MAX = 8;
hipError_t launch_tr_p4(int src, const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);
hipError_t launch_tr_s8(int src, const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);
hipError_t launch_tr_s16(int src, const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);
hipError_t launch_tr_s32(int src, const MdqDesc *, int, long long, int, int, bool, unsigned long long *, const StepArgs &, bool, hipStream_t);

hipError_t launch_math(int which, const float *x, float *y, long long n, hipStream_t s);
hipError_t launch_math_digests(int which, unsigned first, unsigned count, unsigned chunk,
                               unsigned long long *dig, hipStream_t s);
hipError_t launch_log_approx_err(unsigned first, unsigned count, double slope, unsigned long long *out,
                                 hipStream_t s);
hipError_t launch_hw_ulp_err(int which, unsigned first, unsigned count, unsigned *out, hipStream_t s);

}  // namespace mdq
