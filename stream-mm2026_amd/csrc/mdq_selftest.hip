// Device-side evaluation of the step's fp32 math (mdq_math.h) so it can be
// compared bit for bit with a CPU implementation.
#include <hip/hip_runtime.h>

#include "mdq_kernel.h"
#include "mdq_launch.h"
#include "mdq_math.h"

namespace mdq {

// which: 0 e^x, 1 log x, 3 the correctly rounded reciprocal of the stochastic requant
__device__ __forceinline__ float eval_math(int which, float x)
{
    return which == 0 ? mdq_expf(x) : which == 1 ? mdq_logf(x) : mdq_rcp_rn(x);
}

__global__ __launch_bounds__(256) void math_kernel(int which, const float *__restrict__ x,
                                                   float *__restrict__ y, long long n)
{
    if (which == 2) {   // (dv, vmin) pairs -> (c1, c0) pairs of the fast v-code path
        for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n / 2;
             i += (long long)gridDim.x * blockDim.x) {
            const VCodeMap m = mdq_vcode_map(x[2 * i], x[2 * i + 1]);
            y[2 * i] = m.c1;
            y[2 * i + 1] = m.c0;
        }
        return;
    }
    if (which == 4) {   // (x, kv, dv, vmin, lmax, QV) -> (Zh, ep, 0, 0, 0, 0) of the stochastic fast v code
        for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n / 6;
             i += (long long)gridDim.x * blockDim.x) {
            const float *a = x + 6 * i;
            const SrVFast f = mdq_sr_vfast(a[2], a[3], a[4], mdq_sr_ep0(a[5]));
            y[6 * i] = mdq_sr_vfast_z(a[0], mdq_u16_uniform_minus_half((uint32_t)a[1]), f);
            y[6 * i + 1] = f.ep;
            for (int k = 2; k < 6; ++k) y[6 * i + k] = 0.0f;
        }
        return;
    }
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (long long)gridDim.x * blockDim.x)
        y[i] = eval_math(which, x[i]);
}

__device__ __forceinline__ unsigned long long mix64(unsigned long long z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Each thread sums 64 consecutive bit patterns (chunk is a multiple of 64, so
// a run never straddles two chunks) and adds the sum to its chunk's digest.
__global__ __launch_bounds__(256) void math_digest_kernel(int which, unsigned first, unsigned count,
                                                          unsigned chunk,
                                                          unsigned long long *__restrict__ dig)
{
    const unsigned long long runs = ((unsigned long long)count + 63) / 64;
    for (unsigned long long r = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; r < runs;
         r += (unsigned long long)gridDim.x * blockDim.x) {
        const unsigned off0 = (unsigned)(r * 64);
        unsigned long long acc = 0;
        for (unsigned k = 0; k < 64 && off0 + k < count; ++k) {
            const unsigned b = first + off0 + k;
            const float y = eval_math(which, bits_f(b));
            acc += mix64(((unsigned long long)b << 32) | f_bits(y));
        }
        atomicAdd(dig + off0 / chunk, acc);
    }
}

// max(0, max over x = bits_f(first .. first+count-1) of
// |log2_hw(x) * ln 2 - mdq_logf(x)| - slope * |mdq_logf(x)|) in fp64, as the bit pattern
// of a non-negative double (atomic max over uint64 orders those).
__global__ __launch_bounds__(256) void log_approx_err_kernel(unsigned first, unsigned count, double slope,
                                                             unsigned long long *__restrict__ out)
{
    double m = 0.0;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (unsigned long long)gridDim.x * blockDim.x) {
        const float x = bits_f(first + (unsigned)i);
        const double l = (double)mdq_logf(x);
        const double e = fabs((double)__builtin_amdgcn_logf(x) * 0.69314718055994530942 - l) - slope * fabs(l);
        m = e > m ? e : m;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const double o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) atomicMax(out, (unsigned long long)__double_as_longlong(m));
}

// The largest distance in units in the last place between the hardware square root
// (which = 0) or reciprocal (which = 1) the step's parameter update uses and the
// correctly rounded result, over x = bits_f(first .. first+count-1) (positive floats
// whose result is a positive normal float).  The correctly rounded result is the fp64
// operation (correctly rounded) rounded to fp32: rounding twice is exact for sqrt and
// division when the wider format has at least 2p + 2 bits (53 >= 2 * 24 + 2), so it
// equals IEEE sqrtf / 1.0f / x.
__global__ __launch_bounds__(256) void hw_ulp_err_kernel(int which, unsigned first, unsigned count,
                                                         unsigned *__restrict__ out)
{
    unsigned m = 0;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (unsigned long long)gridDim.x * blockDim.x) {
        const float x = bits_f(first + (unsigned)i);
        const float hw = which == 0 ? __builtin_amdgcn_sqrtf(x) : __builtin_amdgcn_rcpf(x);
        const float rn = which == 0 ? (float)__builtin_sqrt((double)x) : (float)(1.0 / (double)x);
        const unsigned a = f_bits(hw), b = f_bits(rn);
        const unsigned d = a > b ? a - b : b - a;
        m = d > m ? d : m;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const unsigned o = (unsigned)__shfl_xor((int)m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) atomicMax(out, m);
}

hipError_t launch_hw_ulp_err(int which, unsigned first, unsigned count, unsigned *out, hipStream_t s)
{
    if (count == 0) return hipSuccess;
    unsigned long long blocks = ((unsigned long long)count + 255) / 256;
    int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(hw_ulp_err_kernel, dim3(grid), dim3(256), 0, s, which, first, count, out);
    return hipGetLastError();
}

hipError_t launch_log_approx_err(unsigned first, unsigned count, double slope, unsigned long long *out,
                                 hipStream_t s)
{
    if (count == 0) return hipSuccess;
    unsigned long long blocks = ((unsigned long long)count + 255) / 256;
    int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(log_approx_err_kernel, dim3(grid), dim3(256), 0, s, first, count, slope, out);
    return hipGetLastError();
}

hipError_t launch_math(int which, const float *x, float *y, long long n, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    long long blocks = (n + 255) / 256;
    int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(math_kernel, dim3(grid), dim3(256), 0, s, which, x, y, n);
    return hipGetLastError();
}

hipError_t launch_math_digests(int which, unsigned first, unsigned count, unsigned chunk,
                               unsigned long long *dig, hipStream_t s)
{
    if (count == 0) return hipSuccess;
    unsigned long long runs = ((unsigned long long)count + 63) / 64;
    unsigned long long blocks = (runs + 255) / 256;
    int grid = (int)(blocks < 65536 ? blocks : 65536);
    hipLaunchKernelGGL(math_digest_kernel, dim3(grid), dim3(256), 0, s, which, first, count, chunk, dig);
    return hipGetLastError();
}

}  // namespace mdq
