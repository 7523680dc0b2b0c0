// mdq_stats.hip -- per-tensor gradient statistics of the MDQ bit decision,
// for a whole tensor list in two launches.
//
// The reference computes, per tensor and before the step (stquant_opt_simple.py:93-98),
//   n_l = sqrt(mean(g^2)),  r_l = std(g) / (mean(|g|) + 1e-12),  v_l = mean(g^2)
// with std unbiased, as separate torch reductions per tensor.  Here:
//   1. stats_partial_kernel: one 512-thread workgroup per 32768-element tile of one tensor
//      accumulates sum g, sum g^2, sum |g| in fp64 (each fp32 square is exact
//      in fp64) and writes the three partial sums of its tile;
//   2. stats_finish_kernel: one workgroup per tensor adds its tiles' partials
//      in a fixed order and rounds to the reference's fp32 outputs.
// Both orders are fixed by the tensor list, so results are deterministic.
#include <hip/hip_runtime.h>

#include "mdq_desc.h"
#include "mdq_stats.h"

namespace mdq {

namespace {

constexpr int ST_THREADS = 512;
constexpr int ST_WAVES = ST_THREADS / 64;

__device__ __forceinline__ float bf16_to_f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float f16_to_f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

template <int GT>
__device__ __forceinline__ float load_one(const void *g, int64_t e)
{
    if constexpr (GT == GT_F32) return static_cast<const float *>(g)[e];
    else if constexpr (GT == GT_BF16) return bf16_to_f(static_cast<const unsigned short *>(g)[e]);
    else return f16_to_f(static_cast<const unsigned short *>(g)[e]);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Elements per 16-byte load.
template <int GT> constexpr int vec_elems() { return GT == GT_F32 ? 4 : 8; }

// One 16-byte non-temporal load at element e (16-byte aligned), widened to fp32.
template <int GT>
__device__ __forceinline__ void load_vec(const void *g, int64_t e, float (&x)[vec_elems<GT>()])
{
    if constexpr (GT == GT_F32) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(static_cast<const float *>(g) + e));
        x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    } else {
        const u32x4 v = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(static_cast<const unsigned short *>(g) + e));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[2 * k] = GT == GT_BF16 ? bf16_to_f(w[k] & 0xffffu) : f16_to_f(w[k] & 0xffffu);
            x[2 * k + 1] = GT == GT_BF16 ? bf16_to_f(w[k] >> 16) : f16_to_f(w[k] >> 16);
        }
    }
}

__device__ __forceinline__ void acc(double &s1, double &s2, double &sa, float x)
{
    const double d = (double)x;
    s1 += d;
    s2 = fma(d, d, s2);
    sa += fabs(d);
}

// Sum of three doubles over the workgroup; the result is valid in thread 0.
__device__ __forceinline__ void block_sum3(double &s1, double &s2, double &sa, double (*lds)[3])
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        s1 += __shfl_xor(s1, off, 64);
        s2 += __shfl_xor(s2, off, 64);
        sa += __shfl_xor(sa, off, 64);
    }
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0) {
        lds[w][0] = s1;
        lds[w][1] = s2;
        lds[w][2] = sa;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        s1 = lds[0][0];
        s2 = lds[0][1];
        sa = lds[0][2];
#pragma unroll
        for (int k = 1; k < ST_WAVES; ++k) {
            s1 += lds[k][0];
            s2 += lds[k][1];
            sa += lds[k][2];
        }
    }
}

template <int GT>
__global__ __launch_bounds__(ST_THREADS) void stats_partial_kernel(const StatDesc *__restrict__ d, int n,
                                                                   const long long *__restrict__ tb,
                                                                   double *__restrict__ partials)
{
    __shared__ double lds[ST_WAVES][3];
    // Workgroup b runs on XCD x = b % 8 as its j-th (j = b / 8); the tiles go to
    // the XCDs in round-robin chunks of 16 (2^19 elements), the workgroups of the
    // last, partial round of 8 chunks take tile b (a bijection on [0, grid)).
    // LLaMA-7B bf16 grads, same-allocation A/B: 1.89 ms against 2.00 ms for
    // tile = b; chunks of 32-128 tiles run as 16.
    constexpr unsigned CK = 16u;
    const unsigned grid = gridDim.x, b = blockIdx.x, j = b >> 3, x = b & 7u;
    const long long tile = b < grid / (8u * CK) * (8u * CK) ? (long long)((j / CK) * 8u + x) * CK + (j % CK)
                                                            : (long long)b;
    // the tensor owning this tile: the last i with tile_begin[i] <= tile
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tb[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    const StatDesc t = d[lo];
    const int64_t base = (tile - t.tile_begin) * STAT_TILE;
    double s1 = 0.0, s2 = 0.0, sa = 0.0;
    const bool vec = base + STAT_TILE <= t.numel && (reinterpret_cast<uintptr_t>(t.g) % 16) == 0;
    if (vec) {
        // all loads of the thread first (STAT_TILE / ST_THREADS elements), then the sums
        constexpr int V = vec_elems<GT>();
        constexpr int NL = STAT_TILE / (V * ST_THREADS);
        float x[NL][V];
#pragma unroll
        for (int k = 0; k < NL; ++k) load_vec<GT>(t.g, base + V * ((int64_t)k * ST_THREADS + threadIdx.x), x[k]);
#pragma unroll
        for (int k = 0; k < NL; ++k)
#pragma unroll
            for (int j = 0; j < V; ++j) acc(s1, s2, sa, x[k][j]);
    } else {
        for (int k = 0; k < STAT_TILE / ST_THREADS; ++k) {
            const int64_t e = base + (int64_t)k * ST_THREADS + threadIdx.x;
            if (e < t.numel) acc(s1, s2, sa, load_one<GT>(t.g, e));
        }
    }
    block_sum3(s1, s2, sa, lds);
    if (threadIdx.x == 0) {
        partials[3 * tile + 0] = s1;
        partials[3 * tile + 1] = s2;
        partials[3 * tile + 2] = sa;
    }
}

__global__ __launch_bounds__(ST_THREADS) void stats_finish_kernel(const StatDesc *__restrict__ d,
                                                                  const double *__restrict__ partials,
                                                                  float *__restrict__ out)
{
    __shared__ double lds[ST_WAVES][3];
    const StatDesc t = d[blockIdx.x];
    double s1 = 0.0, s2 = 0.0, sa = 0.0;
    for (long long k = t.tile_begin + threadIdx.x; k < t.tile_end; k += ST_THREADS) {
        s1 += partials[3 * k + 0];
        s2 += partials[3 * k + 1];
        sa += partials[3 * k + 2];
    }
    block_sum3(s1, s2, sa, lds);
    if (threadIdx.x == 0) {
        // fp32 outputs in the reference's operation order: mean and std are fp32
        // tensors, then sqrt / divide / add in fp32.  numel 0 gives NaN means and
        // numel 1 a NaN std (unbiased), as torch does.
        const double N = (double)t.numel;
        const float mean_sq = (float)(s2 / N);
        const float mean_abs = (float)(sa / N);
        const double var = (s2 - s1 * (s1 / N)) / (N - 1.0);
        const float sd = (float)sqrt(var > 0.0 ? var : (var == var ? 0.0 : var));
        out[3 * blockIdx.x + 0] = sqrtf(mean_sq);
        out[3 * blockIdx.x + 1] = sd / (mean_abs + 1e-12f);
        out[3 * blockIdx.x + 2] = mean_sq;
    }
}

}  // namespace

hipError_t launch_grad_stats(const StatDesc *d, const long long *tb, int n, long long tiles, int grad_dt,
                             double *partials, float *out, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    if (tiles > 0) {
        const dim3 grid((unsigned)tiles), block(ST_THREADS);
        switch (grad_dt) {
        case GT_F32: stats_partial_kernel<GT_F32><<<grid, block, 0, s>>>(d, n, tb, partials); break;
        case GT_BF16: stats_partial_kernel<GT_BF16><<<grid, block, 0, s>>>(d, n, tb, partials); break;
        default: stats_partial_kernel<GT_F16><<<grid, block, 0, s>>>(d, n, tb, partials); break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    stats_finish_kernel<<<dim3((unsigned)n), dim3(ST_THREADS), 0, s>>>(d, partials, out);
    return hipGetLastError();
}

}  // namespace mdq
