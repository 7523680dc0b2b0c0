// mdq_stats.hip -- per-tensor gradient statistics of the MDQ bit decision,
// for a whole tensor list in two launches.
//
// The reference computes, per tensor and before the step (stquant_opt_simple.py:93-98),
//   n_l = sqrt(mean(g^2)),  r_l = std(g) / (mean(|g|) + 1e-12),  v_l = mean(g^2)
// with std unbiased, as separate fp32 torch reductions per tensor.  Here:
//   1. stats_partial_kernel: one 512-thread workgroup per 32768-element tile of
//      one tensor.  It holds the tile in registers and writes four fp64 partials:
//      - sum g;
//      - sum (g - tile mean)^2, from a second pass over the registers;
//      - sum g^2, each square rounded to fp32 as the reference's grad * grad is;
//      - sum |g|.
//   2. stats_finish_kernel: one workgroup per tensor combines its tiles in a fixed
//      order.  The squared deviations combine by Chan's pairwise formula,
//      M2 = sum M2_i + sum n_i (mean_i - mean)^2, which stays exact to fp64
//      rounding however large |mean| is against the spread.  The results are
//      rounded to the reference's fp32 outputs.  A sum whose exact value exceeds
//      FLT_MAX gives inf, as the reference's fp32 accumulators overflow.
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

// fp64 sums of one element: g, g^2 (the fp32 square), |g|
__device__ __forceinline__ void acc(double &s1, double &s2, double &sa, float x)
{
    s1 += (double)x;
    s2 += (double)(x * x);
    sa += fabs((double)x);
}

// Sum of K doubles over the workgroup; the totals are returned in every thread
// (through LDS), summed in a fixed order.
template <int K>
__device__ __forceinline__ void block_sum(double (&v)[K], double (*lds)[K])
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
        for (int k = 0; k < K; ++k) v[k] += __shfl_xor(v[k], off, 64);
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) == 0)
#pragma unroll
        for (int k = 0; k < K; ++k) lds[w][k] = v[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) {
        double t = lds[0][k];
#pragma unroll
        for (int q = 1; q < ST_WAVES; ++q) t += lds[q][k];
        v[k] = t;
    }
    __syncthreads();   // lds is free for the next block_sum
}

template <int GT>
__global__ __launch_bounds__(ST_THREADS) void stats_partial_kernel(const StatDesc *__restrict__ d, int n,
                                                                   const long long *__restrict__ tb,
                                                                   double *__restrict__ partials)
{
    __shared__ double lds3[ST_WAVES][3];
    __shared__ double lds1[ST_WAVES][1];
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
    const int64_t cnt = t.numel - base < STAT_TILE ? t.numel - base : STAT_TILE;   // elements of this tile
    double s[3] = {0.0, 0.0, 0.0};      // sum g, sum g^2, sum |g|
    double m2[1] = {0.0};               // sum (g - tile mean)^2
    const bool vec = cnt == STAT_TILE && (reinterpret_cast<uintptr_t>(t.g) % 16) == 0;
    if (vec) {
        // the whole tile in registers (STAT_TILE / ST_THREADS elements per thread):
        // one pass for the sums, a second over the registers for the deviations
        constexpr int V = vec_elems<GT>();
        constexpr int NL = STAT_TILE / (V * ST_THREADS);
        float xv[NL][V];
#pragma unroll
        for (int k = 0; k < NL; ++k) load_vec<GT>(t.g, base + V * ((int64_t)k * ST_THREADS + threadIdx.x), xv[k]);
#pragma unroll
        for (int k = 0; k < NL; ++k)
#pragma unroll
            for (int e = 0; e < V; ++e) acc(s[0], s[1], s[2], xv[k][e]);
        block_sum<3>(s, lds3);
        const double mean = s[0] / (double)STAT_TILE;
#pragma unroll
        for (int k = 0; k < NL; ++k)
#pragma unroll
            for (int e = 0; e < V; ++e) {
                const double dv = (double)xv[k][e] - mean;
                m2[0] = fma(dv, dv, m2[0]);
            }
    } else {
        for (int k = 0; k < STAT_TILE / ST_THREADS; ++k) {
            const int64_t e = (int64_t)k * ST_THREADS + threadIdx.x;
            if (e < cnt) acc(s[0], s[1], s[2], load_one<GT>(t.g, base + e));
        }
        block_sum<3>(s, lds3);
        const double mean = s[0] / (double)cnt;
        for (int k = 0; k < STAT_TILE / ST_THREADS; ++k) {
            const int64_t e = (int64_t)k * ST_THREADS + threadIdx.x;
            if (e < cnt) {
                const double dv = (double)load_one<GT>(t.g, base + e) - mean;
                m2[0] = fma(dv, dv, m2[0]);
            }
        }
    }
    block_sum<1>(m2, lds1);
    if (threadIdx.x == 0) {
        partials[4 * tile + 0] = s[0];
        partials[4 * tile + 1] = m2[0];
        partials[4 * tile + 2] = s[1];
        partials[4 * tile + 3] = s[2];
    }
}

// fp32 value of a sum of non-negative terms as an fp32 accumulator holds it:
// inf once the exact sum exceeds FLT_MAX.
__device__ __forceinline__ float f32_sum(double x) { return x > (double)__FLT_MAX__ ? __builtin_inff() : (float)x; }

__global__ __launch_bounds__(ST_THREADS) void stats_finish_kernel(const StatDesc *__restrict__ d,
                                                                  const double *__restrict__ partials,
                                                                  float *__restrict__ out)
{
    __shared__ double lds3[ST_WAVES][3];
    __shared__ double lds1[ST_WAVES][1];
    const StatDesc t = d[blockIdx.x];
    double s[3] = {0.0, 0.0, 0.0};      // sum g, sum g^2, sum |g|
    for (long long k = t.tile_begin + threadIdx.x; k < t.tile_end; k += ST_THREADS) {
        s[0] += partials[4 * k + 0];
        s[1] += partials[4 * k + 2];
        s[2] += partials[4 * k + 3];
    }
    block_sum<3>(s, lds3);
    const double N = (double)t.numel;
    const double mean = s[0] / N;
    // Chan et al.'s combination of the tiles' (count, mean, M2)
    double m2[1] = {0.0};
    for (long long k = t.tile_begin + threadIdx.x; k < t.tile_end; k += ST_THREADS) {
        const int64_t first = (k - t.tile_begin) * STAT_TILE;
        const double ni = (double)(t.numel - first < STAT_TILE ? t.numel - first : STAT_TILE);
        const double dm = partials[4 * k + 0] / ni - mean;
        m2[0] += fma(ni * dm, dm, partials[4 * k + 1]);
    }
    block_sum<1>(m2, lds1);
    if (threadIdx.x == 0) {
        // The reference's fp32 results: mean(g * g) and mean(|g|) from fp32 sums, std from
        // an fp32 M2 (torch's Welford accumulators on the GPU), then sqrt / divide / add in
        // fp32.  numel 0 gives NaN means and numel 0 or 1 a NaN std (unbiased), as torch does.
        const float sum_sq = f32_sum(s[1]), sum_abs = f32_sum(s[2]), m2f = f32_sum(m2[0]);
        const float mean_sq = sum_sq == __builtin_inff() ? sum_sq : (float)(s[1] / N);
        const float mean_abs = sum_abs == __builtin_inff() ? sum_abs : (float)(s[2] / N);
        const float sd = t.numel < 2 ? __builtin_nanf("")
                                     : (m2f == __builtin_inff() ? m2f : (float)sqrt(m2[0] / (N - 1.0)));
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
