// mdq_stats.hip -- per-tensor gradient statistics of the MDQ bit decision,
// for a whole tensor list in two launches.
//
// The reference computes, per tensor and before the step (stquant_opt_simple.py:93-98),
//   n_l = sqrt(mean(g^2)),  r_l = std(g) / (mean(|g|) + 1e-12),  v_l = mean(g^2)
// with std unbiased, as separate fp32 torch reductions per tensor.  Here:
//   1. stats_partial_kernel: one 512-thread workgroup per 32768-element tile of
//      one tensor writes four fp64 partials: sum g, M2 = sum (g - tile mean)^2,
//      sum g^2 (fp32 squares, as the reference's grad * grad) and sum |g|.
//      Each thread loads its 64 elements with 16-byte loads and sums x, x^2 and |x|
//      over each load pairwise in fp32 (at most 3 roundings, 1.8e-7 of the summed
//      magnitudes), and these short sums across loads in fp64.  Near the HBM
//      roofline the kernel is close to VALU-bound (about ten lane instructions per
//      element fit in the memory time); this path takes about seven.  The thread's M2 comes from sum x^2 - (sum x)^2 / 64
//      where that cancellation loses at most a bit; where the mean dominates the
//      spread the registers are summed again as deviations from the thread's fp32
//      mean, and non-finite or tiny (squares below fp32's normal range) values are
//      redone in fp64.  The threads' (mean, M2) then merge pairwise by Chan's
//      formula for equal counts, across lanes and across the workgroup's waves.
//      Ragged tiles and views not 16-byte aligned take per-element fp64 sums and a
//      second pass over the tile for the deviations from its mean.
//   2. stats_finish_kernel: one workgroup per tensor combines its tiles in a fixed
//      order.  The squared deviations combine by Chan's pairwise formula,
//      M2 = sum M2_i + sum n_i (mean_i - mean)^2, which stays accurate however
//      large |mean| is against the spread.  The results are rounded to the
//      reference's fp32 outputs.  A sum whose exact value exceeds FLT_MAX gives
//      inf, as the reference's fp32 accumulators overflow.
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

// The grads' pointers come from the descriptor table, so the compiler cannot tell
// they are global memory: without the cast it emits flat loads, which it can only
// wait for all together.
#define ST_GLOBAL __attribute__((address_space(1)))

template <int GT>
__device__ __forceinline__ float load_one(const void *g, int64_t e)
{
    if constexpr (GT == GT_F32) return ((const ST_GLOBAL float *)g)[e];
    else if constexpr (GT == GT_BF16) return bf16_to_f(((const ST_GLOBAL unsigned short *)g)[e]);
    else return f16_to_f(((const ST_GLOBAL unsigned short *)g)[e]);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Elements per 16-byte load.
template <int GT> constexpr int vec_elems() { return GT == GT_F32 ? 4 : 8; }

// One 16-byte non-temporal load at element e (16-byte aligned), kept as loaded
// (16-bit grads take half the registers of their fp32 values).
template <int GT>
__device__ __forceinline__ u32x4 load_raw(const void *g, int64_t e)
{
    constexpr int ES = GT == GT_F32 ? 4 : 2;   // bytes per element
    return __builtin_nontemporal_load((const ST_GLOBAL u32x4 *)(static_cast<const char *>(g) + ES * e));
}

// The fp32 values of one loaded 16-byte vector.
template <int GT>
__device__ __forceinline__ void widen(const u32x4 v, float (&x)[vec_elems<GT>()])
{
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    if constexpr (GT == GT_F32) {
#pragma unroll
        for (int k = 0; k < 4; ++k) x[k] = __uint_as_float(w[k]);
    } else {
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

// Pairwise fp32 sum of N = 4 or 8 values.
template <int N>
__device__ __forceinline__ float pair_sum(const float (&x)[N])
{
    const float a = (x[0] + x[1]) + (x[2] + x[3]);
    if constexpr (N == 4) return a;
    else return a + ((x[4] + x[5]) + (x[6] + x[7]));
}

// Chan et al.'s merge of two disjoint parts of n elements each into (mean, M2) of
// their union: mean = (mean_a + mean_b) / 2, M2 = M2_a + M2_b + (n / 2) delta^2.
// Symmetric in the two parts, bit for bit, so both lanes of a butterfly exchange
// hold the same result.
__device__ __forceinline__ void merge_equal(double &mean, double &m2, double om, double om2, int n)
{
    const double dl = om - mean;
    m2 = fma(dl, dl * (0.5 * n), m2 + om2);
    mean = (mean + om) * 0.5;
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
    __shared__ double lds4[ST_WAVES][4];
    __shared__ double lds3[ST_WAVES][3];
    __shared__ double lds2[ST_WAVES][2];
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
    const bool vec = cnt == STAT_TILE && (reinterpret_cast<uintptr_t>(t.g) % 16) == 0;
    if (vec) {
        // One pass: each thread loads its STAT_TILE / ST_THREADS elements and sums x,
        // x^2 and |x| (fp32 over each loaded group, pairwise; fp64 across groups).
        constexpr int V = vec_elems<GT>();
        constexpr int NL = STAT_TILE / (V * ST_THREADS);
        constexpr double NT = (double)(V * NL);        // elements per thread
        u32x4 raw[NL];
#pragma unroll
        for (int k = 0; k < NL; ++k) raw[k] = load_raw<GT>(t.g, base + V * ((int64_t)k * ST_THREADS + threadIdx.x));
        double sx = 0.0, sq = 0.0, ab = 0.0;
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            float x[V], x2[V], xa[V];
            widen<GT>(raw[k], x);
#pragma unroll
            for (int e = 0; e < V; ++e) {
                x2[e] = x[e] * x[e];
                xa[e] = fabsf(x[e]);
            }
            sx += (double)pair_sum<V>(x);
            sq += (double)pair_sum<V>(x2);
            ab += (double)pair_sum<V>(xa);
        }
        // The thread's M2 = sum x^2 - (sum x)^2 / n loses at most one bit to cancellation
        // where (sum x)^2 / n <= sum x^2 / 2, i.e. the mean is not large against the spread
        // (zero-mean-like gradients).  Elsewhere the registers are summed again as
        // deviations from the fp32 thread mean (exact where x is within a factor 2 of it);
        // non-finite sums (a non-finite x, or fp32 sums beyond FLT_MAX) and values so small
        // that fp32 squares lose bits (mean |x| or mean |x - mean| below 2^-60) are redone
        // in fp64 from memory.
        double mean = sx * (1.0 / NT);
        double m2 = fma(-sx, mean, sq);
        bool exact = fabs(sx) <= __DBL_MAX__ && sq <= __DBL_MAX__ && !(ab > 0.0 && ab < 0x1p-60 * NT);
        if (exact && !(sx * sx <= 0.5 * NT * sq)) {
            const float c = (float)mean;
            double s1 = 0.0, s2 = 0.0, sd = 0.0;
#pragma unroll
            for (int k = 0; k < NL; ++k) {
                float x[V], dv[V], d2[V], da[V];
                widen<GT>(raw[k], x);
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    dv[e] = x[e] - c;
                    d2[e] = dv[e] * dv[e];
                    da[e] = fabsf(dv[e]);
                }
                s1 += (double)pair_sum<V>(dv);
                s2 += (double)pair_sum<V>(d2);
                sd += (double)pair_sum<V>(da);
            }
            mean = fma(s1, 1.0 / NT, (double)c);
            m2 = fma(-s1, s1 * (1.0 / NT), s2);
            exact = s2 <= __DBL_MAX__ && !(sd > 0.0 && sd < 0x1p-60 * NT);
        }
        if (!exact) {
            double tot = 0.0;
#pragma unroll 1
            for (int k = 0; k < NL; ++k)
#pragma unroll 1
                for (int e = 0; e < V; ++e) tot += (double)load_one<GT>(t.g, base + V * ((int64_t)k * ST_THREADS + threadIdx.x) + e);
            mean = tot * (1.0 / NT);
            m2 = 0.0;
#pragma unroll 1
            for (int k = 0; k < NL; ++k)
#pragma unroll 1
                for (int e = 0; e < V; ++e) {
                    const double dd = (double)load_one<GT>(t.g, base + V * ((int64_t)k * ST_THREADS + threadIdx.x) + e) - mean;
                    m2 = fma(dd, dd, m2);
                }
        }
#pragma unroll
        for (int off = 1, part = V * NL; off < 64; off <<= 1, part <<= 1) {
            const double om = __shfl_xor(mean, off, 64), om2 = __shfl_xor(m2, off, 64);
            sq += __shfl_xor(sq, off, 64);
            ab += __shfl_xor(ab, off, 64);
            merge_equal(mean, m2, om, om2, part);
        }
        const int w = threadIdx.x / 64;
        if ((threadIdx.x & 63) == 0) {
            lds4[w][0] = mean;
            lds4[w][1] = m2;
            lds4[w][2] = sq;
            lds4[w][3] = ab;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            double mw[ST_WAVES], m2w[ST_WAVES];
            sq = ab = 0.0;
#pragma unroll
            for (int q = 0; q < ST_WAVES; ++q) {
                mw[q] = lds4[q][0];
                m2w[q] = lds4[q][1];
                sq += lds4[q][2];
                ab += lds4[q][3];
            }
#pragma unroll
            for (int h = 1; h < ST_WAVES; h <<= 1)
#pragma unroll
                for (int q = 0; q < ST_WAVES; q += 2 * h) merge_equal(mw[q], m2w[q], mw[q + h], m2w[q + h], 64 * V * NL * h);
            partials[4 * tile + 0] = mw[0] * (double)STAT_TILE;
            partials[4 * tile + 1] = m2w[0];
            partials[4 * tile + 2] = sq;
            partials[4 * tile + 3] = ab;
        }
        return;
    }
    // A ragged last tile, or a view not 16-byte aligned: per-element fp64 sums, the
    // tile mean, then a second pass over the tile (re-read) for the squared deviations
    // from it.
    double s[3] = {0.0, 0.0, 0.0};      // sum g, sum g^2, sum |g|
    for (int k = 0; k < STAT_TILE / ST_THREADS; ++k) {
        const int64_t e = (int64_t)k * ST_THREADS + threadIdx.x;
        if (e < cnt) acc(s[0], s[1], s[2], load_one<GT>(t.g, base + e));
    }
    block_sum<3>(s, lds3);
    const double n_t = (double)cnt;
    const float c = (float)(s[0] / n_t);
    double dv[2] = {0.0, 0.0};          // sum d, sum d^2 with d = g - c
    for (int k = 0; k < STAT_TILE / ST_THREADS; ++k) {
        const int64_t e = (int64_t)k * ST_THREADS + threadIdx.x;
        if (e < cnt) {
            const double dd = (double)load_one<GT>(t.g, base + e) - (double)c;
            dv[0] += dd;
            dv[1] = fma(dd, dd, dv[1]);
        }
    }
    block_sum<2>(dv, lds2);
    if (threadIdx.x == 0) {
        // d = g - c is exact in fp64, so M2 = sum d^2 - (sum d)^2 / n and sum g = n c + sum d
        // are as accurate as the tile's spread allows (non-finite g: the first pass's sum)
        partials[4 * tile + 0] = fabs(dv[0]) <= __DBL_MAX__ ? fma(n_t, (double)c, dv[0]) : s[0];
        partials[4 * tile + 1] = dv[1] - dv[0] * (dv[0] / n_t);
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
