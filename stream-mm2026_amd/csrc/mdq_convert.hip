// mdq_convert.hip -- re-storing m/v codes in another storage class, for a
// whole tensor list in one launch.
//
// MDQAdamWSimple changes a tensor's code storage when its bit width changes:
// before the step it aligns the storage to the width (unpack nibbles, widen,
// or clamp to the narrower integer range), after the step it packs 4-bit
// codes into nibbles (/root/reference/CUDA/stquant_opt_simple.py:140-210).
// The reference does that with several torch passes per tensor.  Every one of
// those transitions is the value map decode(src) -> clamp -> encode(dst):
//   decode  P4: m = (byte & 15) - 8, v = byte >> 4;  S8/S16/S32: the integers
//   encode  S8: m in [-128, 127], v in [0, 255];  S16: [-32768, 32767],
//           [0, 65535];  S32: as is;  P4: byte = clamp(m + 8, 0, 15)
//           | clamp(v, 0, 15) << 4
// One 256-thread workgroup per 4096-element tile of one tensor.  In a whole
// tile whose code arrays are 16-byte aligned, each thread converts 8
// contiguous elements per iteration with one 8-byte (1-byte codes), 16-byte
// (2-byte codes) or two 16-byte (4-byte codes) non-temporal access per array,
// so every wave instruction covers whole 128-byte lines; the (src, dst) pair
// is a workgroup-uniform switch.  Tails and unaligned arrays go element by
// element.
#include <hip/hip_runtime.h>

#include "mdq_convert.h"
#include "mdq_desc.h"

namespace mdq {

namespace {

constexpr int CV_THREADS = 256;
constexpr int CV_EPT = 8;                                   // elements per thread and iteration
constexpr int CV_ITERS = CONV_TILE / (CV_THREADS * CV_EPT);
static_assert(CV_ITERS * CV_THREADS * CV_EPT == CONV_TILE, "tile = threads x 8 x iterations");

#define CV_GLOBAL __attribute__((address_space(1)))
typedef uint32_t cu2 __attribute__((ext_vector_type(2)));
typedef uint32_t cu4 __attribute__((ext_vector_type(4)));

template <class T>
__device__ __forceinline__ T ldv(const void *a) { return __builtin_nontemporal_load((const CV_GLOBAL T *)a); }
template <class T>
__device__ __forceinline__ void stv(T v, void *a) { __builtin_nontemporal_store(v, (CV_GLOBAL T *)a); }

// ------------------------------------------------------------ element path
__device__ __forceinline__ void decode(const ConvDesc &t, int64_t i, int64_t &m, int64_t &v)
{
    switch (t.src) {
    case ST_P4: {
        const uint32_t b = static_cast<const uint8_t *>(t.src_m)[i];
        m = (int64_t)(b & 15u) - 8;
        v = b >> 4;
        break;
    }
    case ST_S8:
        m = static_cast<const int8_t *>(t.src_m)[i];
        v = static_cast<const uint8_t *>(t.src_v)[i];
        break;
    case ST_S16:
        m = static_cast<const int16_t *>(t.src_m)[i];
        v = static_cast<const uint16_t *>(t.src_v)[i];
        break;
    default:
        m = static_cast<const int32_t *>(t.src_m)[i];
        v = static_cast<const uint32_t *>(t.src_v)[i];
        break;
    }
}

__device__ __forceinline__ int64_t clamp64(int64_t x, int64_t lo, int64_t hi) { return x < lo ? lo : (x > hi ? hi : x); }

__device__ __forceinline__ void encode(const ConvDesc &t, int64_t i, int64_t m, int64_t v)
{
    switch (t.dst) {
    case ST_P4:
        static_cast<uint8_t *>(t.dst_m)[i] = (uint8_t)(clamp64(m + 8, 0, 15) | (clamp64(v, 0, 15) << 4));
        break;
    case ST_S8:
        static_cast<int8_t *>(t.dst_m)[i] = (int8_t)clamp64(m, -128, 127);
        static_cast<uint8_t *>(t.dst_v)[i] = (uint8_t)clamp64(v, 0, 255);
        break;
    case ST_S16:
        static_cast<int16_t *>(t.dst_m)[i] = (int16_t)clamp64(m, -32768, 32767);
        static_cast<uint16_t *>(t.dst_v)[i] = (uint16_t)clamp64(v, 0, 65535);
        break;
    default:
        static_cast<int32_t *>(t.dst_m)[i] = (int32_t)m;
        static_cast<uint32_t *>(t.dst_v)[i] = (uint32_t)v;
        break;
    }
}

// ------------------------------------------------------------- vector path
// 8 codes of one array as packed bytes / halves / words.
template <int ST> struct Vec8;
template <> struct Vec8<ST_P4> { cu2 w; };
template <> struct Vec8<ST_S8> { cu2 w; };
template <> struct Vec8<ST_S16> { cu4 w; };
template <> struct Vec8<ST_S32> { cu4 lo, hi; };

template <int ST> constexpr int code_size() { return ST == ST_S16 ? 2 : ST == ST_S32 ? 4 : 1; }

// The 8 codes starting at element i: m as int32, v as uint32 (the S32 m range
// is int32 and every v is non-negative, so no wider type is needed).
template <int ST>
__device__ __forceinline__ void load8(const ConvDesc &t, int64_t i, int32_t (&m)[8], uint32_t (&v)[8])
{
    constexpr int cs = code_size<ST>();
    const char *pm = static_cast<const char *>(t.src_m) + i * cs;
    const char *pv = static_cast<const char *>(t.src_v) + i * cs;
    if constexpr (ST == ST_P4) {
        const cu2 w = ldv<cu2>(pm);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t b = ((k < 4 ? w.x : w.y) >> (8 * (k & 3))) & 0xffu;
            m[k] = (int32_t)(b & 15u) - 8;
            v[k] = b >> 4;
        }
    } else if constexpr (ST == ST_S8) {
        const cu2 wm = ldv<cu2>(pm), wv = ldv<cu2>(pv);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            m[k] = (int32_t)(int8_t)((k < 4 ? wm.x : wm.y) >> (8 * (k & 3)));
            v[k] = ((k < 4 ? wv.x : wv.y) >> (8 * (k & 3))) & 0xffu;
        }
    } else if constexpr (ST == ST_S16) {
        const cu4 wm = ldv<cu4>(pm), wv = ldv<cu4>(pv);
        const uint32_t am[4] = {wm.x, wm.y, wm.z, wm.w}, av[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            m[k] = (int32_t)(int16_t)(am[k >> 1] >> (16 * (k & 1)));
            v[k] = (av[k >> 1] >> (16 * (k & 1))) & 0xffffu;
        }
    } else {
        const cu4 m0 = ldv<cu4>(pm), m1 = ldv<cu4>(pm + 16);
        const cu4 v0 = ldv<cu4>(pv), v1 = ldv<cu4>(pv + 16);
        const uint32_t am[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
        const uint32_t av[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            m[k] = (int32_t)am[k];
            v[k] = av[k];
        }
    }
}

__device__ __forceinline__ int32_t clampi(int32_t x, int32_t lo, int32_t hi) { return x < lo ? lo : (x > hi ? hi : x); }
__device__ __forceinline__ uint32_t minu(uint32_t x, uint32_t hi) { return x > hi ? hi : x; }

// Clamps to dst's range and stores the 8 codes at element i.  For P4,
// clamp(m + 8, 0, 15) is written as clamp(m, -8, 7) + 8 so that m + 8 cannot
// overflow int32.
template <int ST>
__device__ __forceinline__ void store8(const ConvDesc &t, int64_t i, const int32_t (&m)[8], const uint32_t (&v)[8])
{
    constexpr int cs = code_size<ST>();
    char *pm = static_cast<char *>(t.dst_m) + i * cs;
    char *pv = static_cast<char *>(t.dst_v) + i * cs;
    if constexpr (ST == ST_P4) {
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t b = (uint32_t)(clampi(m[k], -8, 7) + 8) | (minu(v[k], 15u) << 4);
            w[k >> 2] |= b << (8 * (k & 3));
        }
        stv<cu2>(cu2{w[0], w[1]}, pm);
    } else if constexpr (ST == ST_S8) {
        uint32_t wm[2] = {0u, 0u}, wv[2] = {0u, 0u};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            wm[k >> 2] |= ((uint32_t)clampi(m[k], -128, 127) & 0xffu) << (8 * (k & 3));
            wv[k >> 2] |= minu(v[k], 255u) << (8 * (k & 3));
        }
        stv<cu2>(cu2{wm[0], wm[1]}, pm);
        stv<cu2>(cu2{wv[0], wv[1]}, pv);
    } else if constexpr (ST == ST_S16) {
        uint32_t wm[4] = {0u, 0u, 0u, 0u}, wv[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            wm[k >> 1] |= ((uint32_t)clampi(m[k], -32768, 32767) & 0xffffu) << (16 * (k & 1));
            wv[k >> 1] |= minu(v[k], 65535u) << (16 * (k & 1));
        }
        stv<cu4>(cu4{wm[0], wm[1], wm[2], wm[3]}, pm);
        stv<cu4>(cu4{wv[0], wv[1], wv[2], wv[3]}, pv);
    } else {
        stv<cu4>(cu4{(uint32_t)m[0], (uint32_t)m[1], (uint32_t)m[2], (uint32_t)m[3]}, pm);
        stv<cu4>(cu4{(uint32_t)m[4], (uint32_t)m[5], (uint32_t)m[6], (uint32_t)m[7]}, pm + 16);
        stv<cu4>(cu4{v[0], v[1], v[2], v[3]}, pv);
        stv<cu4>(cu4{v[4], v[5], v[6], v[7]}, pv + 16);
    }
}

// One whole tile: all loads of the thread, then all stores.
template <int SRC, int DST>
__device__ __forceinline__ void tile_vec(const ConvDesc &t, int64_t base)
{
    int32_t m[CV_ITERS][8];
    uint32_t v[CV_ITERS][8];
#pragma unroll
    for (int k = 0; k < CV_ITERS; ++k)
        load8<SRC>(t, base + (int64_t)(k * CV_THREADS + (int)threadIdx.x) * CV_EPT, m[k], v[k]);
#pragma unroll
    for (int k = 0; k < CV_ITERS; ++k)
        store8<DST>(t, base + (int64_t)(k * CV_THREADS + (int)threadIdx.x) * CV_EPT, m[k], v[k]);
}

template <int SRC>
__device__ __forceinline__ void tile_vec_src(const ConvDesc &t, int64_t base)
{
    switch (t.dst) {
    case ST_P4: tile_vec<SRC, ST_P4>(t, base); break;
    case ST_S8: tile_vec<SRC, ST_S8>(t, base); break;
    case ST_S16: tile_vec<SRC, ST_S16>(t, base); break;
    default: tile_vec<SRC, ST_S32>(t, base); break;
    }
}

__device__ __forceinline__ bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__global__ __launch_bounds__(CV_THREADS) void convert_kernel(const ConvDesc *__restrict__ d, int n,
                                                             const long long *__restrict__ tb)
{
    const long long tile = blockIdx.x;
    int lo = 0, hi = n - 1;                       // the last tensor with tile_begin <= tile
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tb[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    const ConvDesc t = d[lo];
    const int64_t base = (tile - t.tile_begin) * CONV_TILE;
    const bool vec = base + CONV_TILE <= t.numel && al16(t.src_m) && al16(t.dst_m) &&
                     (t.src == ST_P4 || al16(t.src_v)) && (t.dst == ST_P4 || al16(t.dst_v));
    if (vec) {
        switch (t.src) {
        case ST_P4: tile_vec_src<ST_P4>(t, base); break;
        case ST_S8: tile_vec_src<ST_S8>(t, base); break;
        case ST_S16: tile_vec_src<ST_S16>(t, base); break;
        default: tile_vec_src<ST_S32>(t, base); break;
        }
        return;
    }
    for (int k = 0; k < CONV_TILE / CV_THREADS; ++k) {
        const int64_t i = base + (int64_t)k * CV_THREADS + threadIdx.x;
        if (i < t.numel) {
            int64_t m, v;
            decode(t, i, m, v);
            encode(t, i, m, v);
        }
    }
}

}  // namespace

hipError_t launch_convert(const ConvDesc *d, const long long *tile_begin, int n, long long tiles, hipStream_t s)
{
    if (n <= 0 || tiles <= 0) return hipSuccess;
    convert_kernel<<<dim3((unsigned)tiles), dim3(CV_THREADS), 0, s>>>(d, n, tile_begin);
    return hipGetLastError();
}

}  // namespace mdq
