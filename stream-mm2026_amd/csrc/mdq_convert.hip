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
// One workgroup per 4096-element tile of one tensor, one element per thread
// and iteration (the codes are 1-4 bytes wide; this runs on bit-width changes
// only).
#include <hip/hip_runtime.h>

#include "mdq_convert.h"
#include "mdq_desc.h"

namespace mdq {

namespace {

constexpr int CV_THREADS = 256;

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
