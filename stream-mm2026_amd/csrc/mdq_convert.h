// mdq_convert.h -- descriptor and launcher of the code-storage conversion
// (mdq_convert.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mdq {

constexpr int CONV_TILE = 4096;   // elements per workgroup tile

// One tensor's codes: numel elements from storage src (mdq::Storage) at
// src_m / src_v to storage dst at dst_m / dst_v (the v pointer is unused for
// ST_P4).  Tiles [tile_begin, tile_begin + ceil(numel / CONV_TILE)).
struct alignas(16) ConvDesc {
    const void *src_m;
    const void *src_v;
    void *dst_m;
    void *dst_v;
    int64_t numel;
    int64_t tile_begin;
    int32_t src, dst;
    int64_t pad;
};

static_assert(sizeof(ConvDesc) == 64, "ConvDesc layout");

hipError_t launch_convert(const ConvDesc *d, const long long *tile_begin, int n, long long tiles, hipStream_t s);

}  // namespace mdq
