// mdq_stats.h -- descriptor and launcher of the multi-tensor gradient
// statistics (mdq_stats.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mdq {

// Elements per workgroup tile of the partial-sum kernel (512 threads x 64).
constexpr int STAT_TILE = 32768;
constexpr int STAT_PARTIALS = 4;   // doubles per tile

// One tensor of a statistics launch: tiles [tile_begin, tile_end) of the
// launch cover its numel elements (none when numel == 0).
struct alignas(16) StatDesc {
    const void *g;
    int64_t numel;
    int64_t tile_begin;
    int64_t tile_end;
};

static_assert(sizeof(StatDesc) == 32, "StatDesc layout");

// partials: 4 doubles per tile (sum g, sum of squared deviations from the tile
// mean, sum g^2, sum |g|); out: 3 floats per tensor (n_l, r_l, v_l).
hipError_t launch_grad_stats(const StatDesc *d, const long long *tile_begin, int n, long long tiles,
                             int grad_dt, double *partials, float *out, hipStream_t s);

}  // namespace mdq
