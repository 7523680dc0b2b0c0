// mdq_desc.h -- per-tensor descriptor of the multi-tensor launch.
//
// The host launcher (mdq_capi.cpp) packs one MdqDesc per tensor into a single
// device buffer; the kernel walks the whole param/grad/state list from it.
// Each tensor owns the contiguous global tile range [tile_begin, tile_end);
// a tile is one workgroup (tile_elems below) and never straddles two tensors.
#pragma once
#include <stdint.h>

namespace mdq {

enum Storage : int { ST_P4 = 0, ST_S8 = 1, ST_S16 = 2, ST_S32 = 3 };
enum GradType : int { GT_F32 = 0, GT_BF16 = 1, GT_F16 = 2 };

enum DescFlags : uint32_t {
    DF_ALIGNED = 1u,        // every pointer meets the vector-access alignment
    DF_CODES_ALIGNED = 2u,  // the code pointers do (p and grads may not)
    DF_LINES = 4u,          // DF_ALIGNED, and p and grads start on 128-byte lines
};

struct alignas(16) MdqDesc {
    float *p;             // [numel] fp32 params, updated in place
    const void *g;        // [numel] grads (GradType of the launch)
    void *code_m;         // P4: packed bytes; else int8/16/32 m codes
    void *code_v;         // P4: unused; else uint8/16/32 v codes
    float *scale_m;       // [nblocks]
    float *scale_v;       // [nblocks]
    float *v_min;         // [nblocks]
    int64_t numel;
    int64_t tile_begin;
    int64_t tile_end;
    // AdamW constants of this tensor (host-computed once per step).
    float b1, omb1, b2, omb2;
    float eps;
    float step_size;      // lr / (1 - beta1^t)
    float inv_sqrt_bc2;   // 1 / sqrt(1 - beta2^t)
    float decay;          // 1 - lr * weight_decay (1 when weight_decay == 0)
    // Code range: m in [-qm, qm - 1], v in [0, qvf]; inv_qm = 1 / qm (a power of
    // two); qvf = (float)(2^bits - 1), the reference's divisor, inv_qvf = RN(1 / qvf).
    float qm, inv_qvf, inv_qm, qvf;
    uint32_t bits;
    uint32_t step;
    uint32_t tensor_id;
    uint32_t flags;
    // Destination codes of a storage-changing step (the source codes are
    // code_m / code_v); unused when the storage stays.
    void *out_m;
    void *out_v;
    // Index of element 0 in the tensor's stochastic-rounding stream (a
    // multiple of B; nonzero for a piece of a larger tensor).
    int64_t rng_origin;
    // The rounding terms of the fast v-code paths' error bounds for this width
    // (mdq_rn_ep0 / mdq_sr_ep0 of qvf).
    float ep0_rn, ep0_sr;
};

static_assert(sizeof(MdqDesc) == 176, "descriptor layout: 176 bytes, 16-byte sized");

// Kernel arguments of a step launch besides its table: the stochastic-rounding
// key and, when every tensor of the launch has the same step_size,
// inv_sqrt_bc2 and step (uniform != 0), those three values.  The descriptors
// then hold 0 in those fields, so the table of a fixed tensor set is the same
// at every step and the host can launch again from a device copy it already
// holds, without an upload.
struct StepArgs {
    unsigned long long seed;
    float step_size;
    float inv_sqrt_bc2;
    uint32_t step;
    uint32_t uniform;
};

// Tile geometry shared by the host launcher and the kernel: a quant block of
// B elements is owned by B/EPL lanes (EPL = min(B, 8) elements per lane, 16 at
// B = 1024, so that a block fits one wave); a workgroup is one wave (two if a
// block needed more than 64 lanes), and one tile is one workgroup.  B = 1024
// as one wave of 16 elements per lane instead of two waves of 8 with an LDS
// exchange and barriers between them: LLaMA-7B 4-bit step 13.66 -> 12.88 ms,
// stochastic rounding 14.34 -> 12.93 ms, 8-bit 16.76 -> 15.65 ms (same
// allocation).  Only blocks of 64 lanes take the plain element layout, which
// handles any number of quads per lane; the paired layout (8, 16 or 32 lanes
// per block) keeps 8 elements per lane.
constexpr int tile_epl(int B) { return B >= 1024 ? 16 : B >= 8 ? 8 : B; }
constexpr int tile_threads(int B) { return B / tile_epl(B) > 64 ? 2 * 64 : 64; }
constexpr int tile_elems(int B) { return tile_threads(B) * tile_epl(B); }

}  // namespace mdq
