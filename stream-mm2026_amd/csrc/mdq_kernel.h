// mdq_kernel.h -- the fused dequant -> AdamW -> requant step for gfx950.
//
// One launch walks every tensor of a (code storage, grad dtype, block size,
// rounding) class from a packed MdqDesc table.  The codes are read in a source
// storage and written in a destination storage: the same for an ordinary
// step, different for a step whose bit width changed (the reference's align ->
// kernel -> pack, /root/reference/CUDA/stquant_opt_simple.py:140-280, in one
// pass).  Semantics per element follow /root/reference/CUDA/stquant_kernel.cu:
// 53-401 (see mdq_step_tile below for the line-by-line map); the layout and
// schedule are this file's own:
//
// * A tile is one wave x EPL elements (EPL = 8 for 8 <= B <= 512, 16 for
//   B = 1024; tile_epl), one workgroup per tile.  A quant block of B elements is owned by
//   LPB = B/EPL consecutive lanes; lane j of a block owns quads j, j+LPB, ...,
//   so every 16-lane row reads one contiguous 256-byte span per 16-byte load,
//   or, when 1-byte codes are involved and LPB is 8, 16 or 32, the permuted
//   quads of paired_codes below (8-byte code accesses plus one lane swap).
// * Block reductions (max|m|, max/min log v) run in registers, then across
//   the LPB lanes with DPP row operations (quad_perm, row_half_mirror,
//   row_mirror), ds_swizzle for 32 lanes, ds_bpermute for 64 (and an LDS
//   exchange between the waves of a block wider than one wave, which the tile
//   geometry of tile_epl never forms).  They skip NaN as
//   the reference's fmaxf / fminf trees do, and non-finite quotients give
//   code 0, as its (int) conversion of NaN does.
// * A tile whose params do not start on a 128-byte line (views of one buffer)
//   writes them line by line through LDS (store_p_lines).
// * Packed 4-bit v codes dequantise through a 16-entry exp table per block
//   built in LDS (16 exp per block instead of one per element).
// * Requant uses mdq_round_half_away (exact fp32) for code widths <= 16 bits
//   and the reference's FP64 divide + round for wider codes.
// * The parameter update uses v_sqrt_f32 / v_rcp_f32 (the tolerance on p is
//   1e-6 relative; codes and scales are exact).
#pragma once
#include <hip/hip_runtime.h>

#include "mdq_desc.h"
#include "mdq_math.h"

namespace mdq {

// |v_log_f32(x) * ln 2 - mdq_logf(x)| <= MDQ_LOG_APPROX_ERR + MDQ_LOG_APPROX_SLOPE *
// |mdq_logf(x)| for every float x in [1e-12, FLT_MAX].  Measured on gfx950 over
// all those inputs (stq_device_log_approx_error): the difference never exceeds
// 1.8e-7 |mdq_logf(x)|, and 9.114e-6 in absolute terms.
#define MDQ_LOG_APPROX_SLOPE 2.0e-7f
#define MDQ_LOG_APPROX_ERR 2.5e-7f
// Relative error bound of the fast v-code path's c1 + that of its c0 (each
// within 2^-24 (1 + 2^-16) of the exact quotient; mdq_vcode_map).
#define MDQ_VCODE_MAP_ERR 1.3e-7f
// The stochastic v code's fast path.  The exact code is floor(T), T = fl(fma(u, fl(1/dv), uv)),
// u = fl(log x - vmin), uv = (k + 1/2) 2^-16 with k the element's 16-bit random half.  The path
// evaluates Zh = fl(z + uvh), z = fl(log2_hw(x) c1 + c0) with c1, c0 from mdq_vcode_map (as the
// nearest path) and uvh = uv - 1/2 (exact: mdq_u16_uniform_minus_half), so that Zh approximates
// T - 1/2.  |Zh - (T - 1/2)| <= ep, the sum of
// - the hardware log and the quotients c1, c0 (the nearest path's term): (A + (S + 1.3e-7) L) / dv,
//   L = max(|lmax|, |lmin|) >= |log x| and >= |vmin| in the block;
// - the roundings of u, of z, of u / dv vs u fl(1/dv), of T and of Zh (|z|, |Zh| < QV + 1):
//   5 (QV + 2) 2^-24 < 3e-7 (QV + 2),
// with r = v_rcp_f32(dv) for 1 / dv (the factor 1.001 covers the difference; the last term is
// the descriptor's ep0_sr, mdq_sr_ep0).  Where Zh lies farther than ep from a half-integer,
// T - 1/2 lies within 1/2 of k = rint(Zh), so k < T < k + 1 and floor(T) = k.  Checked against
// fp64 on the device (stq_device_math, which 4).
struct SrVFast {
    float c1, c0, ep;
};
// max(|lmax|, |vmin|) for vmin <= lmax, both finite: max(lmax, -vmin), one instruction (written
// out: the compiler's maxnum first quiets both operands, two more instructions)
__device__ __forceinline__ float mdq_log_span(float lmax, float vmin)
{
#if defined(__HIP_DEVICE_COMPILE__)
    float r;
    __asm__("v_max_f32_e64 %0, %1, -%2" : "=v"(r) : "v"(lmax), "v"(vmin));
    return r;
#else
    return lmax > -vmin ? lmax : -vmin;
#endif
}
__device__ __forceinline__ SrVFast mdq_sr_vfast(float dv, float vmin, float lmax, float ep0_sr)
{
    const VCodeMap vm = mdq_vcode_map(dv, vmin);
    const float L = mdq_log_span(lmax, vmin);
    const float ep = fma_(fma_(L, MDQ_LOG_APPROX_SLOPE + MDQ_VCODE_MAP_ERR, MDQ_LOG_APPROX_ERR), vm.r * 1.001f, ep0_sr);
    return {vm.c1, vm.c0, ep};
}
// Zh for x = v + 1e-12 and the element's uvh = uv - 1/2 (see mdq_sr_vfast).
__device__ __forceinline__ float mdq_sr_vfast_z(float x, float uvh, const SrVFast &f)
{
    return fma_(__builtin_amdgcn_logf(x), f.c1, f.c0) + uvh;
}

// Lanes per block of the paired code layout (paired_codes).
constexpr bool paired_lpb(int lpb) { return lpb == 8 || lpb == 16 || lpb == 32; }

template <int LOG2B>
struct Cfg {
    static constexpr int B = 1 << LOG2B;
    static constexpr int EPL = tile_epl(B);                // elements per lane
    static constexpr int LPB = B / EPL;                    // lanes per quant block
    static constexpr int QPL = EPL >= 4 ? EPL / 4 : 0;     // 4-element quads per lane
    static constexpr int WAVES = LPB > 64 ? LPB / 64 : 1;  // waves per workgroup (tile); 1 for every B
    static_assert(!(paired_lpb(LPB) && EPL != 8), "the paired code layout moves two quads per lane");
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int TILE = THREADS * EPL;             // elements per tile
    static constexpr int TB = TILE / B;                    // quant blocks per tile
    static_assert(TB * B == TILE, "tile must hold whole blocks");
    static_assert(EPL == tile_epl(B) && THREADS == tile_threads(B) && TILE == tile_elems(B),
                  "kernel tile geometry must match the host launcher's");
};

// Native vector types for the streaming accesses (the nontemporal builtins
// take clang vector types, not HIP's struct vectors).
typedef float vf4 __attribute__((ext_vector_type(4)));
typedef uint32_t vu2 __attribute__((ext_vector_type(2)));
typedef uint32_t vu4 __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) global accesses: every byte of p, g and the codes
// is touched once per step, so they bypass cache allocation.
// The tensor pointers come from the descriptor table, so the compiler cannot
// infer their address space; casting to address space 1 (global) turns the
// accesses into global_* instead of flat_* instructions.
#define MDQ_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ T ld_nt(const void *a) { return __builtin_nontemporal_load((const MDQ_GLOBAL T *)a); }
template <class T>
__device__ __forceinline__ void st_nt(T v, void *a) { __builtin_nontemporal_store(v, (MDQ_GLOBAL T *)a); }
// The same streaming accesses for an address aligned only to A bytes (a view at an
// arbitrary element offset): gfx9 global loads and stores take any alignment
// (the compiler's unaligned-buffer-access feature of this target; it emits the
// same single dwordx4 / dwordx2 instruction), at the cost of touching one more
// cache line per wave instruction.
template <class T, int A>
__device__ __forceinline__ T ld_nt_al(const void *a)
{
    typedef T TA __attribute__((aligned(A)));
    return __builtin_nontemporal_load((const MDQ_GLOBAL TA *)a);
}
template <class T, int A>
__device__ __forceinline__ void st_nt_al(T v, void *a)
{
    typedef T TA __attribute__((aligned(A)));
    __builtin_nontemporal_store(v, (MDQ_GLOBAL TA *)a);
}
template <class T>
__device__ __forceinline__ T ld_g(const void *a) { return *(const MDQ_GLOBAL T *)a; }
template <class T>
__device__ __forceinline__ void st_g(T v, void *a) { *(MDQ_GLOBAL T *)a = v; }

constexpr bool one_byte_codes(int st) { return st == ST_P4 || st == ST_S8; }

// Element layout of a tile whose codes are read in storage SRC and written in
// storage DST (the same storage except on a storage-changing step).
template <int SRC, int DST, int LOG2B>
constexpr bool paired_codes()
{
    // 1-byte codes (packed 4-bit, or int8 + uint8), 8, 16 or 32 lanes per block: each lane
    // moves its codes as one contiguous 8-byte access per array (full 128-byte lines per
    // instruction) and swaps half of them with lane j ^ LPB/2, so the lane's quads are
    // k*LPB + pi(j) with pi(j) = 2 (j mod LPB/2) + j div LPB/2 for every array.  LLaMA set,
    // same-box A/B against 4-byte quad accesses: packed 4-bit -3.4 %, int8 + uint8 -6 %.
    // Wider codes on the other side of a storage change move as 4-element quads at the
    // same permuted quad positions.
    return (one_byte_codes(SRC) || one_byte_codes(DST)) && paired_lpb(Cfg<LOG2B>::LPB);
}

// Quad k (0 .. QPL-1) of lane j within its quant block.
template <bool PAIRED, int LOG2B>
__device__ __forceinline__ int lane_quad(int j, int k)
{
    constexpr int LPB = Cfg<LOG2B>::LPB, H = LPB / 2;
    if constexpr (PAIRED) return k * LPB + 2 * (j % H) + j / H;
    else return j + k * LPB;
}

// Offset within the quant block of the lane's element e.
template <bool PAIRED, int LOG2B>
__device__ __forceinline__ int elem_off(int j, int e)
{
    using C = Cfg<LOG2B>;
    if constexpr (C::QPL > 0) return 4 * lane_quad<PAIRED, LOG2B>(j, e >> 2) + (e & 3);
    else return e;
}

// x from lane j ^ H (H = 8: DPP row_ror:8 within a 16-lane row; H = 4 or 16: ds_swizzle in
// bit mode with xor mask H).
template <int H>
__device__ __forceinline__ uint32_t swap_half(uint32_t x)
{
    static_assert(H == 4 || H == 8 || H == 16, "lane pairs at distance 4, 8 or 16");
    if constexpr (H == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, true);
    else return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, (H << 10) | 0x1F);
}

// Paired code layout (paired_codes): lane j reads bytes [8j, 8j + 8) of its block's codes
// (quads 2j, 2j + 1) and keeps / receives its own quads pi(j) (k = 0) and LPB + pi(j) (k = 1);
// pair_out is the inverse for the store.
template <int H>
__device__ __forceinline__ uint32_t pair_in(vu2 w, int j, int k)
{
    const bool lo = j < H;
    const uint32_t y = swap_half<H>(lo ? w.y : w.x);
    return k == 0 ? (lo ? w.x : y) : (lo ? y : w.y);
}

template <int H>
__device__ __forceinline__ vu2 pair_out(uint32_t q0, uint32_t q1, int j)
{
    const bool lo = j < H;
    const uint32_t y = swap_half<H>(lo ? q1 : q0);
    return lo ? vu2{q0, y} : vu2{y, q1};
}

// ---------------------------------------------------------------- grad loads
template <int GT> struct GradIO;
template <> struct GradIO<GT_F32> {
    // four grads from LDS at a 4-byte aligned address
    static __device__ __forceinline__ void lds4(const char *a, float *o) {
        const float *q = (const float *)a;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = q[c];
    }
    // four grads from LDS at a 16-byte aligned address (one 16-byte read)
    static __device__ __forceinline__ void lds4a(const char *a, float *o) {
        const vf4 v = *(const vf4 *)a;
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    static __device__ __forceinline__ void load4(const void *g, int64_t i, float *o) {
        vf4 v = ld_nt<vf4>(static_cast<const float *>(g) + i);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    // four grads at an address aligned only to the element size
    static __device__ __forceinline__ void load4u(const void *g, int64_t i, float *o) {
        vf4 v = ld_nt_al<vf4, 4>(static_cast<const float *>(g) + i);
        o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    }
    static __device__ __forceinline__ float load1(const void *g, int64_t i) {
        return ld_g<float>(static_cast<const float *>(g) + i);
    }
    static __device__ __forceinline__ float load1nt(const void *g, uint32_t i) {
        return ld_nt<float>(static_cast<const float *>(g) + i);
    }
};
template <> struct GradIO<GT_BF16> {
    static __device__ __forceinline__ void lds4(const char *a, float *o) {
        const uint16_t *q = (const uint16_t *)a;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = bits_f((uint32_t)q[c] << 16);
    }
    // four grads from LDS at an 8-byte aligned address (one 8-byte read)
    static __device__ __forceinline__ void lds4a(const char *a, float *o) { unpack(*(const vu2 *)a, o); }
    static __device__ __forceinline__ void unpack(vu2 v, float *o) {
        o[0] = bits_f(v.x << 16); o[1] = bits_f(v.x & 0xffff0000u);
        o[2] = bits_f(v.y << 16); o[3] = bits_f(v.y & 0xffff0000u);
    }
    static __device__ __forceinline__ void load4(const void *g, int64_t i, float *o) {
        unpack(ld_nt<vu2>(static_cast<const uint16_t *>(g) + i), o);
    }
    static __device__ __forceinline__ void load4u(const void *g, int64_t i, float *o) {
        unpack(ld_nt_al<vu2, 2>(static_cast<const uint16_t *>(g) + i), o);
    }
    static __device__ __forceinline__ float load1(const void *g, int64_t i) {
        return bits_f((uint32_t)ld_g<uint16_t>(static_cast<const uint16_t *>(g) + i) << 16);
    }
    static __device__ __forceinline__ float load1nt(const void *g, uint32_t i) {
        return bits_f((uint32_t)ld_nt<uint16_t>(static_cast<const uint16_t *>(g) + i) << 16);
    }
};
template <> struct GradIO<GT_F16> {
    static __device__ __forceinline__ void lds4(const char *a, float *o) {
        const uint16_t *q = (const uint16_t *)a;
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = (float)__builtin_bit_cast(_Float16, q[c]);
    }
    // four grads from LDS at an 8-byte aligned address (one 8-byte read)
    static __device__ __forceinline__ void lds4a(const char *a, float *o) { unpack(*(const vu2 *)a, o); }
    static __device__ __forceinline__ float h2f(uint32_t h) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    }
    static __device__ __forceinline__ void unpack(vu2 v, float *o) {
        o[0] = h2f(v.x & 0xffffu); o[1] = h2f(v.x >> 16);
        o[2] = h2f(v.y & 0xffffu); o[3] = h2f(v.y >> 16);
    }
    static __device__ __forceinline__ void load4(const void *g, int64_t i, float *o) {
        unpack(ld_nt<vu2>(static_cast<const uint16_t *>(g) + i), o);
    }
    static __device__ __forceinline__ void load4u(const void *g, int64_t i, float *o) {
        unpack(ld_nt_al<vu2, 2>(static_cast<const uint16_t *>(g) + i), o);
    }
    static __device__ __forceinline__ float load1(const void *g, int64_t i) {
        return h2f(ld_g<uint16_t>(static_cast<const uint16_t *>(g) + i));
    }
    static __device__ __forceinline__ float load1nt(const void *g, uint32_t i) {
        return h2f(ld_nt<uint16_t>(static_cast<const uint16_t *>(g) + i));
    }
};

// ---------------------------------------------------------------- code I/O
// mc: the m code as float (for packed nibbles the stored nibble q + 8, which
// dequant_m offsets by 8); vc: the raw v code.
template <int ST> struct CodeIO;
template <> struct CodeIO<ST_P4> {
    static __device__ __forceinline__ void load4(const MdqDesc &d, int64_t i, float *mc, uint32_t *vc) {
        const uint32_t w = ld_nt<uint32_t>(static_cast<const uint8_t *>(d.code_m) + i);
        const uint32_t lo = w & 0x0f0f0f0fu;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            mc[k] = (float)((lo >> (8 * k)) & 0xffu);
            vc[k] = (w >> (8 * k + 4)) & 15u;
        }
    }
    static __device__ __forceinline__ void load1(const MdqDesc &d, int64_t i, float &mc, uint32_t &vc) {
        uint32_t b = ld_g<uint8_t>(static_cast<const uint8_t *>(d.code_m) + i);
        mc = (float)(b & 15u);
        vc = b >> 4;
    }
    // The paired layout's codes in two steps: raw8 issues the lane's 8-byte load, decode8
    // (after every load of the tile is in flight) swaps half of it with the pair lane.
    // vc receives 4 x the v code: the byte offset of its entry in the block's exp table.
    // Both nibble fields are masked once per word (the empty asm keeps the masks from being
    // folded into per-element bit-field extracts), so each element takes one byte-select
    // conversion (m) and one byte-select add (the table address).
    typedef vu2 Raw8;
    static __device__ __forceinline__ Raw8 raw8(const MdqDesc &d, uint32_t blk_off, int j) {
        return ld_nt<vu2>(static_cast<const uint8_t *>(d.code_m) + blk_off + 8 * j);
    }
    template <int H>
    static __device__ __forceinline__ void decode8(Raw8 w, int j, float *mc, uint32_t *vc) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t q = pair_in<H>(w, j, h);
            uint32_t lo = q & 0x0f0f0f0fu;
            uint32_t v4 = (q >> 2) & 0x3c3c3c3cu;
            asm volatile("" : "+v"(lo), "+v"(v4));
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                mc[4 * h + k] = (float)((lo >> (8 * k)) & 0xffu);
                vc[4 * h + k] = (v4 >> (8 * k)) & 0xffu;
            }
        }
    }
    template <int H>
    static __device__ __forceinline__ void store8f(const MdqDesc &d, uint32_t blk_off, int j, const float *pk) {
        uint32_t q[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(pk[4 * h + 0], 0, 0u);
            w = __builtin_amdgcn_cvt_pk_u8_f32(pk[4 * h + 1], 1, w);
            w = __builtin_amdgcn_cvt_pk_u8_f32(pk[4 * h + 2], 2, w);
            q[h] = __builtin_amdgcn_cvt_pk_u8_f32(pk[4 * h + 3], 3, w);
        }
        st_nt<vu2>(pair_out<H>(q[0], q[1], j), static_cast<uint8_t *>(d.code_m) + blk_off + 8 * j);
    }
    // byte values already formed as floats (exact integers 0..255)
    static __device__ __forceinline__ void store4f(const MdqDesc &d, int64_t i, const float *pk) {
        uint32_t w = __builtin_amdgcn_cvt_pk_u8_f32(pk[0], 0, 0u);
        w = __builtin_amdgcn_cvt_pk_u8_f32(pk[1], 1, w);
        w = __builtin_amdgcn_cvt_pk_u8_f32(pk[2], 2, w);
        w = __builtin_amdgcn_cvt_pk_u8_f32(pk[3], 3, w);
        st_nt<uint32_t>(w, static_cast<uint8_t *>(d.code_m) + i);
    }
    static __device__ __forceinline__ void store1f(const MdqDesc &d, int64_t i, float pk) {
        st_g<uint8_t>((uint8_t)(uint32_t)pk, static_cast<uint8_t *>(d.code_m) + i);
    }
    static __device__ __forceinline__ uint32_t pack(int32_t qm, uint32_t qv) {
        return (qv << 4) | (uint32_t)(qm + 8);
    }
    static __device__ __forceinline__ void store4(const MdqDesc &d, int64_t i, const int32_t *qm, const uint32_t *qv) {
        uint32_t w = pack(qm[0], qv[0]) | (pack(qm[1], qv[1]) << 8) |
                     (pack(qm[2], qv[2]) << 16) | (pack(qm[3], qv[3]) << 24);
        st_nt<uint32_t>(w, static_cast<uint8_t *>(d.code_m) + i);
    }
    static __device__ __forceinline__ void store1(const MdqDesc &d, int64_t i, int32_t qm, uint32_t qv) {
        st_g<uint8_t>((uint8_t)pack(qm, qv), static_cast<uint8_t *>(d.code_m) + i);
    }
};
template <> struct CodeIO<ST_S8> {
    static __device__ __forceinline__ void load4(const MdqDesc &d, int64_t i, float *mc, uint32_t *vc) {
        uint32_t wm = ld_nt<uint32_t>(static_cast<const int8_t *>(d.code_m) + i);
        uint32_t wv = ld_nt<uint32_t>(static_cast<const uint8_t *>(d.code_v) + i);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            mc[k] = (float)(int8_t)(wm >> (8 * k));
            vc[k] = (wv >> (8 * k)) & 0xffu;
        }
    }
    static __device__ __forceinline__ void load1(const MdqDesc &d, int64_t i, float &mc, uint32_t &vc) {
        mc = (float)ld_g<int8_t>(static_cast<const int8_t *>(d.code_m) + i);
        vc = ld_g<uint8_t>(static_cast<const uint8_t *>(d.code_v) + i);
    }
    // the paired layout's m and v codes: raw8 loads, decode8 swaps and converts (CodeIO<ST_P4>)
    typedef vu4 Raw8;
    static __device__ __forceinline__ Raw8 raw8(const MdqDesc &d, uint32_t blk_off, int j) {
        const vu2 wm = ld_nt<vu2>(static_cast<const int8_t *>(d.code_m) + blk_off + 8 * j);
        const vu2 wv = ld_nt<vu2>(static_cast<const uint8_t *>(d.code_v) + blk_off + 8 * j);
        return vu4{wm.x, wm.y, wv.x, wv.y};
    }
    template <int H>
    static __device__ __forceinline__ void decode8(Raw8 w, int j, float *mc, uint32_t *vc) {
        const vu2 wm = {w.x, w.y}, wv = {w.z, w.w};
        const uint32_t m0 = pair_in<H>(wm, j, 0), m1 = pair_in<H>(wm, j, 1);
        const uint32_t v0 = pair_in<H>(wv, j, 0), v1 = pair_in<H>(wv, j, 1);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            mc[k] = (float)(int8_t)(m0 >> (8 * k));
            mc[4 + k] = (float)(int8_t)(m1 >> (8 * k));
            vc[k] = (v0 >> (8 * k)) & 0xffu;
            vc[4 + k] = (v1 >> (8 * k)) & 0xffu;
        }
    }
    template <int H>
    static __device__ __forceinline__ void store8(const MdqDesc &d, uint32_t blk_off, int j, const int32_t *qm,
                                                  const uint32_t *qv) {
        uint32_t wm[2] = {0, 0}, wv[2] = {0, 0};
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                wm[q] |= ((uint32_t)qm[4 * q + k] & 0xffu) << (8 * k);
                wv[q] |= (qv[4 * q + k] & 0xffu) << (8 * k);
            }
        st_nt<vu2>(pair_out<H>(wm[0], wm[1], j), static_cast<int8_t *>(d.code_m) + blk_off + 8 * j);
        st_nt<vu2>(pair_out<H>(wv[0], wv[1], j), static_cast<uint8_t *>(d.code_v) + blk_off + 8 * j);
    }
    static __device__ __forceinline__ void store4(const MdqDesc &d, int64_t i, const int32_t *qm, const uint32_t *qv) {
        uint32_t wm = 0, wv = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            wm |= ((uint32_t)qm[k] & 0xffu) << (8 * k);
            wv |= (qv[k] & 0xffu) << (8 * k);
        }
        st_nt<uint32_t>(wm, static_cast<int8_t *>(d.code_m) + i);
        st_nt<uint32_t>(wv, static_cast<uint8_t *>(d.code_v) + i);
    }
    static __device__ __forceinline__ void store1(const MdqDesc &d, int64_t i, int32_t qm, uint32_t qv) {
        st_g<int8_t>((int8_t)qm, static_cast<int8_t *>(d.code_m) + i);
        st_g<uint8_t>((uint8_t)qv, static_cast<uint8_t *>(d.code_v) + i);
    }
};
template <> struct CodeIO<ST_S16> {
    static __device__ __forceinline__ void load4(const MdqDesc &d, int64_t i, float *mc, uint32_t *vc) {
        vu2 wm = ld_nt<vu2>(static_cast<const int16_t *>(d.code_m) + i);
        vu2 wv = ld_nt<vu2>(static_cast<const uint16_t *>(d.code_v) + i);
        mc[0] = (float)(int16_t)wm.x; mc[1] = (float)(int16_t)(wm.x >> 16);
        mc[2] = (float)(int16_t)wm.y; mc[3] = (float)(int16_t)(wm.y >> 16);
        vc[0] = wv.x & 0xffffu; vc[1] = wv.x >> 16; vc[2] = wv.y & 0xffffu; vc[3] = wv.y >> 16;
    }
    static __device__ __forceinline__ void load1(const MdqDesc &d, int64_t i, float &mc, uint32_t &vc) {
        mc = (float)ld_g<int16_t>(static_cast<const int16_t *>(d.code_m) + i);
        vc = ld_g<uint16_t>(static_cast<const uint16_t *>(d.code_v) + i);
    }
    static __device__ __forceinline__ void store4(const MdqDesc &d, int64_t i, const int32_t *qm, const uint32_t *qv) {
        vu2 wm, wv;
        wm.x = ((uint32_t)qm[0] & 0xffffu) | ((uint32_t)qm[1] << 16);
        wm.y = ((uint32_t)qm[2] & 0xffffu) | ((uint32_t)qm[3] << 16);
        wv.x = (qv[0] & 0xffffu) | (qv[1] << 16);
        wv.y = (qv[2] & 0xffffu) | (qv[3] << 16);
        st_nt<vu2>(wm, static_cast<int16_t *>(d.code_m) + i);
        st_nt<vu2>(wv, static_cast<uint16_t *>(d.code_v) + i);
    }
    static __device__ __forceinline__ void store1(const MdqDesc &d, int64_t i, int32_t qm, uint32_t qv) {
        st_g<int16_t>((int16_t)qm, static_cast<int16_t *>(d.code_m) + i);
        st_g<uint16_t>((uint16_t)qv, static_cast<uint16_t *>(d.code_v) + i);
    }
};
template <> struct CodeIO<ST_S32> {
    static __device__ __forceinline__ void load4(const MdqDesc &d, int64_t i, float *mc, uint32_t *vc) {
        vu4 wm = ld_nt<vu4>(static_cast<const int32_t *>(d.code_m) + i);
        vu4 wv = ld_nt<vu4>(static_cast<const uint32_t *>(d.code_v) + i);
        mc[0] = (float)(int32_t)wm.x; mc[1] = (float)(int32_t)wm.y;
        mc[2] = (float)(int32_t)wm.z; mc[3] = (float)(int32_t)wm.w;
        vc[0] = wv.x; vc[1] = wv.y; vc[2] = wv.z; vc[3] = wv.w;
    }
    static __device__ __forceinline__ void load1(const MdqDesc &d, int64_t i, float &mc, uint32_t &vc) {
        mc = (float)ld_g<int32_t>(static_cast<const int32_t *>(d.code_m) + i);
        vc = ld_g<uint32_t>(static_cast<const uint32_t *>(d.code_v) + i);
    }
    static __device__ __forceinline__ void store4(const MdqDesc &d, int64_t i, const int32_t *qm, const uint32_t *qv) {
        vu4 wm = {(uint32_t)qm[0], (uint32_t)qm[1], (uint32_t)qm[2], (uint32_t)qm[3]};
        vu4 wv = {qv[0], qv[1], qv[2], qv[3]};
        st_nt<vu4>(wm, static_cast<int32_t *>(d.code_m) + i);
        st_nt<vu4>(wv, static_cast<uint32_t *>(d.code_v) + i);
    }
    static __device__ __forceinline__ void store1(const MdqDesc &d, int64_t i, int32_t qm, uint32_t qv) {
        st_g<int32_t>(qm, static_cast<int32_t *>(d.code_m) + i);
        st_g<uint32_t>(qv, static_cast<uint32_t *>(d.code_v) + i);
    }
};

// The raw words of CodeIO<ST>::raw8 (storages without the paired layout: unused).
template <int ST> struct Raw8Of { typedef int type; };
template <> struct Raw8Of<ST_P4> { typedef CodeIO<ST_P4>::Raw8 type; };
template <> struct Raw8Of<ST_S8> { typedef CodeIO<ST_S8>::Raw8 type; };

// ------------------------------------------------------- cross-lane reduction
// Block reductions run on integer keys: |m| >= 0 orders like its bit pattern,
// and log v maps to a signed key that orders like the float (negative values
// get their magnitude bits flipped).  Integer max/min need no NaN
// canonicalisation, so the DPP row operations fold into them.
__device__ __forceinline__ int32_t f2key(float x)
{
    const int32_t b = __builtin_bit_cast(int32_t, x);
    return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float key2f(int32_t k) { return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7fffffff)); }

template <int CTRL>
__device__ __forceinline__ int32_t dpp_i(int32_t x) { return __builtin_amdgcn_mov_dpp(x, CTRL, 0xF, 0xF, true); }

template <bool IS_MAX>
__device__ __forceinline__ int32_t iop(int32_t a, int32_t b) { return IS_MAX ? (a > b ? a : b) : (a < b ? a : b); }

// Reduce over aligned groups of LANES lanes (LANES <= 64); every lane of the
// group receives the result.
template <int LANES, bool IS_MAX>
__device__ __forceinline__ int32_t group_reduce(int32_t x)
{
    if constexpr (LANES >= 2) x = iop<IS_MAX>(x, dpp_i<0xB1>(x));   // quad_perm [1,0,3,2]
    if constexpr (LANES >= 4) x = iop<IS_MAX>(x, dpp_i<0x4E>(x));   // quad_perm [2,3,0,1]
    if constexpr (LANES >= 8) x = iop<IS_MAX>(x, dpp_i<0x141>(x));  // row_half_mirror
    if constexpr (LANES >= 16) x = iop<IS_MAX>(x, dpp_i<0x140>(x)); // row_mirror
    if constexpr (LANES >= 32) x = iop<IS_MAX>(x, __builtin_amdgcn_ds_swizzle(x, 0x401F));  // lane ^ 16
    if constexpr (LANES >= 64) x = iop<IS_MAX>(x, __shfl_xor(x, 32));
    return x;
}

// Every lane of an aligned group of min(LANES, 64) lanes receives the value
// of the group's first lane: ds_swizzle in bit mode (and-mask clears the low
// lane bits) within 32 lanes, readfirstlane for a whole wave.
template <int LANES>
__device__ __forceinline__ float block_bcast(float x)
{
    if constexpr (LANES <= 1) {
        return x;
    } else if constexpr (LANES <= 32) {
        constexpr int and_mask = 0x1F & ~(LANES - 1);
        return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), and_mask));
    } else {
        return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
    }
}

struct ProfAcc {
    unsigned long long c[5];
};

constexpr int code_size(int st) { return st == ST_S16 ? 2 : st == ST_S32 ? 4 : 1; }

// The descriptor with its element pointers advanced to element `off`
// (workgroup-uniform, so the copies live in scalar registers).
template <int SRC, int DST, int GT>
__device__ __forceinline__ MdqDesc tile_view(const MdqDesc &d, int64_t off)
{
    MdqDesc t = d;
    t.p = d.p + off;
    t.g = static_cast<const char *>(d.g) + off * (GT == GT_F32 ? 4 : 2);
    t.code_m = static_cast<char *>(d.code_m) + off * code_size(SRC);
    if constexpr (SRC != ST_P4) t.code_v = static_cast<char *>(d.code_v) + off * code_size(SRC);
    if constexpr (SRC != DST) {
        t.out_m = static_cast<char *>(d.out_m) + off * code_size(DST);
        if constexpr (DST != ST_P4) t.out_v = static_cast<char *>(d.out_v) + off * code_size(DST);
    }
    return t;
}

// The view the new codes are stored through: the descriptor itself, or on a
// storage-changing step one whose code pointers are the destination's.
template <int SRC, int DST>
__device__ __forceinline__ MdqDesc out_view(const MdqDesc &d)
{
    MdqDesc t = d;
    if constexpr (SRC != DST) {
        t.code_m = d.out_m;
        t.code_v = d.out_v;
    }
    return t;
}

// A storage-changing step first re-stores the old codes as the reference's
// alignment for the new width does (stquant_opt_simple.py:140-173): clamped to
// int8 / uint8 for widths up to 8 bits (destination P4 or S8), to int16 /
// uint16 for 16 bits, unchanged for 32; the old scales are kept.  Only int16
// and int32 sources can fall outside those ranges.
template <int SRC, int DST>
constexpr bool narrows_codes()
{
    constexpr int src_bits = SRC == ST_S16 ? 16 : SRC == ST_S32 ? 32 : 8;
    constexpr int dst_bits = DST == ST_S16 ? 16 : DST == ST_S32 ? 32 : 8;
    return src_bits > dst_bits;
}

// Dequantised m from its stored code.  Packed nibbles hold mu = q + 8;
// ((float)mu - 8) * sm == fma(mu, sm, -8 * sm) exactly (one rounding of the
// same real number; -8*sm is exact), up to the sign of a zero product.
template <int ST>
__device__ __forceinline__ float dequant_m(float code, float sm, float neg8sm)
{
    if constexpr (ST == ST_P4) return fma_(code, sm, neg8sm);
    else return code * sm;
}

// ---------------------------------------------------------------- one tile
// Tile modes.  TILE_VECTOR: every element of the tile lies inside the tensor and
// all pointers are 16-byte aligned (p and grads of a one-wave tile on 128-byte
// lines), so each lane moves its own quads as vectors.  TILE_STAGED (one-wave
// tiles): the tile lies inside the tensor and the codes are aligned, but p or the
// grads do not start on a 128-byte line (views at arbitrary element offsets of one
// buffer, as a flat parameter buffer hands them over).  The lanes' own 16-byte
// pieces would then split lines between instructions, so p and the grads come in
// as whole aligned lines straight into LDS (global_load_lds) and p goes out through
// LDS line by line (store_p_lines); codes move as in TILE_VECTOR.  Config 5 as
// views back to back, B = 64: 64 % of HBM peak with the lanes' own element-aligned
// vectors, 80 % staged, level with separate allocations.  TILE_UNALIGNED_PG (tiles
// of more than one wave, and 32-bit codes with stochastic rounding from B = 256 on,
// staged_mode):
// codes as in TILE_VECTOR, p and grads loaded as the lanes' vectors at element-aligned
// addresses, and p stored through LDS when it does not start on a line.
// TILE_GUARDED: every access element by element, guarded by idx < numel.
enum TileMode : int { TILE_GUARDED = 0, TILE_VECTOR = 1, TILE_UNALIGNED_PG = 2, TILE_STAGED = 3 };

// Whether tiles with p or grads off their 128-byte lines take TILE_STAGED (else
// TILE_UNALIGNED_PG).  Same-allocation A/B on config 5 as packed views, stochastic
// rounding, with the tile's loads all in flight before its first cross-lane DS
// instruction (mdq_step_tile): staged against element-aligned vectors, B = 128 4-bit
// 72.4 -> 78.7 % of HBM peak, 8-bit 74.2 -> 77.8 %; B = 256 4-bit 77.5 -> 79.2 %, 8-bit
// 77.6 -> 78.8 / 77.7 -> 79.0 % (two boxes), 16-bit 77.5 -> 79.4 %; B = 512 4-bit 78.6 ->
// 79.6 %, 8-bit 77.8 -> 78.9 %, 16-bit 77.5 -> 78.0 %; B = 1024 level; 32-bit codes B = 256
// 75.0 -> 74.4 % (kept on element-aligned vectors from B = 256 on).  Nearest rounding:
// faster at every B.
template <int SRC, int DST, bool SR, int LOG2B>
constexpr bool staged_mode()
{
    return Cfg<LOG2B>::QPL > 0 && Cfg<LOG2B>::WAVES == 1 &&
           (!SR || LOG2B <= 7 || (SRC != ST_S32 && DST != ST_S32));
}

// Bytes of LDS a one-wave staged tile uses for the lines of p (4 B per element) and
// of the grads (GB B per element), each with one more line for a start inside a line
// and 16 bytes in front for the shifted base of lines_to_lds.
constexpr int staged_lds_bytes(int tile, int gb) { return 16 + 4 * tile + 128 + 16 + gb * tile + 128; }

// The 128-byte lines that hold src[0 .. NB) (bytes), as aligned 16-byte pieces from
// the line of src's first byte on, into LDS by direct global -> LDS loads
// (non-temporal).  Piece w of the lines lands at lds - s + 16 w with s = off & 12 (the
// direct loads write whole dwords, so the shift is a multiple of 4): src's byte b lands
// at lds + (off & ~12) + b.  For a src on a 4-byte boundary (p, fp32 grads, 2-byte
// grads at even element offsets) its 16-byte groups then start on 16-byte LDS
// addresses (lds is 16-byte aligned with 16 bytes of room in front), and each lane
// reads its quads as one aligned 16-byte (8-byte for 2-byte grads) LDS access.  With
// the lines' own alignment instead, every quad of a view at an odd element offset
// straddles 16-byte groups and takes element-wise reads, which the paired lane order
// turns into 4-way bank conflicts.  Lines are 128-byte aligned, so none crosses a
// page: the bytes around src that they carry lie on pages that src's own bytes map.
// One wave; the caller waits (vmcnt) before reading the LDS.
template <int NB>
__device__ __forceinline__ void lines_to_lds(const void *src, char *lds, uint32_t off, int lane)
{
    const char *l0 = (const char *)src - off;
    lds -= off & 12u;
    const uint32_t nv = ((off + (uint32_t)NB + 127u) >> 7) * 8u;   // pieces of the covering lines
    constexpr int R = (NB / 16 + 8 + 63) / 64;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // the piece of lane l in round r is w = 64 r + l: LDS address = base of the round + 16 l
        if (64u * r + lane < nv)
            __builtin_amdgcn_global_load_lds((const MDQ_GLOBAL void *)(l0 + 1024 * r + 16 * lane),
                                             (__attribute__((address_space(3))) void *)(lds + 1024 * r), 16, 0,
                                             2 /* nt */);
    }
}

// A whole tile's p stores when p does not start on a 128-byte line (pst: TILE floats
// of LDS, 16-byte aligned, holding the tile's new p; dl = the tile's offset in its
// first line, in elements, 1..31).  The lanes' own 16-byte pieces would split every
// line between two store instructions wherever a block's span of lanes does not
// start on a line (every line at B = 64), and partial line writes cost memory time
// far beyond their bytes.  Here the full lines go out as aligned 16-byte vectors
// from one instruction per line, and the two edge lines, which the neighbouring
// tiles (or views) share, element by element through L2 (temporal stores: the two
// halves of such a line then mostly meet in L2 and leave as one line).
template <int THREADS, int TILE>
__device__ __forceinline__ void store_p_lines(float *p, const float *pst, uint32_t dl)
{
    static_assert(TILE % 32 == 0 && TILE >= 64 && THREADS >= 32, "tile geometry of the staged store");
    if constexpr (THREADS == 64) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
        __syncthreads();
    }
    // position q of the tile's lines holds element q - dl: line 0 starts dl
    // elements before the tile, line TILE / 32 ends 32 - dl elements after it
    const uint32_t t = threadIdx.x;
    float *pl = p - dl;
    if (t < 32u) {
        // edge elements: positions dl .. 31 (line 0) and TILE .. TILE + dl - 1 (last line)
        const uint32_t q = t < dl ? TILE + t : t;
        st_g<float>(pst[q - dl], pl + q);
    }
    constexpr int NV = TILE / 4 - 8;                      // 16-byte vectors of lines 1 .. TILE/32 - 1
#pragma unroll
    for (int r = 0; r < (NV + THREADS - 1) / THREADS; ++r) {
        const uint32_t w = t + r * THREADS;
        if (w < (uint32_t)NV) {
            const uint32_t q = 32 + 4 * w, e = q - dl;
            const vf4 o = {pst[e], pst[e + 1], pst[e + 2], pst[e + 3]};
            st_nt<vf4>(o, pl + q);
        }
    }
}

template <int SRC, int DST, int GT, int LOG2B, bool SR, bool VIEWS, int MODE>
__device__ __forceinline__ void mdq_step_tile(const MdqDesc &d, int64_t tl, int lane, int wave,
                                              float *lut, int32_t *xw, float *pst, const StepArgs &sa,
                                              bool prof_on, ProfAcc &pa)
{
    using C = Cfg<LOG2B>;
    constexpr int B = C::B, EPL = C::EPL, LPB = C::LPB;
    constexpr bool USE_LUT = (SRC == ST_P4) && B >= 32;
    constexpr bool PAIRED = paired_codes<SRC, DST, LOG2B>();
    constexpr bool FULL = MODE != TILE_GUARDED;           // the whole tile lies inside the tensor
    constexpr bool VEC_PG = MODE == TILE_VECTOR;          // p and grads 16-byte aligned
    constexpr bool STAGED = MODE == TILE_STAGED;
    // packed codes in the paired layout: vc holds each v code's byte offset in the exp table
    constexpr bool VC_BYTES = FULL && C::QPL > 0 && PAIRED && SRC == ST_P4;
    static_assert(!VC_BYTES || USE_LUT, "the paired packed-code load addresses the exp table");
    static_assert(MODE != TILE_UNALIGNED_PG || C::QPL > 0, "unaligned p/g mode needs 4-element quads");
    static_assert(!STAGED || (C::QPL > 0 && C::WAVES == 1), "the staged mode is for one-wave tiles of quads");
    constexpr uint32_t GB = GT == GT_F32 ? 4u : 2u;       // bytes per grad
    // STAGED: pst holds the lines of p (later the staged p stores), then those of g
    char *const stp = (char *)pst + 16;
    char *const stg = (char *)pst + 16 + 4 * C::TILE + 128 + 16;
    uint32_t offp = 0, offg = 0;                          // p's / g's byte offset in their first line

    unsigned long long t0 = 0;
    if (prof_on) t0 = clock64();
    // the step-dependent constants: kernel arguments when the launch shares them
    [[maybe_unused]] const uint32_t step_no = sa.uniform ? sa.step : d.step;
    const float step_size = sa.uniform ? sa.step_size : d.step_size;
    const float inv_sqrt_bc2 = sa.uniform ? sa.inv_sqrt_bc2 : d.inv_sqrt_bc2;

    int bi, j;
    if constexpr (LPB <= 64) { bi = lane / LPB; j = lane % LPB; }
    else { bi = 0; j = (wave << 6) | lane; }
    const int64_t n = d.numel;
    const int64_t blk = tl * C::TB + bi;
    const int64_t base = blk << LOG2B;
    const bool blk_ok = FULL || base < n;

    // old block scales (stquant_kernel.cu:67-69): the block's first lane of
    // each wave loads them and the block's other lanes take them by broadcast
    // (one active lane per block keeps the small loads from occupying the
    // whole wave's address path).  The broadcasts, like the paired codes' lane
    // swaps, are cross-lane DS instructions, and the compiler makes every DS
    // instruction after a direct global -> LDS load (TILE_STAGED) wait for all
    // loads in flight: they run after every load of the tile is issued and the
    // Philox words are drawn, so the tile makes one memory round trip.
    float sm = 0.0f, sv = 0.0f, vmin = 0.0f;
    const bool loader = (LPB <= 64 ? j == 0 : lane == 0) && blk_ok;
    if (loader) {
        sm = ld_g<float>(d.scale_m + blk);
        sv = ld_g<float>(d.scale_v + blk);
        vmin = ld_g<float>(d.v_min + blk);
    }

    float pv[EPL], gv[EPL], mc[EPL];
    uint32_t vc[EPL];
    bool ok[EPL];
    [[maybe_unused]] typename Raw8Of<SRC>::type craw{};   // paired 1-byte codes as loaded
    // FULL tiles address through a workgroup-uniform tile base (scalar
    // registers) plus a 32-bit lane offset, so loads and stores take the
    // saddr + voffset form instead of 64-bit per-lane address arithmetic.
    const int64_t tbase = tl * C::TILE;
    const uint32_t lbase = (uint32_t)bi * B;
    if constexpr (FULL && C::QPL > 0) {
        const MdqDesc dt = tile_view<SRC, DST, GT>(d, tbase);
        if constexpr (STAGED) {
            offp = (uint32_t)reinterpret_cast<uintptr_t>(dt.p) & 127u;
            offg = (uint32_t)reinterpret_cast<uintptr_t>(dt.g) & 127u;
            lines_to_lds<4 * C::TILE>(dt.p, stp, offp, lane);
            lines_to_lds<(int)GB * C::TILE>(dt.g, stg, offg, lane);
        }
#pragma unroll
        for (int k = 0; k < C::QPL; ++k) {
            const uint32_t i = lbase + 4 * lane_quad<PAIRED, LOG2B>(j, k);
            if constexpr (!STAGED) {
                vf4 p4;
                if constexpr (VEC_PG) {
                    p4 = ld_nt<vf4>(dt.p + i);
                    GradIO<GT>::load4(dt.g, i, gv + 4 * k);
                } else {
                    p4 = ld_nt_al<vf4, 4>(dt.p + i);
                    GradIO<GT>::load4u(dt.g, i, gv + 4 * k);
                }
                pv[4 * k + 0] = p4.x; pv[4 * k + 1] = p4.y; pv[4 * k + 2] = p4.z; pv[4 * k + 3] = p4.w;
            }
            if constexpr (!(PAIRED && one_byte_codes(SRC))) CodeIO<SRC>::load4(dt, i, mc + 4 * k, vc + 4 * k);
        }
        if constexpr (PAIRED && one_byte_codes(SRC)) craw = CodeIO<SRC>::raw8(dt, lbase, j);
#pragma unroll
        for (int e = 0; e < EPL; ++e) ok[e] = true;
    } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int64_t i = base + elem_off<PAIRED, LOG2B>(j, e);
            ok[e] = FULL || i < n;
            pv[e] = 0.0f; gv[e] = 0.0f; mc[e] = 0.0f; vc[e] = 0;
            if (ok[e]) {
                pv[e] = ld_g<float>(d.p + i);
                gv[e] = GradIO<GT>::load1(d.g, i);
                CodeIO<SRC>::load1(d, i, mc[e], vc[e]);
            }
        }
    }
    // The Philox words of stochastic rounding depend only on the element
    // indices, the step and the seed: drawn here, while the loads above are in
    // flight, their integer work overlaps the memory latency.  Counter
    // (quad index lo, hi, tensor id, step), key = seed; word i serves element
    // 4q+i.  Element indices count from rng_origin (a multiple of B, so of 4
    // wherever a lane owns whole quads).
    uint32_t rw[SR && C::QPL > 0 ? EPL : 1];
    if constexpr (SR && C::QPL > 0) {
        // The tile's first quad index (workgroup-uniform); a lane's quads lie less than
        // TILE / 4 above it, so where its low word leaves that much room below 2^32 the high
        // word is the same for the whole tile and stays in scalar registers (round 0's
        // first output word and round 1's first product are then scalar work).
        const uint64_t qt = (uint64_t)((tbase + d.rng_origin) >> 2);
        if ((uint32_t)qt <= 0xFFFFFFFFu - (uint32_t)(C::TILE / 4)) {
            const uint32_t qlo = (uint32_t)qt, qhi = (uint32_t)(qt >> 32);
#pragma unroll
            for (int k = 0; k < C::QPL; ++k) {
                const uint32_t off = (lbase >> 2) + (uint32_t)lane_quad<PAIRED, LOG2B>(j, k);
                const U4 r = mdq_philox4x32_uk<MDQ_SR_ROUNDS>(U4{qlo + off, qhi, d.tensor_id, step_no},
                                                  (uint32_t)sa.seed, (uint32_t)(sa.seed >> 32));
                rw[4 * k + 0] = r.x;
                rw[4 * k + 1] = r.y;
                rw[4 * k + 2] = r.z;
                rw[4 * k + 3] = r.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < C::QPL; ++k) {
                const uint64_t q = (uint64_t)(((base + d.rng_origin) >> 2) + lane_quad<PAIRED, LOG2B>(j, k));
                const U4 r = mdq_philox4x32_uk<MDQ_SR_ROUNDS>(U4{(uint32_t)q, (uint32_t)(q >> 32), d.tensor_id, step_no},
                                                  (uint32_t)sa.seed, (uint32_t)(sa.seed >> 32));
                rw[4 * k + 0] = r.x;
                rw[4 * k + 1] = r.y;
                rw[4 * k + 2] = r.z;
                rw[4 * k + 3] = r.w;
            }
        }
    }
    sm = block_bcast<LPB>(sm);
    sv = block_bcast<LPB>(sv);
    vmin = block_bcast<LPB>(vmin);
    if constexpr (FULL && C::QPL > 0 && PAIRED && one_byte_codes(SRC))
        CodeIO<SRC>::template decode8<LPB / 2>(craw, j, mc, vc);
    if constexpr (narrows_codes<SRC, DST>()) {
        constexpr float lo = DST == ST_S16 ? -32768.0f : -128.0f;
        constexpr float hi = DST == ST_S16 ? 32767.0f : 127.0f;
        constexpr uint32_t vhi = DST == ST_S16 ? 65535u : 255u;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            mc[e] = __builtin_amdgcn_fmed3f(mc[e], lo, hi);    // int32 -> float is monotonic
            vc[e] = vc[e] < vhi ? vc[e] : vhi;
        }
    }

    // exp table of the 16 packed v codes of this block (stquant_kernel.cu:75).  The
    // arguments fma(e, sv, vmin), e = 0 .. 15, are non-decreasing in e when sv >= 0, so they
    // lie in [vmin, fma(15, sv, vmin)]; when that interval is inside [-104, 89] for every
    // block of the wave, mdq_expf_core gives mdq_expf's bits without its clamps and selects
    // (as the per-element exp below).
    if constexpr (USE_LUT) {
        float *tab = lut + bi * 16;
        const bool in = !blk_ok || (sv >= 0.0f && vmin >= -104.0f && fma_(15.0f, sv, vmin) <= 89.0f);
        if (__builtin_amdgcn_ballot_w64(!in) == 0) {
            if (blk_ok) {
#pragma unroll
                for (int r = 0; r < (16 + LPB - 1) / LPB; ++r) {
                    const int e = j + r * LPB;
                    if (e < 16) tab[e] = mdq_expf_core(fma_((float)e, sv, vmin));
                }
            }
        } else if (blk_ok) {
#pragma unroll
            for (int r = 0; r < (16 + LPB - 1) / LPB; ++r) {
                const int e = j + r * LPB;
                if (e < 16) tab[e] = mdq_expf(fma_((float)e, sv, vmin));
            }
        }
        if constexpr (C::WAVES == 1) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        } else {
            __syncthreads();
        }
    }
    if constexpr (STAGED) {
        // the direct LDS loads count in vmcnt and the compiler does not wait for them
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int k = 0; k < C::QPL; ++k) {
            const uint32_t i = lbase + 4 * lane_quad<PAIRED, LOG2B>(j, k);
            // aligned quads: lines_to_lds shifted the lines by off & 12 (p is 4-byte aligned)
            const vf4 q = *(const vf4 *)(stp + (offp & ~15u) + 4 * i);
            pv[4 * k + 0] = q.x; pv[4 * k + 1] = q.y; pv[4 * k + 2] = q.z; pv[4 * k + 3] = q.w;
            if (GB == 4 || (offg & 3u) == 0)
                GradIO<GT>::lds4a(stg + (offg & ~15u) + GB * i, gv + 4 * k);
            else   // 2-byte grads at an odd element offset: element-wise reads
                GradIO<GT>::lds4(stg + (offg & ~12u) + GB * i, gv + 4 * k);
        }
    }
    if (prof_on) { unsigned long long t = clock64(); pa.c[0] += t - t0; t0 = t; }

    // dequant + AdamW moments (stquant_kernel.cu:71-85); contraction fixed as
    // one fma for the v exponent and one for each moment.
    const float neg8sm = -8.0f * sm;
    float m[EPL], v[EPL], lv[EPL];
    // Without the table every element takes an exp.  Its argument
    // fma(c, sv, vmin) is non-decreasing in the code c when sv >= 0, so with
    // c <= cmax (the storage's largest code) it lies in [vmin, fma(cmax, sv,
    // vmin)]; when that interval is inside [-104, 89] for every lane of the
    // wave, mdq_expf_core gives mdq_expf's bits without its clamps and selects.
    bool core_exp = false;
    if constexpr (!USE_LUT) {
        constexpr float cmax = SRC == ST_P4 ? 15.0f : SRC == ST_S8 ? 255.0f : SRC == ST_S16 ? 65535.0f
                                                                                           : 4294967296.0f;
        const bool in = sv >= 0.0f && vmin >= -104.0f && fma_(cmax, sv, vmin) <= 89.0f;
        core_exp = __builtin_amdgcn_ballot_w64(!in) == 0;
    }
    if (core_exp) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float m0 = dequant_m<SRC>(mc[e], sm, neg8sm);
            const float v0 = mdq_expf_core(fma_((float)vc[e], sv, vmin));
            const float g = gv[e];
            m[e] = fma_(d.b1, m0, d.omb1 * g);
            v[e] = fma_(d.b2, v0, (d.omb2 * g) * g);
        }
    } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float m0 = dequant_m<SRC>(mc[e], sm, neg8sm);
            float v0;
            if constexpr (VC_BYTES) v0 = *(const float *)((const char *)(lut + bi * 16) + vc[e]);
            else if constexpr (USE_LUT) v0 = lut[bi * 16 + vc[e]];
            else v0 = mdq_expf(fma_((float)vc[e], sv, vmin));
            const float g = gv[e];
            m[e] = fma_(d.b1, m0, d.omb1 * g);
            v[e] = fma_(d.b2, v0, (d.omb2 * g) * g);
        }
    }
    if (prof_on) { unsigned long long t = clock64(); pa.c[1] += t - t0; t0 = t; }

    // Fast v-code path: code width <= 8 bits, a one-wave tile with every
    // element inside the tensor and every x = v + 1e-12 a finite float >= 1e-12
    // (wave-uniform).  log is non-decreasing on that
    // range (checked for every float), so the block's max / min of log x are
    // the logs of its max / min x: two exact logs per lane instead of one per
    // element.  The per-element v codes then come from the hardware log (see
    // the requant below).
    constexpr bool FAST_OK = FULL && C::WAVES == 1;
    bool fastv = false;
    // The lane's largest and smallest x as int32 bit patterns.  A float x satisfies
    // 1e-12 <= x <= FLT_MAX exactly when its pattern lies in [bits(1e-12), bits(FLT_MAX)]:
    // +inf and +NaN patterns lie above, negative values, -0 and -NaN (negative as int32)
    // and values below 1e-12 below.  So the two integer extremes decide the test for all
    // EPL elements (three-input integer max / min), and on the fast path, where every x is
    // a positive finite float and floats order as their patterns, they are the lane's
    // max / min x for the block reductions.
    int32_t xhi = 0, xlo = 0;
    if constexpr (FAST_OK) {
        if (d.bits <= 8u) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int32_t b = __builtin_bit_cast(int32_t, v[e] + 1e-12f);
                xhi = e == 0 ? b : (b > xhi ? b : xhi);
                xlo = e == 0 ? b : (b < xlo ? b : xlo);
            }
            const bool good = xlo >= (int32_t)0x2b8cbcccu && xhi <= (int32_t)0x7f7fffffu;  // 1e-12f, FLT_MAX
            fastv = __builtin_amdgcn_ballot_w64(!good) == 0;
        }
    }

    // |m|, log(v + 1e-12) and the three block reductions (:92-97); lanes
    // outside the tensor contribute 0 to all three.
    float amax = 0.0f, lmax = 0.0f, lmin = 0.0f;
    int32_t ka, kx, kn;
    if (fastv) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float a = fabsf(m[e]);
            amax = e == 0 ? a : fmaxf(amax, a);
        }
        // positive finite floats order as their int32 bit patterns
        ka = __builtin_bit_cast(int32_t, amax);
        kx = xhi;
        kn = xlo;
    } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float a = ok[e] ? fabsf(m[e]) : 0.0f;
            const float l = ok[e] ? mdq_logf(v[e] + 1e-12f) : 0.0f;
            lv[e] = l;
            if (e == 0) { amax = a; lmax = l; lmin = l; }
            else { amax = fmaxf(amax, a); lmax = fmaxf(lmax, l); lmin = fminf(lmin, l); }
        }
        // The reference reduces with fmaxf / fminf (:26-50), which skip NaN:
        // fmaxf / fminf above do so within the lane, and a lane left with NaN
        // (all its elements NaN) offers a key every other lane beats.
        ka = amax == amax ? __builtin_bit_cast(int32_t, amax) : -1;
        kx = lmax == lmax ? f2key(lmax) : INT32_MIN;
        kn = lmin == lmin ? f2key(lmin) : INT32_MAX;
    }
    if constexpr (LPB <= 64) {
        ka = group_reduce<LPB, true>(ka);
        kx = group_reduce<LPB, true>(kx);
        kn = group_reduce<LPB, false>(kn);
    } else {
        ka = group_reduce<64, true>(ka);
        kx = group_reduce<64, true>(kx);
        kn = group_reduce<64, false>(kn);
        if (lane == 0) { xw[wave * 3 + 0] = ka; xw[wave * 3 + 1] = kx; xw[wave * 3 + 2] = kn; }
        __syncthreads();
        const int o = (wave ^ 1) * 3;
        ka = iop<true>(ka, xw[o + 0]);
        kx = iop<true>(kx, xw[o + 1]);
        kn = iop<false>(kn, xw[o + 2]);
    }
    amax = __builtin_bit_cast(float, ka);
    if (fastv) {
        if constexpr (LPB >= 2) {
            // one exact log per lane: even lanes log(xmax), odd lanes log(xmin),
            // then each lane takes both from its lane pair (quad_perm DPP)
            const int32_t ks = (lane & 1) ? kn : kx;
            const int32_t ls = __builtin_bit_cast(int32_t, mdq_logf(__builtin_bit_cast(float, ks)));
            lmax = __builtin_bit_cast(float, dpp_i<0xA0>(ls));   // quad_perm [0,0,2,2]
            lmin = __builtin_bit_cast(float, dpp_i<0xF5>(ls));   // quad_perm [1,1,3,3]
        } else {
            lmax = mdq_logf(__builtin_bit_cast(float, kx));
            lmin = mdq_logf(__builtin_bit_cast(float, kn));
        }
    } else {
        // keys no lane beat: every element of the block is NaN (NaN scales, as
        // fmaxf of NaN only)
        if (ka < 0) amax = __builtin_nanf("");
        lmax = kx == INT32_MIN ? __builtin_nanf("") : key2f(kx);
        lmin = kn == INT32_MAX ? __builtin_nanf("") : key2f(kn);
    }

    // new scales (:101-106)
    const float s_sm = (amax + 1e-12f) * d.inv_qm;            // == / 2^(bits-1), exact
    const float s_sv = mdq_div_code_range((lmax - lmin) + 1e-12f, d.qvf, d.inv_qvf);  // == IEEE division
    const float s_vmin = lmin;
    if (j == 0 && blk_ok) {
        st_g<float>(s_sm, d.scale_m + blk);
        st_g<float>(s_sv, d.scale_v + blk);
        st_g<float>(s_vmin, d.v_min + blk);
    }
    if (prof_on) { unsigned long long t = clock64(); pa.c[2] += t - t0; t0 = t; }

    // requant (:112-131)
    const float dm = s_sm + 1e-12f, dv = s_sv + 1e-12f;
    int32_t qmi[EPL];
    uint32_t qvi[EPL];
    float pk[EPL];                                            // packed byte values (P4)
    const bool wide = (DST == ST_S32) && d.bits > 16;         // uniform per tensor
    if (!wide) {
        float qmf[EPL], qvf[EPL];
        if constexpr (SR) {
            // 1.0f / d: through mdq_rcp_rn where every lane's d lies below 2^126 (the
            // range where it equals IEEE division), by division otherwise
            float inv_dm, inv_dv;
            if (__builtin_amdgcn_ballot_w64(!(dm < 0x1p126f && dv < 0x1p126f)) == 0) {
                inv_dm = mdq_rcp_rn(dm);
                inv_dv = mdq_rcp_rn(dv);
            } else {
                inv_dm = 1.0f / dm;
                inv_dv = 1.0f / dv;
            }
            // um: the m code's uniform; uvh: the v code's uniform minus 1/2 (exact: the
            // centred 2^-16 grid minus 1/2 is a multiple of 2^-17 below 1/2), so that the fast
            // path rounds to nearest where floor(z + uv) = rint(z + uvh) away from integers
            float um[EPL], uvh[EPL];
            // Philox4x32 (MDQ_SR_ROUNDS rounds) per 4-element quad of the tensor:
            // counter (quad index lo, hi, tensor id, step), key = seed; word i of
            // the output serves element 4q+i (low half -> m, high half -> v).
            // Element indices count from rng_origin (a multiple of B, so of 4
            // wherever a lane owns whole quads).
            if constexpr (C::QPL > 0) {
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    um[e] = mdq_u16_uniform(rw[e] & 0xffffu);
                    uvh[e] = mdq_u16_uniform_minus_half(rw[e] >> 16);
                }
            } else {
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const uint64_t idx = (uint64_t)(base + d.rng_origin + e);
                    const uint64_t q = idx >> 2;
                    U4 r = mdq_philox4x32_uk<MDQ_SR_ROUNDS>(U4{(uint32_t)q, (uint32_t)(q >> 32), d.tensor_id, step_no},
                                                (uint32_t)sa.seed, (uint32_t)(sa.seed >> 32));
                    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
                    const uint32_t ww = w[idx & 3];
                    um[e] = mdq_u16_uniform(ww & 0xffffu);
                    uvh[e] = mdq_u16_uniform_minus_half(ww >> 16);
                }
            }
            if (fastv) {
                // Zh approximates T - 1/2 within ep (mdq_sr_vfast): where Zh lies farther than
                // ep from a half-integer, rint(Zh) is the exact code (one rint and one test per
                // element); the elements of a wave with any closer Zh take the exact path.  In a
                // flat block every x is equal, so log x - vmin = 0 and the code is floor(uv) = 0;
                // there (its tiny dv flags every element) c1 = c0 = 0 make Zh = uvh exactly,
                // |uvh| < 1/2, so rint(Zh) = 0 without the exact path.
                const bool flat = kx == kn;
                SrVFast f = mdq_sr_vfast(dv, s_vmin, lmax, d.ep0_sr);
                f.c1 = flat ? 0.0f : f.c1;
                f.c0 = flat ? 0.0f : f.c0;
                const float near = 0.5f - f.ep;
                bool redo[EPL];
                bool any = false;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    qmf[e] = floor_(fma_(m[e], inv_dm, um[e]));
                    const float Zh = mdq_sr_vfast_z(v[e] + 1e-12f, uvh[e], f);
                    const float k = rint_(Zh);
                    qvf[e] = k;
                    redo[e] = fabsf(Zh - k) >= near;
                    any = any || redo[e];
                }
                if (__builtin_amdgcn_ballot_w64(any && !flat)) {
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        if (redo[e] && !flat)
                            qvf[e] = floor_(fma_(mdq_logf(v[e] + 1e-12f) - s_vmin, inv_dv, uvh[e] + 0.5f));
                    }
                }
            } else {
                // non-finite quotients give code 0, as in the nearest path below
                const bool sm_fin = dm <= __FLT_MAX__, sv_fin = dv <= __FLT_MAX__;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const float u = lv[e] - s_vmin;
                    qmf[e] = sm_fin && fabsf(m[e]) <= __FLT_MAX__ ? floor_(fma_(m[e], inv_dm, um[e])) : 0.0f;
                    qvf[e] = sv_fin && u <= __FLT_MAX__ ? floor_(fma_(u, inv_dv, uvh[e] + 0.5f)) : 0.0f;
                }
            }
        } else {
            // A block whose m scale is 2^126 or more (1- or 2-bit codes of |m| near FLT_MAX)
            // has a subnormal reciprocal, which the roundings below cannot use.  There m and
            // dm are both scaled by 2^-64 (msc), exact wherever the code depends on it (a
            // quotient at or above 1/2 needs |m| >= dm / 2 >= 2^125), and every element of
            // the block takes the exact rounding.
            const bool bigm = dm >= 0x1p126f;
            const float msc = bigm ? 0x1p-64f : 1.0f;
            const float dmq = dm * msc;
            const float hdm = 0.5f * dmq, hdv = 0.5f * dv;
            const float ilm = mdq_inv_lo(__builtin_amdgcn_rcpf(dmq));
            const float ilv = mdq_inv_lo(__builtin_amdgcn_rcpf(dv));
            if (fastv) {
                // The exact code is K = round-half-away(u / dv), u = fl(log x - vmin).
                // z = fl(log2_hw(x) * c1 + c0), with c1 = ln 2 / dv and c0 = -vmin / dv each
                // within 2^-24 (1 + 2^-16) relative (mdq_vcode_map), differs from u / dv by at
                // most E = G / dv + 2 (QV + 1) 2^-24, G = A + (S + 1.3e-7) L: A + S |log x|
                // bounds |log2_hw(x) ln 2 - log x| for every float x >= 1e-12
                // (MDQ_LOG_APPROX_ERR, MDQ_LOG_APPROX_SLOPE, measured exhaustively on the
                // device), L = max(|lmax|, |lmin|) >= |log x| within the block, 1.3e-7 L / dv
                // bounds the errors of c1 and c0 times |log2_hw(x) ln 2| and |vmin|, and the
                // last term the roundings of u and of z (z < QV + 1).  Where z is farther than
                // E from a half-integer, rint(z) (exact) is K; the elements within E of a
                // half-integer take the exact path.  The factor 1.001 covers r vs 1 / dv.
                // The m code likewise: zm = fl(m * rcp(dm)) differs from q = m / dm by at most
                // |q| (2^-21 + 2^-24) < (QM + 1) 6e-7 (rcp within 4 ulp, |q| <= QM), so where
                // zm is farther than that from a half-integer, rint(zm) is round-half-away(q)
                // (no tie), and the rest take mdq_round_half_away.  LLaMA 8-bit step 1.1 %
                // faster than the exact rounding for every element; 4-bit level.
                const VCodeMap vmap = mdq_vcode_map(dv, s_vmin);
                const float r = vmap.r, c1 = vmap.c1, c0 = vmap.c0;
                const float L = mdq_log_span(lmax, s_vmin);
                // the last term: the descriptor's ep0_rn = (QV + 1) 1.2e-7 * 1.001 (mdq_rn_ep0)
                const float ep = fma_(fma_(L, MDQ_LOG_APPROX_SLOPE + MDQ_VCODE_MAP_ERR, MDQ_LOG_APPROX_ERR),
                                      r * 1.001f, d.ep0_rn);
                const float near = 0.5f - ep;
                const float rdm = __builtin_amdgcn_rcpf(dm);
                const float nearm = bigm ? -1.0f : 0.5f - fma_(d.qm, 6.0e-7f, 6.0e-7f);
                bool redo[EPL], redo_m[EPL];
                bool any = false;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const float zm = m[e] * rdm;
                    const float km = rint_(zm);
                    qmf[e] = km;
                    redo_m[e] = fabsf(zm - km) >= nearm;
                    const float z = fma_(__builtin_amdgcn_logf(v[e] + 1e-12f), c1, c0);
                    const float kv = rint_(z);
                    qvf[e] = kv;
                    redo[e] = fabsf(z - kv) >= near;
                    any = any || redo[e] || redo_m[e];
                }
                if (__builtin_amdgcn_ballot_w64(any)) {
                    // every x of a flat block equals xmin, so log x - vmin = 0 and the
                    // code is 0 (its tiny dv flags every element above)
                    const bool flat = kx == kn;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        if (redo_m[e])
                            qmf[e] = __builtin_copysignf(mdq_round_half_away(fabsf(m[e]) * msc, dmq, ilm, hdm), m[e]);
                        if (flat) qvf[e] = 0.0f;
                        else if (redo[e]) qvf[e] = mdq_round_half_away(mdq_logf(v[e] + 1e-12f) - s_vmin, dv, ilv, hdv);
                    }
                }
            } else {
                // A quotient that is no finite number (a NaN or infinite m or log v, or a
                // NaN or infinite scale) reaches the reference's (int) conversion as NaN,
                // which gives 0 on its target (PTX cvt maps NaN to 0); finite / inf is 0
                // as well (:113-127).  The fast path runs only when every v, and so every
                // m and both scales, is finite.
                const bool sm_fin = dm <= __FLT_MAX__, sv_fin = dv <= __FLT_MAX__;
                float K[EPL];
                if (__builtin_amdgcn_ballot_w64(bigm)) {
#pragma unroll
                    for (int e = 0; e < EPL; ++e) K[e] = mdq_round_half_away(fabsf(m[e]) * msc, dmq, ilm, hdm);
                } else {
#pragma unroll
                    for (int e = 0; e < EPL; ++e) K[e] = mdq_round_half_away(fabsf(m[e]), dm, ilm, hdm);
                }
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const float u = lv[e] - s_vmin;
                    qmf[e] = sm_fin && fabsf(m[e]) <= __FLT_MAX__ ? __builtin_copysignf(K[e], m[e]) : 0.0f;
                    qvf[e] = sv_fin && u <= __FLT_MAX__ ? mdq_round_half_away(u, dv, ilv, hdv) : 0.0f;
                }
            }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float qm = __builtin_amdgcn_fmed3f(qmf[e], -d.qm, d.qm - 1.0f);
            const float qv = __builtin_amdgcn_fmed3f(qvf[e], 0.0f, d.qvf);
            if constexpr (DST == ST_P4) {
                pk[e] = fma_(qv, 16.0f, qm + 8.0f);           // (v << 4) | (m + 8), exact
            } else {
                qmi[e] = (int32_t)qm;
                qvi[e] = (uint32_t)(int32_t)qv;
            }
        }
    } else {
        // 17..32-bit codes: the reference's FP64 path verbatim.
        const double qlm = (double)d.qm;                        // 2^(bits-1), exact
        const double qlv = __builtin_ldexp(1.0, (int)d.bits) - 1.0;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            // a NaN quotient converts to 0 (the reference's (int) of NaN on its target)
            double qm_ = __builtin_round((double)m[e] / (double)dm);
            qm_ = qm_ == qm_ ? qm_ : 0.0;
            qm_ = qm_ < -qlm ? -qlm : qm_;
            qm_ = qm_ > qlm - 1.0 ? qlm - 1.0 : qm_;
            double qv_ = __builtin_round((double)(lv[e] - s_vmin) / (double)dv);
            qv_ = qv_ == qv_ ? qv_ : 0.0;
            qv_ = qv_ < 0.0 ? 0.0 : qv_;
            qv_ = qv_ > qlv ? qlv : qv_;
            qmi[e] = (int32_t)qm_;
            qvi[e] = (uint32_t)qv_;
        }
    }
    if (prof_on) { unsigned long long t = clock64(); pa.c[3] += t - t0; t0 = t; }

    // parameter update with the unquantised m, v (:135-144)
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const float den = fma_(__builtin_amdgcn_sqrtf(v[e]), inv_sqrt_bc2, d.eps);
        const float upd = m[e] * __builtin_amdgcn_rcpf(den);
        pv[e] = fma_(-step_size, upd, pv[e] * d.decay);
    }

    if constexpr (FULL && C::QPL > 0) {
        const MdqDesc dt = tile_view<SRC, DST, GT>(d, tbase);
        const MdqDesc ot = out_view<SRC, DST>(dt);
        // p's offset in its 128-byte line, in elements (the same for every tile of the
        // tensor); nonzero: the lanes' p go to LDS and store_p_lines writes them.  A
        // one-wave TILE_VECTOR tile starts on a line.  The LDS reads of p above were
        // this wave's, issued in order before the writes below.
        constexpr bool MAY_STAGE = VIEWS && (MODE != TILE_VECTOR || C::WAVES > 1);
        const uint32_t dl = MAY_STAGE ? (uint32_t)(reinterpret_cast<uintptr_t>(dt.p) >> 2) & 31u : 0u;
#pragma unroll
        for (int k = 0; k < C::QPL; ++k) {
            const uint32_t i = lbase + 4 * lane_quad<PAIRED, LOG2B>(j, k);
            if constexpr (!(PAIRED && one_byte_codes(DST))) {
                if constexpr (DST == ST_P4) CodeIO<DST>::store4f(ot, i, pk + 4 * k);
                else CodeIO<DST>::store4(ot, i, qmi + 4 * k, qvi + 4 * k);
            }
            const vf4 o = {pv[4 * k + 0], pv[4 * k + 1], pv[4 * k + 2], pv[4 * k + 3]};
            if (dl != 0u) *(vf4 *)(pst + i) = o;
            else if constexpr (VEC_PG) st_nt<vf4>(o, dt.p + i);
            else st_nt_al<vf4, 4>(o, dt.p + i);
        }
        if constexpr (PAIRED && one_byte_codes(DST)) {
            if constexpr (DST == ST_P4) CodeIO<DST>::template store8f<LPB / 2>(ot, lbase, j, pk);
            else CodeIO<DST>::template store8<LPB / 2>(ot, lbase, j, qmi, qvi);
        }
        if (dl != 0u) store_p_lines<C::THREADS, C::TILE>(dt.p, pst, dl);
    } else {
        const MdqDesc od = out_view<SRC, DST>(d);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            if (ok[e]) {
                const int64_t i = base + elem_off<PAIRED, LOG2B>(j, e);
                if constexpr (DST == ST_P4) CodeIO<DST>::store1f(od, i, pk[e]);
                else CodeIO<DST>::store1(od, i, qmi[e], qvi[e]);
                st_g<float>(pv[e], d.p + i);
            }
        }
    }
    if (prof_on) { unsigned long long t = clock64(); pa.c[4] += t - t0; }
}

// One workgroup per tile.  Workgroup b runs on XCD x = b % 8 (the hardware's
// round-robin) as that XCD's j-th workgroup, j = b / 8.  The tiles are dealt
// to the XCDs in chunks of K consecutive tiles (K tiles = 65536 elements,
// 256 KB of fp32 params): workgroup b takes tile ((j / K) * 8 + x) * K + j % K,
// so the 8 XCDs stream neighbouring chunks of every array at any moment.
// Workgroups of the last, partial round of 8 chunks take tile b (a bijection
// on [0, grid)).  Same-allocation A/B on the LLaMA set against one contiguous
// eighth per XCD: 4-bit 12.93 vs 13.26 ms, 8-bit level, GPT-2 small 0.282 vs
// 0.297 ms; chunks of 1, 8, 32, 96 or 512+ tiles were slower.
template <int LOG2B>
__device__ __forceinline__ long long xcd_tile()
{
    using C = Cfg<LOG2B>;
    const unsigned grid = gridDim.x, b = blockIdx.x;
    constexpr unsigned K = C::TILE >= 65536 ? 1u : 65536u / C::TILE;   // tiles per chunk
    const unsigned j = b >> 3, x = b & 7u;
    return b < grid / (8u * K) * (8u * K) ? (long long)((j / K) * 8u + x) * K + (j % K) : (long long)b;
}

// LDS of one tile: the exp table of packed 4-bit codes, the cross-wave reduction slots, and
// for staged tiles the lines of p and grads, then the p stores (tiles of several waves: the
// p stores).
template <int SRC, int DST, int GT, int LOG2B, bool SR, bool VIEWS>
struct StepLds {
    using C = Cfg<LOG2B>;
    static constexpr int LUT = (SRC == ST_P4) && C::B >= 32 ? C::TB * 16 : 1;
    static constexpr int PST = !VIEWS || C::QPL == 0 ? 1
                               : staged_mode<SRC, DST, SR, LOG2B>() ? staged_lds_bytes(C::TILE, GT == GT_F32 ? 4 : 2) / 4
                                                                    : C::TILE;
};

// Tile `tile` (tl within its tensor d) in the mode its tensor's flags allow.  Profiling
// (prof != null) samples every 64th tile; only the phase ratios of the cycle sums are
// meaningful.  VIEWS: the variant with the staged tile modes (and their LDS), which the host
// launches only when some tensor with whole tiles and aligned codes has p or grads off their
// 128-byte lines; the other variant has the vector and guarded modes alone, so aligned
// launches run code without the staged paths' register pressure (LLaMA-7B 4-bit stochastic:
// 13.71 ms with them in one kernel, 13.36 without, same box).
template <int SRC, int DST, int GT, int LOG2B, bool SR, bool VIEWS>
__device__ __forceinline__ void mdq_step_tile_any(const MdqDesc &d, long long tile, long long tl, float *lut_s,
                                                  int32_t *xw_s, float *pst_s, unsigned long long *prof,
                                                  const StepArgs &sa)
{
    using C = Cfg<LOG2B>;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const bool prof_on = prof != nullptr && (tile & 63) == 0;
    ProfAcc pa = {{0, 0, 0, 0, 0}};
    const bool inside = (tl + 1) * C::TILE <= d.numel;
    // DF_LINES: p and grads on 128-byte lines (tiles start every 2 KB of p, 1 KB of 2-byte grads)
    if constexpr (!VIEWS) {
        // the host launches this variant only when every tensor with whole tiles and aligned
        // codes has DF_LINES
        if (inside && (d.flags & DF_LINES))
            mdq_step_tile<SRC, DST, GT, LOG2B, SR, false, TILE_VECTOR>(d, tl, lane, wave, lut_s, xw_s, pst_s, sa, prof_on, pa);
        else
            mdq_step_tile<SRC, DST, GT, LOG2B, SR, false, TILE_GUARDED>(d, tl, lane, wave, lut_s, xw_s, pst_s, sa, prof_on, pa);
    } else {
        if (inside && (d.flags & DF_ALIGNED) && (C::WAVES > 1 || (d.flags & DF_LINES))) {
            mdq_step_tile<SRC, DST, GT, LOG2B, SR, true, TILE_VECTOR>(d, tl, lane, wave, lut_s, xw_s, pst_s, sa, prof_on, pa);
        } else if (C::QPL > 0 && inside && (d.flags & DF_CODES_ALIGNED)) {
            if constexpr (staged_mode<SRC, DST, SR, LOG2B>())
                mdq_step_tile<SRC, DST, GT, LOG2B, SR, true, TILE_STAGED>(d, tl, lane, wave, lut_s, xw_s, pst_s, sa, prof_on, pa);
            else if constexpr (C::QPL > 0)
                mdq_step_tile<SRC, DST, GT, LOG2B, SR, true, TILE_UNALIGNED_PG>(d, tl, lane, wave, lut_s, xw_s, pst_s, sa, prof_on, pa);
        } else {
            mdq_step_tile<SRC, DST, GT, LOG2B, SR, true, TILE_GUARDED>(d, tl, lane, wave, lut_s, xw_s, pst_s, sa, prof_on, pa);
        }
    }
    if (prof_on && threadIdx.x == 0) {
#pragma unroll
        for (int s = 0; s < 5; ++s) atomicAdd(prof + s, pa.c[s]);
    }
}

// Occupancy cap at 7 waves per SIMD in both kernels below: the clobber reserves v0..v71, so
// the register file never holds 8 of these waves, whatever the compiler's count.  With one
// contiguous eighth of the tiles per XCD, 8 waves ran the LLaMA 4-bit step 1 % slower
// (same-allocation A/B 13.36 vs 13.23 ms); with the chunked tile order the two are level
// (+-0.3 %).  Steps on int8 + uint8 codes, and with nearest rounding steps on packed 4-bit
// codes and storage-changing steps, are capped at 6 (v0..v79 reserved): their waves spend most
// of a tile waiting for its loads, and one wave fewer per SIMD contends less.  Same-allocation
// A/B, nearest rounding: 8-bit config 5 B = 64 / 128 / 256 -2.0 / -1.9 / -1.3 %, as packed views
// B = 128 -1.6 %, LLaMA-7B -0.7 %; 4-bit (three boxes) LLaMA-7B -0.3 to -0.6 %, GPT-2 small
// -0.3 %, config 5 B = 64 -1.0 %, as packed views B = 128 -2.2 to -2.7 %; storage changes on
// the LLaMA-7B set 8 -> 16 -3.0 %, 4 -> 8 -1.9 %, 16 -> 4 -2.5 %, 16 -> 8 -0.7 %.  Packed
// 4-bit codes with stochastic rounding keep 7 (6: LLaMA-7B +0.8 %, views B = 64 +1.2 %); most
// other stochastic kernels need 73-85 VGPRs and hold 5-6 anyway.
template <int SRC, int DST, bool SR>
__device__ __forceinline__ void occupancy_cap()
{
    if constexpr ((SRC == ST_S8 && DST == ST_S8) || (!SR && (SRC == ST_P4 || SRC != DST))) asm volatile("" ::: "v79");
    else asm volatile("" ::: "v71");
}

// The launch over a descriptor table: the tile's tensor is the largest t with
// tile_begin[t] <= tile (tile_begin: compact int64 copy of the descriptors' tile starts, so
// the ~log2(n_desc) dependent scalar loads hit a few cache lines).
template <int SRC, int DST, int GT, int LOG2B, bool SR, bool VIEWS>
__global__ __launch_bounds__(Cfg<LOG2B>::THREADS) void mdq_step_kernel(const MdqDesc *__restrict__ descs,
                                                                      const long long *__restrict__ tile_begin,
                                                                      int n_desc,
                                                                      unsigned long long *__restrict__ prof,
                                                                      const StepArgs sa)
{
    occupancy_cap<SRC, DST, SR>();
    using L = StepLds<SRC, DST, GT, LOG2B, SR, VIEWS>;
    __shared__ float lut_s[L::LUT];
    __shared__ int32_t xw_s[6];
    __shared__ __attribute__((aligned(16))) float pst_s[L::PST];
    const long long tile = xcd_tile<LOG2B>();
    int lo = 0, hi = n_desc - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_begin[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    const MdqDesc &d = descs[__builtin_amdgcn_readfirstlane(lo)];
    mdq_step_tile_any<SRC, DST, GT, LOG2B, SR, VIEWS>(d, tile, tile - d.tile_begin, lut_s, xw_s, pst_s, prof, sa);
}

// The launch over one tensor whose descriptor is a kernel argument (tile_begin 0): no table
// in device memory to upload or look up (the flat 4,194,304-element step 14.6 -> 11.9 us per
// call), and a call on a stream that is capturing a HIP graph records a plain kernel node.
// The variant with every tile mode (a one-tensor LLaMA-size step runs level with the
// table-driven kernel).
template <int SRC, int GT, int LOG2B, bool SR>
__global__ __launch_bounds__(Cfg<LOG2B>::THREADS) void mdq_step_kernel_one(const MdqDesc d,
                                                                          unsigned long long *__restrict__ prof,
                                                                          const StepArgs sa)
{
    occupancy_cap<SRC, SRC, SR>();
    using L = StepLds<SRC, SRC, GT, LOG2B, SR, true>;
    __shared__ float lut_s[L::LUT];
    __shared__ int32_t xw_s[6];
    __shared__ __attribute__((aligned(16))) float pst_s[L::PST];
    const long long tile = xcd_tile<LOG2B>();
    mdq_step_tile_any<SRC, SRC, GT, LOG2B, SR, true>(d, tile, tile, lut_s, xw_s, pst_s, prof, sa);
}

}  // namespace mdq
