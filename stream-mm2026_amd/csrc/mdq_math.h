// mdq_math.h -- fp32 math of the fused MDQ AdamW step, compiled for both the
// gfx950 device pass and the host pass of hipcc.
//
// The device kernels use these functions; the host copies are exported by the
// C-ABI library (stq_host_*) so that the same source can be checked on a CPU.
//
// * mdq_expf / mdq_logf: faithful (< 1 ulp) replacements for the CUDA expf /
//   logf calls of /root/reference/CUDA/stquant_kernel.cu:75,93.  Cody-Waite
//   exp with a degree-5 minimax polynomial, and log over f in [2/3, 4/3) with
//   a degree-8 minimax polynomial; coefficients are fp32 bit patterns.  Only
//   IEEE fma/mul/add, rint, ldexp and integer bit operations are used, in a
//   fixed order, and the library is built with -ffp-contract=off, so every
//   caller gets the same bits on any IEEE-conforming target.
// * mdq_round_half_away: round(u / d) for u >= 0 with ties away from zero,
//   exactly as round((double)u / (double)d) (stquant_kernel.cu:113,123)
//   evaluates for quotients below 2^19, using one fp32 fma residual.
// * mdq_philox4x32<R>: R rounds of Philox4x32 (Salmon et al., SC'11); R = 10 is
//   the published default, and stochastic rounding uses R = 7 (MDQ_SR_ROUNDS),
//   the round count the paper reports as passing TestU01's BigCrush.
// * mdq_rcp_rn: 1 / d correctly rounded, from the hardware reciprocal and one
//   fma Newton step.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define MDQ_HD __host__ __device__ __forceinline__
#else
#define MDQ_HD static inline
#endif

namespace mdq {

MDQ_HD float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }
MDQ_HD uint32_t f_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

#if defined(__HIP_DEVICE_COMPILE__)
MDQ_HD float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
MDQ_HD float rint_(float a) { return __builtin_rintf(a); }
MDQ_HD float floor_(float a) { return __builtin_floorf(a); }
MDQ_HD float ldexp_(float a, int e) { return __builtin_amdgcn_ldexpf(a, e); }
#else
MDQ_HD float fma_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
MDQ_HD float rint_(float a) { return __builtin_rintf(a); }
MDQ_HD float floor_(float a) { return __builtin_floorf(a); }
MDQ_HD float ldexp_(float a, int e) { return __builtin_ldexpf(a, e); }
#endif

// The body of mdq_expf for xc in [-104, 89]: there the clamps and special-value
// selects of mdq_expf leave xc and the result unchanged, so a caller that has
// shown its arguments lie in that range may call this directly and gets the
// same bits.
MDQ_HD float mdq_expf_core(float xc)
{
    const float log2e = bits_f(0x3fb8aa3bu);
    const float ln2_hi = bits_f(0x3f317218u);
    const float ln2_lo = bits_f(0xb102e308u);
    float kf = rint_(xc * log2e);
    float r = fma_(-kf, ln2_hi, xc);
    r = fma_(-kf, ln2_lo, r);
    float q = bits_f(0x3950bf17u);
    q = fma_(q, r, bits_f(0x3ab6a1a3u));
    q = fma_(q, r, bits_f(0x3c088856u));
    q = fma_(q, r, bits_f(0x3d2aaa74u));
    q = fma_(q, r, bits_f(0x3e2aaaabu));
    q = fma_(q, r, bits_f(0x3f000000u));
    float r2 = r * r;
    float t = fma_(r2, q, r);
    float e = 1.0f + t;
    return ldexp_(e, (int)kf);
}

// e^x.  NaN -> NaN, x > 89 -> +inf, x < -104 -> 0; in between the result is
// 2^k * (1 + (r + r^2 E(r))) with a single rounding in the final scale.
MDQ_HD float mdq_expf(float x)
{
    // Clamp first so the integer conversion in the body is always in range;
    // the special results are selected at the end.
    float xc = x < -104.0f ? -104.0f : x;
    xc = xc > 89.0f ? 89.0f : xc;
    xc = (x == x) ? xc : 0.0f;
    float res = mdq_expf_core(xc);
    res = x > 89.0f ? bits_f(0x7f800000u) : res;
    res = x < -104.0f ? 0.0f : res;
    return (x == x) ? res : x;
}

// log(x) for x a positive normal float, +inf or NaN (returned unchanged).
// The kernel only ever evaluates log(v + 1e-12f) with v >= 0, a positive
// normal; zero, denormal and negative inputs are outside this function's
// domain.
MDQ_HD float mdq_logf(float x)
{
    uint32_t ix = f_bits(x);
    int32_t t = (int32_t)(ix - 0x3f2aaaabu);
    int32_t k = t >> 23;                            // in [-256, 255]
    float f = bits_f(ix - (uint32_t)(k * 8388608)); // == (t & 0x7fffff) + 0x3f2aaaab

    float r = f - 1.0f;
    float kf = (float)k;
    float p = bits_f(0xbe05ac99u);
    p = fma_(p, r, bits_f(0x3e0cde1du));
    p = fma_(p, r, bits_f(0xbdf8cd34u));
    p = fma_(p, r, bits_f(0x3e0fea42u));
    p = fma_(p, r, bits_f(0xbe2ad591u));
    p = fma_(p, r, bits_f(0x3e4cdfffu));
    p = fma_(p, r, bits_f(0xbe7fff4au));
    p = fma_(p, r, bits_f(0x3eaaaa96u));
    p = fma_(p, r, bits_f(0xbf000000u));
    float r2 = r * r;
    float lo = fma_(kf, bits_f(0x35bfbe8eu), r2 * p);
    float res = fma_(kf, bits_f(0x3f317200u), r + lo);
    return ix >= 0x7f800000u ? x : res;
}

#if defined(__HIPCC__)
// c1 = ln 2 / dv and c0 = -vmin / dv of the fast v-code path (a v code is
// about log2_hw(x) * c1 + c0), each within 2^-24 (1 + 2^-16) relative of the
// exact quotient.  r = v_rcp_f32(dv) is within a few ulp of 1/dv; q = a * r,
// and one residual step q + fma(-q, dv, a) * r leaves an error far below an
// ulp before the final rounding (for ln 2 the residual also adds
// ln 2 - RN(ln 2)).  dv must be a positive normal float.
struct VCodeMap {
    float r, c1, c0;
};
__device__ __forceinline__ VCodeMap mdq_vcode_map(float dv, float vmin)
{
    const float r = __builtin_amdgcn_rcpf(dv);
    const float ln2_hi = bits_f(0x3f317218u);                // RN(ln 2)
    const float ln2_lo = bits_f(0xb102e308u);                // RN(ln 2 - ln2_hi)
    const float q1 = ln2_hi * r;
    const float c1 = fma_(fma_(-q1, dv, ln2_hi) + ln2_lo, r, q1);
    const float a = -vmin;
    const float q0 = a * r;
    const float c0 = fma_(fma_(-q0, dv, a), r, q0);
    return {r, c1, c0};
}
#endif

// K = floor(u/d + 1/2) for u >= 0 and d a positive normal float, i.e.
// round-half-away(u/d), computed exactly in fp32 as long as u/d < 2^19.
// inv_lo must lie below 1/d by a relative 2^-23 .. 2^-20 (the kernel takes
// the hardware reciprocal, within 1 ulp, and steps it down 4 ulp).  Then the
// candidate k0 = floor(u*inv_lo + 1/2) is K or K-1, never above K, and
// R = u - k0*d (one fma) decides: K = k0 + (R >= d/2).  R is exact when
// u >= d/2 (u and k0*d share the 2^(E_d-24) grid and |R| < 2^(E_d)), or else
// |R| >= 2^(E_d) > d/2 and only its sign matters; when u < d/2, k0 = 0 and R = u.
// hd must be d/2 exactly.
MDQ_HD float mdq_round_half_away(float u, float d, float inv_lo, float hd)
{
    const float k0 = floor_(fma_(u, inv_lo, 0.5f));
    const float R = fma_(-k0, d, u);
    return R >= hd ? k0 + 1.0f : k0;
}

// x / D correctly rounded for D = (float)(2^bits - 1), bits 1..32, given
// y = RN(1/D): q = x*y is within an ulp, the fma residual x - q*D is exact,
// and one correction q + r*y rounds to RN(x/D).  Checked against IEEE
// division for every positive float x and every bits value.  For x = +inf
// the residual is NaN and q = +inf is the quotient; NaN stays NaN.
MDQ_HD float mdq_div_code_range(float x, float D, float y)
{
    const float q = x * y;
    const float r = fma_(-q, D, x);
    return r == r ? fma_(r, y, q) : q;
}

// The reciprocal of d stepped down by 4 ulp, for mdq_round_half_away.
MDQ_HD float mdq_inv_lo(float inv_d_within_1ulp) { return bits_f(f_bits(inv_d_within_1ulp) - 4u); }

struct U4 { uint32_t x, y, z, w; };

// Philox4x32 rounds of the stochastic-rounding stream.
#define MDQ_SR_ROUNDS 7

template <int R>
MDQ_HD U4 mdq_philox4x32(U4 c, uint32_t k0, uint32_t k1)
{
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
        U4 n;
        n.x = (uint32_t)(p1 >> 32) ^ c.y ^ k0;
        n.y = (uint32_t)p1;
        n.z = (uint32_t)(p0 >> 32) ^ c.w ^ k1;
        n.w = (uint32_t)p0;
        c = n;
    }
    return c;
}

MDQ_HD U4 mdq_philox4x32_10(U4 c, uint32_t k0, uint32_t k1) { return mdq_philox4x32<10>(c, k0, k1); }

#if defined(__HIPCC__)
// a ^ b ^ k as one v_bitop3_b32 (truth table 0x96, the three-input XOR), which
// the compiler does not form by itself.  k is passed in a scalar register, so
// it must be wave-uniform.
__device__ __forceinline__ uint32_t xor3_uk(uint32_t a, uint32_t b, uint32_t k)
{
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t r;
    asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
    return r;
#else
    return a ^ b ^ k;
#endif
}

// mdq_philox4x32<R> for a wave-uniform key (the step kernel's seed), same
// result.  Round 0 keeps the plain XORs (its tensor-id and step words are
// uniform too, so the compiler folds them in scalar registers); the other
// rounds fuse each output word's two XORs.
template <int R>
__device__ __forceinline__ U4 mdq_philox4x32_uk(U4 c, uint32_t k0, uint32_t k1)
{
    {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
        c = U4{(uint32_t)(p1 >> 32) ^ c.y ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c.w ^ k1, (uint32_t)p0};
    }
#pragma unroll
    for (int r = 1; r < R; ++r) {
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
        const uint64_t p0 = (uint64_t)0xD2511F53u * c.x;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.z;
        c = U4{xor3_uk((uint32_t)(p1 >> 32), c.y, k0), (uint32_t)p1, xor3_uk((uint32_t)(p0 >> 32), c.w, k1),
               (uint32_t)p0};
    }
    return c;
}
#endif

// The rounding terms of the fast v-code paths' error bounds for codes in [0, qvf]
// (qvf = 2^bits - 1), each with headroom and times the paths' factor 1.001 for
// v_rcp_f32(dv) against 1 / dv: the nearest path's 2 (QV + 1) 2^-24 and the stochastic
// path's 5 (QV + 2) 2^-24 (mdq_kernel.h, mdq_sr_vfast).  Per tensor, in its descriptor.
MDQ_HD float mdq_rn_ep0(float qvf) { return (qvf + 1.0f) * 1.2e-7f * 1.001f; }
MDQ_HD float mdq_sr_ep0(float qvf) { return (qvf + 2.0f) * 3.0e-7f * 1.001f; }

// Uniforms on the centred 2^-16 grid: (k + 1/2) / 65536, k in [0, 65535].
// (k16 + 0.5) / 2^16 as k16 * 2^-16 + 2^-17: both terms and the sum are exact
// (17 significant bits), so the one fma equals the add-then-multiply form.
MDQ_HD float mdq_u16_uniform(uint32_t k16) { return fma_((float)k16, 1.0f / 65536.0f, 1.0f / 131072.0f); }
// The same uniform minus 1/2: (2 k16 + 1 - 65536) 2^-17, a multiple of 2^-17 of magnitude below
// 1/2, so the fma (whose addend 2^-17 - 1/2 is exact too) is exact and
// mdq_u16_uniform_minus_half(k) + 0.5f == mdq_u16_uniform(k) exactly.
MDQ_HD float mdq_u16_uniform_minus_half(uint32_t k16)
{
    return fma_((float)k16, 1.0f / 65536.0f, 1.0f / 131072.0f - 0.5f);
}

// 1 / d correctly rounded for a positive normal d below 2^126 (where 1 / d is a
// normal float).  On the device: the hardware reciprocal r (within 1 ulp) and
// one Newton step r + r (1 - d r) with an fma residual; equal to IEEE 1.0f / d
// for every float of that range, and for no larger d (checked exhaustively
// against the oracle's division, stq_device_math_digests).  The host build
// divides.
MDQ_HD float mdq_rcp_rn(float d)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const float r = __builtin_amdgcn_rcpf(d);
    return fma_(r, fma_(-d, r, 1.0f), r);
#else
    return 1.0f / d;
#endif
}

}  // namespace mdq
