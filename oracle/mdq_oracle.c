/*
 * mdq_oracle.c -- CPU oracle for the fused dequant -> AdamW -> requant step.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker / CPU baseline, never by the
 * shipped library.  Build: oracle/Makefile (gcc, -ffp-contract=off, OpenMP).
 *
 * Every function cites the reference lines it restates.  Parity status of
 * each part (how it is pinned) is listed in the header comment of
 * oracle/mdq_oracle.py.
 */
#include "mdq_oracle.h"

#include <math.h>
#include <string.h>
#include <stddef.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* ------------------------------------------------------------------------
 * expf: Cody-Waite reduction x = k*ln2 + r, |r| <= ln2/2, then
 * e^r = 1 + (r + r^2 * E(r)) with E a degree-5 minimax fit of
 * (e^r - 1 - r)/r^2 on [-ln2/2, ln2/2] (coefficients rounded to fp32,
 * derived by oracle/derive_math_constants.py), then an exact scale by 2^k.
 * Max error 0.988 ulp over every fp32 input in [-87, 88]
 * (tests/test_oracle_math.py).  Stands in for CUDA expf at
 * stquant_kernel.cu:75,169,254,339.
 * ---------------------------------------------------------------------- */
static const uint32_t EXP_C[6] = {0x3f000000u, 0x3e2aaaabu, 0x3d2aaa74u,
                                  0x3c088856u, 0x3ab6a1a3u, 0x3950bf17u};

float mdq_oracle_expf(float x)
{
    if (x != x) return x;                       /* NaN passes through      */
    if (x > 89.0f) return u2f(0x7f800000u);     /* overflow                */
    if (x < -104.0f) return 0.0f;               /* below half the min denormal */
    const float log2e = u2f(0x3fb8aa3bu);
    const float ln2_hi = u2f(0x3f317218u);
    const float ln2_lo = u2f(0xb102e308u);
    float kf = rintf(x * log2e);
    float r = fmaf(-kf, ln2_hi, x);
    r = fmaf(-kf, ln2_lo, r);
    float q = u2f(EXP_C[5]);
    for (int i = 4; i >= 0; --i) q = fmaf(q, r, u2f(EXP_C[i]));
    float r2 = r * r;
    float t = fmaf(r2, q, r);
    float e = 1.0f + t;
    return ldexpf(e, (int)kf);
}

/* ------------------------------------------------------------------------
 * logf: x = 2^k * f with f in [c, 2c), c = 0x3f2aaaab (~2/3), r = f - 1
 * (exact), log(1+r) = r + r^2 * P(r) with P a degree-8 minimax fit of
 * (log1p(r) - r)/r^2 on [c-1, 2c-1) (fp32 coefficients from
 * oracle/derive_math_constants.py), then + k*ln2 split hi/lo.
 * Max error 0.974 ulp over every positive normal fp32
 * (tests/test_oracle_math.py).  Stands in for CUDA logf at
 * stquant_kernel.cu:93,185,270,355, whose argument v + 1e-12f is always
 * >= 1e-12f, a positive normal.
 * ---------------------------------------------------------------------- */
static const uint32_t LOG_C[9] = {0xbf000000u, 0x3eaaaa96u, 0xbe7fff4au,
                                  0x3e4cdfffu, 0xbe2ad591u, 0x3e0fea42u,
                                  0xbdf8cd34u, 0x3e0cde1du, 0xbe05ac99u};

float mdq_oracle_logf(float x)
{
    uint32_t ix = f2u(x);
    if (ix >= 0x7f800000u) {                    /* +inf, NaN, or sign bit set */
        if (x != x || x == u2f(0x7f800000u)) return x;
        if (x == 0.0f) return u2f(0xff800000u); /* -0 -> -inf */
        return u2f(0x7fc00000u);                /* negative -> NaN */
    }
    int32_t kadj = 0;
    if (ix < 0x00800000u) {                     /* +0 or denormal */
        if (ix == 0) return u2f(0xff800000u);
        x = x * 8388608.0f;                     /* 2^23, exact */
        ix = f2u(x);
        kadj = -23;
    }
    int32_t t = (int32_t)(ix - 0x3f2aaaabu);
    int32_t k = (t >> 23) + kadj;               /* arithmetic shift */
    float f = u2f(((uint32_t)t & 0x007fffffu) + 0x3f2aaaabu);
    float r = f - 1.0f;
    float kf = (float)k;
    float p = u2f(LOG_C[8]);
    for (int i = 7; i >= 0; --i) p = fmaf(p, r, u2f(LOG_C[i]));
    float r2 = r * r;
    const float ln2_hi = u2f(0x3f317200u);      /* 16 significant bits */
    const float ln2_lo = u2f(0x35bfbe8eu);
    float lo = fmaf(kf, ln2_lo, r2 * p);
    return fmaf(kf, ln2_hi, r + lo);
}

void mdq_oracle_expf_n(const float *x, float *y, int64_t n)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = mdq_oracle_expf(x[i]);
}

void mdq_oracle_logf_n(const float *x, float *y, int64_t n)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = mdq_oracle_logf(x[i]);
}

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void mdq_oracle_math_chunk_digests(int which, uint32_t first, uint32_t count,
                                   uint32_t chunk, uint64_t *digests)
{
    uint32_t nchunks = (count + chunk - 1) / chunk;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t c = 0; c < (int64_t)nchunks; ++c) {
        uint64_t acc = 0;
        uint32_t lo = first + (uint32_t)c * chunk;
        uint32_t hi = (c + 1 == nchunks) ? first + count : lo + chunk;
        for (uint32_t b = lo; b < hi; ++b) {
            float x = u2f(b);
            float y = which == 0 ? mdq_oracle_expf(x) : which == 1 ? mdq_oracle_logf(x) : 1.0f / x;
            acc += mix64(((uint64_t)b << 32) | f2u(y));
        }
        digests[c] = acc;
    }
}

/* The largest error, in units in the last place of the float nearest the true
 * value, of mdq_oracle_expf (which = 0) or mdq_oracle_logf (1) over the float
 * bit patterns first .. first+count-1, against libm's double exp / log (whose
 * own error, below 1 double ulp, is 2^-29 of a float ulp).  Inputs whose true
 * value is not a finite nonzero float are skipped. */
double mdq_oracle_max_ulp_err(int which, uint32_t first, uint32_t count)
{
    double worst = 0.0;
#pragma omp parallel for schedule(static, 1 << 16) reduction(max : worst)
    for (int64_t i = 0; i < (int64_t)count; ++i) {
        const float x = u2f(first + (uint32_t)i);
        const double ref = which == 0 ? exp((double)x) : log((double)x);
        const float ref32 = (float)fabs(ref);
        if (!(ref32 > 0.0f) || isinf(ref32)) continue;
        int e = 0;
        (void)frexp((double)ref32, &e);
        double ulp = ldexp(1.0, e - 24);
        if (ulp < ldexp(1.0, -149)) ulp = ldexp(1.0, -149);
        const float y = which == 0 ? mdq_oracle_expf(x) : mdq_oracle_logf(x);
        const double err = fabs((double)y - ref) / ulp;
        if (err > worst || err != err) worst = err != err ? INFINITY : err;
    }
    return worst;
}

/* round() of the FP64 quotient, as stquant_kernel.cu:113,123 compute it. */
double mdq_oracle_round_div(float num, float den)
{
    return round((double)num / (double)den);
}

/* ------------------------------------------------------------------------
 * Philox4x32 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy
 * as 1, 2, 3", SC'11): `rounds` rounds of the 4x32 S-P network with
 * multipliers 0xD2511F53 / 0xCD9E8D57 and Weyl key increments
 * 0x9E3779B9 / 0xBB67AE85.  Ten rounds are the published default, pinned by
 * the Random123 known-answer vectors; any round count is pinned against
 * rocRAND's own round function (tests/test_oracle_philox.py).  Stochastic
 * rounding draws from seven rounds (MDQO_SR_ROUNDS), the count the paper
 * reports as passing TestU01's BigCrush.
 * ---------------------------------------------------------------------- */
void mdq_oracle_philox4x32(const uint32_t ctr[4], const uint32_t key[2], int rounds, uint32_t out[4])
{
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < rounds; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

void mdq_oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    mdq_oracle_philox4x32(ctr, key, 10, out);
}

/* Two uniforms on the centred 2^-16 grid for element idx of a tensor: word
 * idx mod 4 of the Philox4x32 output for counter (idx / 4 low, high, tensor id,
 * step) and key seed; its low half drives m, its high half v. */
static inline void sr_uniforms(uint64_t idx, uint32_t tensor_id, int32_t step,
                               uint64_t seed, float *um, float *uv)
{
    uint32_t ctr[4] = {(uint32_t)(idx >> 2), (uint32_t)(idx >> 34), tensor_id, (uint32_t)step};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    mdq_oracle_philox4x32(ctr, key, MDQO_SR_ROUNDS, out);
    uint32_t w = out[idx & 3];
    *um = ((float)(w & 0xffffu) + 0.5f) * (1.0f / 65536.0f);
    *uv = ((float)(w >> 16) + 0.5f) * (1.0f / 65536.0f);
}

static inline float load_grad(const void *g, int dtype, int64_t i)
{
    if (dtype == MDQO_GRAD_F32) return ((const float *)g)[i];
    uint16_t h = ((const uint16_t *)g)[i];
    if (dtype == MDQO_GRAD_BF16) return u2f((uint32_t)h << 16);
    /* IEEE binary16 -> binary32, exact */
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f);   /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* ------------------------------------------------------------------------
 * One fused step for one tensor: stquant_kernel.cu:53-146 (packed4),
 * :149-231 (s8/u8), :234-316 (s16/u16), :319-401 (s32/u32).  One reference
 * CUDA block == one quant block of B lanes; lanes past numel are "invalid"
 * and feed 0 to all three reductions (:92-93).
 * ---------------------------------------------------------------------- */
int mdq_oracle_step(const mdqo_tensor *t, const mdqo_hparams *h)
{
    const int64_t n = t->numel;
    const int B = t->block_size;
    if (n < 0 || B < 1 || B > 1024 || (B & (B - 1)) != 0) return -1;
    if (t->bits < 1 || t->bits > 32 || t->step < 1) return -1;
    if (t->storage == MDQO_STORE_P4 && t->bits != 4) return -1;
    if (t->storage == MDQO_STORE_S8 && t->bits > 8) return -1;
    if (t->storage == MDQO_STORE_S16 && t->bits > 16) return -1;
    if (t->storage < 0 || t->storage > 3) return -1;
    if (t->elem_offset < 0) return -1;
    if (n == 0) return 0;
    const int64_t nb = (n + B - 1) / B;

    const float b1 = h->beta1, b2 = h->beta2, lr = h->lr, wd = h->weight_decay, eps = h->eps;
    const double qlm = pow(2.0, t->bits - 1);          /* :88-89 */
    const double qlv = pow(2.0, t->bits) - 1.0;
    const float omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    /* :136-137 bias corrections; :141 decay factor */
    const float bc1 = 1.0f - powf(b1, (float)t->step);
    const float bc2 = 1.0f - powf(b2, (float)t->step);
    const float sqrt_bc2 = sqrtf(bc2);
    const float step_size = lr / bc1;
    const float decay = 1.0f - lr * wd;
    const int stochastic = (h->rounding == MDQO_ROUND_STOCHASTIC) && t->bits <= 16;

    int nthreads = 1;
#ifdef _OPENMP
    nthreads = h->threads > 0 ? h->threads : omp_get_max_threads();
#endif
#pragma omp parallel num_threads(nthreads)
    {
        float mv[1024], vv[1024], lv[1024];
#pragma omp for schedule(static)
        for (int64_t b = 0; b < nb; ++b) {
            const int64_t base = b * B;
            const float sm = t->scale_m[b], sv = t->scale_v[b], vmin = t->v_min[b];  /* :67-69 */
            float max_m = 0.0f, max_lv = 0.0f, min_lv = 0.0f;
            int first = 1;
            for (int i = 0; i < B; ++i) {
                const int64_t idx = base + i;
                float a = 0.0f, l = 0.0f;               /* invalid lanes: :92-93 */
                if (idx < n) {
                    float m, v;
                    float g = load_grad(t->grad, t->grad_dtype, idx);
                    switch (t->storage) {               /* dequant :71-75 / :168-169 */
                    case MDQO_STORE_P4: {
                        uint8_t pk = ((const uint8_t *)t->code_m)[idx];
                        int mu = pk & 0x0f, vq = (pk >> 4) & 0x0f;
                        m = ((float)mu - 8.0f) * sm;
                        v = mdq_oracle_expf(fmaf((float)vq, sv, vmin));
                        break;
                    }
                    case MDQO_STORE_S8:
                        m = (float)((const int8_t *)t->code_m)[idx] * sm;
                        v = mdq_oracle_expf(fmaf((float)((const uint8_t *)t->code_v)[idx], sv, vmin));
                        break;
                    case MDQO_STORE_S16:
                        m = (float)((const int16_t *)t->code_m)[idx] * sm;
                        v = mdq_oracle_expf(fmaf((float)((const uint16_t *)t->code_v)[idx], sv, vmin));
                        break;
                    default:
                        m = (float)((const int32_t *)t->code_m)[idx] * sm;
                        v = mdq_oracle_expf(fmaf((float)((const uint32_t *)t->code_v)[idx], sv, vmin));
                        break;
                    }
                    /* moments :83-84 -- contraction fixed as one fmaf each */
                    m = fmaf(b1, m, omb1 * g);
                    v = fmaf(b2, v, (omb2 * g) * g);
                    a = fabsf(m);
                    l = mdq_oracle_logf(v + 1e-12f);
                    mv[i] = m; vv[i] = v; lv[i] = l;
                }
                /* block reductions :95-97 with fmaxf / fminf (:26-50): NaN is ignored
                 * unless every lane is NaN; otherwise order-free (max/min are exact) */
                if (first) { max_m = a; max_lv = l; min_lv = l; first = 0; }
                else {
                    max_m = fmaxf(max_m, a);
                    max_lv = fmaxf(max_lv, l);
                    min_lv = fminf(min_lv, l);
                }
            }
            /* new scales :101-106 */
            const float s_sm = (max_m + 1e-12f) / (float)qlm;
            const float s_sv = ((max_lv - min_lv) + 1e-12f) / (float)qlv;
            const float s_vmin = min_lv;
            t->scale_m[b] = s_sm;
            t->scale_v[b] = s_sv;
            t->v_min[b] = s_vmin;
            const float dm = s_sm + 1e-12f, dv = s_sv + 1e-12f;
            const float inv_dm = 1.0f / dm, inv_dv = 1.0f / dv;

            const int valid = (int)((n - base) < B ? (n - base) : B);
            for (int i = 0; i < valid; ++i) {
                const int64_t idx = base + i;
                const float m = mv[i], v = vv[i], l = lv[i];
                double qm, qv;
                if (stochastic) {
                    float um, uv;
                    sr_uniforms((uint64_t)(idx + t->elem_offset), t->tensor_id, t->step, h->seed, &um, &uv);
                    qm = (double)floorf(fmaf(m, inv_dm, um));
                    qv = (double)floorf(fmaf(l - s_vmin, inv_dv, uv));
                } else {
                    qm = round((double)m / (double)dm);            /* :113 */
                    qv = round((double)(l - s_vmin) / (double)dv); /* :123 */
                }
                /* A NaN quotient (NaN or infinite m or log v over an infinite or NaN
                 * scale) passes the clamps below and reaches the reference's (int)
                 * conversion (:118,126), which gives 0 on its target (PTX cvt maps NaN
                 * to 0); C leaves that conversion undefined, so it is spelled out. */
                if (qm != qm) qm = 0.0;
                if (qv != qv) qv = 0.0;
                if (qm < -qlm) qm = -qlm;                           /* :114-117 */
                if (qm > qlm - 1.0) qm = qlm - 1.0;
                if (qv < 0.0) qv = 0.0;                             /* :124-125 */
                if (qv > qlv) qv = qlv;
                switch (t->storage) {
                case MDQO_STORE_P4: {                               /* :118-130 */
                    int mu = (int)qm + 8;
                    if (mu < 0) mu = 0;
                    if (mu > 15) mu = 15;
                    int vi = (int)qv;
                    if (vi < 0) vi = 0;
                    if (vi > 15) vi = 15;
                    ((uint8_t *)t->code_m)[idx] = (uint8_t)((vi << 4) | (mu & 0x0f));
                    break;
                }
                case MDQO_STORE_S8:                                 /* :210,215 */
                    ((int8_t *)t->code_m)[idx] = (int8_t)qm;
                    ((uint8_t *)t->code_v)[idx] = (uint8_t)qv;
                    break;
                case MDQO_STORE_S16:                                /* :295,300 */
                    ((int16_t *)t->code_m)[idx] = (int16_t)qm;
                    ((uint16_t *)t->code_v)[idx] = (uint16_t)qv;
                    break;
                default:                                            /* :380,385 */
                    ((int32_t *)t->code_m)[idx] = (int32_t)qm;
                    ((uint32_t *)t->code_v)[idx] = (uint32_t)qv;
                    break;
                }
                /* parameter update with the unquantised m, v :135-144 */
                const float denom = sqrtf(v) / sqrt_bc2 + eps;
                float w = t->p[idx];
                if (wd != 0.0f) w = w * decay;
                w = w - step_size * (m / denom);
                t->p[idx] = w;
            }
        }
    }
    return 0;
}
