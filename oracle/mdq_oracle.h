/*
 * mdq_oracle.h -- CPU oracle for the fused dequant -> AdamW -> requant step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py use it, and only as the checker / CPU baseline.
 *
 * It restates, element by element, the reference kernels in
 *   /root/reference/CUDA/stquant_kernel.cu:53-146  (packed 4-bit, uint8 per param)
 *   /root/reference/CUDA/stquant_kernel.cu:149-231 (int8 m / uint8 v)
 *   /root/reference/CUDA/stquant_kernel.cu:234-316 (int16 m / uint16 v)
 *   /root/reference/CUDA/stquant_kernel.cu:319-401 (int32 m / uint32 v)
 * and the dispatch rules of launch_fused_mdq_adamw (stquant_kernel.cu:414-465).
 *
 * Where the reference leaves rounding unspecified this oracle fixes it:
 *  - expf/logf are this file's own faithful (<1 ulp, checked exhaustively)
 *    implementations, mdq_oracle_expf / mdq_oracle_logf, because CUDA's libm
 *    results cannot be reproduced here;
 *  - the contractions nvcc may apply are fixed as written in mdq_oracle.c
 *    (one fmaf for each of: v dequant exponent, m moment, v moment).
 * Everything else (fp32 scale arithmetic, the FP64 divide + round-half-away,
 * clamps, tail-lane zeros in the block reductions) follows the reference
 * literally.
 *
 * Stochastic rounding has no reference counterpart; its definition here is
 * the one the HIP kernel implements (seven rounds of Philox4x32, Salmon et al.
 * SC'11).
 */
#ifndef MDQ_ORACLE_H
#define MDQ_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

enum { MDQO_STORE_P4 = 0, MDQO_STORE_S8 = 1, MDQO_STORE_S16 = 2, MDQO_STORE_S32 = 3 };
enum { MDQO_GRAD_F32 = 0, MDQO_GRAD_BF16 = 1, MDQO_GRAD_F16 = 2 };
enum { MDQO_ROUND_NEAREST = 0, MDQO_ROUND_STOCHASTIC = 1 };

typedef struct {
    float *p;              /* [numel] fp32 params, updated in place             */
    const void *grad;      /* [numel] grads, dtype = grad_dtype                 */
    void *code_m;          /* P4: uint8 packed [numel]; else int8/16/32 [numel] */
    void *code_v;          /* P4: unused; else uint8/16/32 [numel]              */
    float *scale_m;        /* [nblocks]                                         */
    float *scale_v;        /* [nblocks]                                         */
    float *v_min;          /* [nblocks]                                         */
    int64_t numel;
    int32_t storage;       /* MDQO_STORE_*                                      */
    int32_t grad_dtype;    /* MDQO_GRAD_*                                       */
    int32_t block_size;    /* power of two, 1..1024                             */
    int32_t bits;          /* 1..32, within the storage width; 4 for P4         */
    int32_t step;          /* already incremented by the caller (>= 1)          */
    uint32_t tensor_id;    /* stochastic rounding stream id                     */
    int64_t elem_offset;   /* index of element 0 in that stream (0: a whole     */
                           /* tensor; a piece's start within its tensor)        */
} mdqo_tensor;

typedef struct {
    float beta1, beta2, lr, weight_decay, eps;
    int32_t rounding;      /* MDQO_ROUND_*                                      */
    uint64_t seed;         /* stochastic rounding key                           */
    int32_t threads;       /* OpenMP threads, <= 0 for the runtime default      */
} mdqo_hparams;

/* One fused step for one tensor.  Returns 0, or -1 on an invalid argument. */
int mdq_oracle_step(const mdqo_tensor *t, const mdqo_hparams *h);

float mdq_oracle_expf(float x);
float mdq_oracle_logf(float x);
void mdq_oracle_expf_n(const float *x, float *y, int64_t n);
void mdq_oracle_logf_n(const float *x, float *y, int64_t n);
/* Max error in float ulps of mdq_oracle_expf (which 0) / mdq_oracle_logf (1)
 * over the bit patterns first .. first+count-1, against double libm. */
double mdq_oracle_max_ulp_err(int which, uint32_t first, uint32_t count);
/* round((double)num / (double)den), half away from zero, as a double. */
double mdq_oracle_round_div(float num, float den);
void mdq_oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* Philox4x32 with any number of rounds (the stochastic-rounding stream uses MDQO_SR_ROUNDS). */
#define MDQO_SR_ROUNDS 7
void mdq_oracle_philox4x32(const uint32_t ctr[4], const uint32_t key[2], int rounds, uint32_t out[4]);
/* Order-independent 64-bit digests over the whole positive-normal range,
 * one per 2^shift-value chunk, for cross-checking another implementation
 * of the same expf / logf without materialising 2^31 outputs. */
void mdq_oracle_math_chunk_digests(int which, uint32_t first, uint32_t count,
                                   uint32_t chunk, uint64_t *digests);

#ifdef __cplusplus
}
#endif
#endif
