/*
 * stquant_hip.h -- C ABI of the MI355X-native fused MDQ AdamW step.
 *
 * The shared library stream-mm2026_amd/mdq_hip/libstquant_hip.so exports
 * these symbols.  Signatures carry plain pointers, sizes and dtype codes only;
 * every device pointer must address memory of the current HIP device and be
 * aligned to its element size (as every torch tensor is), and every call is
 * asynchronous on the given hipStream_t (NULL = the null stream).
 *
 * Return value: STQ_OK, or an STQ_ERR_* code with a message available from
 * stq_last_error() (thread-local).  Argument errors are reported before any
 * device work is queued.
 *
 * The multi-tensor entry points upload a descriptor table per call from
 * staging buffers that later calls reuse (or launch from a device copy of an
 * identical table, see stq_step_table_uploads), so they refuse
 * (STQ_ERR_INVALID, nothing queued) a stream that is capturing a HIP graph: a
 * replay of such a capture would launch with another call's descriptors.  The
 * exception is a step over one tensor that keeps its storage
 * (stq_fused_mdq_adamw, or stq_multi_tensor_mdq_adamw with one tensor with
 * elements): its descriptor travels as a kernel argument (no table), so on a
 * capturing stream the graph records one kernel node that each replay runs
 * with the captured pointers and constants (step, lr, seed ...), as a
 * captured launch of the reference's kernel would (since STQ_ABI_VERSION 4).
 */
#ifndef STQUANT_HIP_H
#define STQUANT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STQ_ABI_VERSION 4

enum stq_status {
    STQ_OK = 0,
    STQ_ERR_INVALID = 1, /* bad argument; nothing was launched            */
    STQ_ERR_HIP = 2      /* HIP runtime error while queueing device work  */
};

/* Element types, named as torch names them in error messages. */
enum stq_dtype {
    STQ_FLOAT = 0,    /* float32  ("Float")    */
    STQ_BFLOAT16 = 1, /* bfloat16 ("BFloat16") */
    STQ_HALF = 2,     /* float16  ("Half")     */
    STQ_BYTE = 3,     /* uint8    ("Byte")     */
    STQ_CHAR = 4,     /* int8     ("Char")     */
    STQ_SHORT = 5,    /* int16    ("Short")    */
    STQ_UINT16 = 6,   /* uint16   ("UInt16")   */
    STQ_INT = 7,      /* int32    ("Int")      */
    STQ_UINT32 = 8,   /* uint32   ("UInt32")   */
    STQ_LONG = 9      /* int64    ("Long")     */
};

enum stq_rounding {
    STQ_ROUND_NEAREST = 0,    /* round half away from zero (the reference) */
    STQ_ROUND_STOCHASTIC = 1  /* floor(x + u), u from Philox4x32-7 (codes <= 16 bits) */
};

/*
 * One fused dequant -> AdamW -> requant step on one parameter tensor.
 *
 * Replaces launch_fused_mdq_adamw (/root/reference/CUDA/stquant_kernel.cu:414-465),
 * which the reference binds to Python as stquant_timetest_cpp.fused_mdq_adamw
 * (/root/reference/CUDA/stquant_core.cpp:3-14).  Same arguments in the same
 * order, each torch::Tensor split into (pointer, dtype, numel):
 *
 *   p           float32[numel], updated in place
 *   grad        float32 (the reference) or bfloat16 / float16 [numel], read only
 *   exp_avg     m codes: uint8 packed nibbles (bits == 4, exp_avg_sq_numel == 0),
 *               else int8 / int16 / int32 [numel]
 *   exp_avg_sq  v codes: empty (packed) or uint8 / uint16 / uint32 [numel]
 *   scale_m, scale_v, v_min   float32[ceil(numel / B)], B = min(block_size, 1024)
 *   beta1 .. eps              AdamW hyper-parameters (fp32)
 *   step        the tensor's step count, already incremented (>= 1)
 *   bits        code width: 4 for packed nibbles, 1..8 / 1..16 / 1..32 otherwise
 *   block_size  quant block size; min(block_size, 1024) must be a power of two
 *   profile_cycles  NULL (profile_numel == 0) or int64[>= 5] device buffer that
 *               receives += clock64 cycles of the dequant / adam_mv /
 *               scale_reduce / quant / update_p phases
 *
 * Extensions beyond the reference: grad dtype, rounding / seed / tensor_id
 * (stochastic rounding stream), the stream argument, and 64-bit numel.
 * Storage dispatch and its error message follow stquant_kernel.cu:430-464.
 * A call on a stream that is capturing a HIP graph is captured as one kernel
 * node (see the top of this file).
 */
int stq_fused_mdq_adamw(float *p, const void *grad, int grad_dtype, int64_t grad_numel,
                        int64_t numel,
                        void *exp_avg, int exp_avg_dtype, int64_t exp_avg_numel,
                        void *exp_avg_sq, int exp_avg_sq_dtype, int64_t exp_avg_sq_numel,
                        float *scale_m, int64_t scale_m_numel,
                        float *scale_v, int64_t scale_v_numel,
                        float *v_min, int64_t v_min_numel,
                        float beta1, float beta2, float lr, float weight_decay, float eps,
                        int step, int bits, int block_size,
                        int64_t *profile_cycles, int64_t profile_numel,
                        int rounding, uint64_t seed, uint32_t tensor_id,
                        void *stream);

/*
 * One tensor of a multi-tensor step; fields as in stq_fused_mdq_adamw, plus
 * elem_offset: the index of element 0 in the stochastic-rounding stream of
 * tensor_id (0 for a whole tensor; for a piece of a larger tensor, the piece's
 * start within it, so that stepping every piece draws the same random numbers
 * as stepping the whole tensor).  It must be >= 0 and a multiple of
 * min(block_size, 1024); nearest rounding does not use it.
 */
typedef struct stq_tensor {
    float *p;
    const void *grad;
    void *exp_avg;
    void *exp_avg_sq;
    float *scale_m;
    float *scale_v;
    float *v_min;
    int64_t numel;
    int64_t grad_numel;
    int64_t exp_avg_numel;
    int64_t exp_avg_sq_numel;
    int64_t scale_m_numel;
    int64_t scale_v_numel;
    int64_t v_min_numel;
    float beta1, beta2, lr, weight_decay, eps;
    int32_t step;
    int32_t bits;
    uint32_t tensor_id;
    int64_t elem_offset;
} stq_tensor;

/*
 * Multi-tensor apply: one kernel launch walks all n_tensors tensors from one
 * packed metadata buffer.  Per-element results are identical to calling
 * stq_fused_mdq_adamw once per tensor.  All tensors share the storage dtype
 * pair, the grad dtype, the block size and the rounding mode; step, bits and
 * the AdamW hyper-parameters are per tensor.  The tensors' arrays must not overlap one another
 * (the tensors are stepped concurrently, not one after the other).
 *
 * No reference counterpart as one call: it replaces the per-tensor launch loop
 * of MDQAdamWSimple.step (/root/reference/CUDA/stquant_opt_simple.py:501-502
 * -> :246-263) and MDQAdamWSimpleFusedIO (/root/reference/CUDA/stquant_opt_fused_io.py:60-77).
 */
int stq_multi_tensor_mdq_adamw(const stq_tensor *tensors, int n_tensors,
                               int grad_dtype, int exp_avg_dtype, int exp_avg_sq_dtype,
                               int block_size, int rounding, uint64_t seed,
                               int64_t *profile_cycles, int64_t profile_numel,
                               void *stream);

/* Tensors per call of stq_multi_tensor_mdq_adamw_noalloc (its fixed descriptor space). */
#define STQ_NOALLOC_MAX_TENSORS 4096

/*
 * stq_multi_tensor_mdq_adamw without any allocation, for callers that cannot
 * allocate: loops that forbid hipMalloc / hipHostMalloc / heap allocation
 * during a step (serving and training loops with a fixed memory plan).  No
 * counterpart in the reference.  Same arguments and results; at most
 * STQ_NOALLOC_MAX_TENSORS tensors per call (more: STQ_ERR_INVALID).
 *
 * The descriptor table lives in a fixed device array of the library
 * (STQ_NOALLOC_MAX_TENSORS * 184 bytes = 736 KiB, held by every GPU the
 * library runs on until the process ends) and is copied there from a static
 * host buffer with hipMemcpyAsync on `stream`: the host buffer is free again
 * when that call returns (pageable memory, copied synchronously).  All calls on
 * one GPU share the array, so each call's copy waits on the device for the
 * previous call's kernel, on whatever stream it ran (an event created once per
 * device at the first call): calls on different streams of one GPU are
 * serialised by the library, each runs on the table it uploaded.  Calls from
 * several host threads are serialised by a lock.
 */
int stq_multi_tensor_mdq_adamw_noalloc(const stq_tensor *tensors, int n_tensors,
                                       int grad_dtype, int exp_avg_dtype, int exp_avg_sq_dtype,
                                       int block_size, int rounding, uint64_t seed,
                                       int64_t *profile_cycles, int64_t profile_numel,
                                       void *stream);

/*
 * Per-tensor gradient statistics of the MDQ bit decision, for a whole tensor
 * list: for tensor i with numel[i] elements of grad_dtype (STQ_FLOAT,
 * STQ_BFLOAT16 or STQ_HALF) at grads[i],
 *   stats[3i + 0] = sqrt(mean(g^2)),
 *   stats[3i + 1] = std(g) / (mean(|g|) + 1e-12)   (std unbiased; NaN if numel == 1),
 *   stats[3i + 2] = mean(g^2)                       (NaN means if numel == 0),
 * into the device array stats[3 * n_tensors].  Sums are accumulated in fp64 in
 * a fixed order (deterministic); the final divisions, square roots and the
 * 1e-12 add are fp32, as the reference's.  Differs from the reference's fp32
 * torch reductions by rounding only (about 1e-7 relative).  grads and numels
 * are host arrays; the library keeps the descriptor table and the partial
 * sums (24 bytes per 32768 elements) in its per-device ring.
 *
 * Replaces MDQAdamWSimple._compute_grad_stats called once per tensor
 * (/root/reference/CUDA/stquant_opt_simple.py:93-98, loop at :427-431).
 */
int stq_multi_tensor_grad_stats(const void *const *grads, const int64_t *numels, int n_tensors,
                                int grad_dtype, float *stats, void *stream);

/* Code storage classes of stq_code_convert (the m/v code layouts the step kernels read). */
enum {
    STQ_STORE_P4 = 0,   /* uint8 bytes (v << 4) | (m + 8), no separate v array */
    STQ_STORE_S8 = 1,   /* int8 m, uint8 v   */
    STQ_STORE_S16 = 2,  /* int16 m, uint16 v */
    STQ_STORE_S32 = 3   /* int32 m, uint32 v */
};

typedef struct stq_code_convert {
    const void *src_exp_avg;     /* m codes (or packed bytes) in src_storage */
    const void *src_exp_avg_sq;  /* v codes in src_storage (unused for STQ_STORE_P4) */
    void *dst_exp_avg;           /* m codes (or packed bytes) in dst_storage */
    void *dst_exp_avg_sq;        /* v codes in dst_storage (unused for STQ_STORE_P4) */
    int64_t numel;
    int32_t src_storage, dst_storage;
} stq_code_convert;

/*
 * Re-stores the m/v codes of n_tensors tensors from one storage class to
 * another, in one launch: the value map decode(src) -> clamp to dst's range
 * -> encode(dst), where P4 decodes to m = (b & 15) - 8, v = b >> 4 and encodes
 * as clamp(m + 8, 0, 15) | clamp(v, 0, 15) << 4, and the integer classes clamp
 * m to their signed and v to their unsigned range.  This is every storage
 * change MDQAdamWSimple makes on a bit-width change: the alignment before the
 * step and the nibble packing after it
 * (/root/reference/CUDA/stquant_opt_simple.py:140-210), which the reference
 * runs as several torch passes per tensor.  Source and destination must not
 * overlap.
 */
int stq_multi_tensor_convert_codes(const stq_code_convert *items, int n_tensors, void *stream);

/* Destination codes of one tensor of stq_multi_tensor_mdq_adamw_restore. */
typedef struct stq_code_out {
    void *exp_avg;              /* new m codes (or packed bytes) in dst_storage */
    void *exp_avg_sq;           /* new v codes in dst_storage (unused for STQ_STORE_P4) */
    int64_t exp_avg_numel;
    int64_t exp_avg_sq_numel;
} stq_code_out;

/*
 * A step that changes the code storage of every tensor in the list, in one
 * launch: the multi-tensor step of stq_multi_tensor_mdq_adamw reading each
 * tensor's codes from tensors[i].exp_avg / exp_avg_sq in src_storage and
 * writing its new codes to out[i] in dst_storage (scales, params in place).
 * The result is exactly that of MDQAdamWSimple's route for a tensor whose bit
 * width changed (/root/reference/CUDA/stquant_opt_simple.py:231-280): align the
 * old codes to the new width (:140-173: unpack nibbles, widen, or clamp to the
 * int8 / int16 range, old scales kept), run the kernel at the new width, pack
 * 4-bit codes into nibbles (:175-210) -- without the separate passes.
 *
 * Every tensor's bits must fit dst_storage as the reference stores that width:
 * STQ_STORE_P4 for bits == 4, STQ_STORE_S8 for 1..8, STQ_STORE_S16 for 9..16,
 * STQ_STORE_S32 for 32; src_storage != dst_storage; min(block_size, 1024) must
 * be 64, 128 or 256.  Source and destination codes must not overlap.  Other
 * arguments as stq_multi_tensor_mdq_adamw.
 */
int stq_multi_tensor_mdq_adamw_restore(const stq_tensor *tensors, const stq_code_out *out, int n_tensors,
                                       int grad_dtype, int src_storage, int dst_storage,
                                       int block_size, int rounding, uint64_t seed,
                                       int64_t *profile_cycles, int64_t profile_numel,
                                       void *stream);

/* Last error message of this thread ("" when none). */
const char *stq_last_error(void);

/* STQ_ABI_VERSION of the loaded library. */
int stq_abi_version(void);

/*
 * *count = the number of descriptor tables the step entry points
 * (stq_fused_mdq_adamw, stq_multi_tensor_mdq_adamw,
 * stq_multi_tensor_mdq_adamw_restore) have uploaded on the current device
 * since the library was loaded.  When every tensor of a call has the same step
 * count and AdamW constants, the step-dependent constants travel as kernel
 * arguments, so the table of a fixed tensor set stays the same from step to
 * step; a call whose table equals one that an earlier call on the same stream
 * left on the device launches from that copy and uploads nothing.  No
 * reference counterpart: it lets a caller (and the tests) check that steady
 * steps run without uploads.
 */
int stq_step_table_uploads(int64_t *count);

/*
 * Device copies of the step's fp32 math, for checking it against a CPU
 * implementation (no reference counterpart: the reference calls CUDA libm).
 *   which = 0: e^x, 1: log x (x a positive normal, +inf or NaN),
 *   3: 1 / x as the stochastic requant computes it (x a positive normal; it
 *   must equal IEEE division).
 * stq_device_math: y[i] = f(x[i]) for device arrays x, y of n floats; or, for
 *   which = 2 (n even), the step kernel's fast v-code map: for each pair
 *   (x[2i], x[2i+1]) = (dv, vmin), dv a positive normal float,
 *   (y[2i], y[2i+1]) = (ln 2 / dv, -vmin / dv) as the kernel computes them;
 *   for which = 4 (n a multiple of 6), the stochastic requant's fast v code:
 *   for each 6-tuple (x, kv, dv, vmin, lmax, QV) the estimate Zh of T - 1/2 and
 *   its error bound ep, as (Zh, ep, 0, 0, 0, 0).
 * stq_device_math_digests: for the bit patterns first .. first+count-1, the
 *   sum over each chunk of mix64(bits(x) << 32 | bits(f(x))) into
 *   digests[ceil(count / chunk)] (device uint64, zeroed by the caller).
 */
int stq_device_math(int which, const float *x, float *y, int64_t n, void *stream);
int stq_device_math_digests(int which, uint32_t first, uint32_t count, uint32_t chunk,
                            uint64_t *digests, void *stream);

/*
 * max(0, max over the floats x with bit patterns first .. first+count-1
 * (positive and finite) of |v_log_f32(x) * ln 2 - l(x)| - slope * |l(x)|),
 * l = the kernels' log, computed in fp64 and atomically max-ed, as the bit
 * pattern of a double, into the device uint64 *max_err_bits (zeroed by the
 * caller).  The step kernel's fast v-code path relies on this bound, with
 * slope 0 and with the slope it uses (no reference counterpart).
 */
int stq_device_log_approx_error(uint32_t first, uint32_t count, double slope, uint64_t *max_err_bits,
                                void *stream);

/*
 * The largest distance, in units in the last place, between the hardware square root
 * (which = 0, v_sqrt_f32) or reciprocal (which = 1, v_rcp_f32) that the step's
 * parameter update uses and the correctly rounded result, over the floats with bit
 * patterns first .. first+count-1 (positive, with positive normal results), atomically
 * max-ed into the device uint32 *max_ulps (zeroed by the caller).  The parameter
 * tolerance of the parity tests is derived from this bound (no reference counterpart:
 * the reference's update uses IEEE sqrtf and division).
 */
int stq_device_hw_ulp_error(int which, uint32_t first, uint32_t count, uint32_t *max_ulps, void *stream);

/* Host (CPU) builds of the same inline functions the kernels use. */
void stq_host_math(int which, const float *x, float *y, int64_t n);
/* out[i] = round-half-away(u[i] / d[i]) via the kernel's fp32 fma method,
 * starting from the correctly rounded 1/d perturbed by inv_ulps units in the
 * last place (the device starts from a hardware reciprocal within 1 ulp). */
void stq_host_round_half_away(const float *u, const float *d, float *out, int64_t n, int inv_ulps);
/* out[i] = x[i] / (2^bits - 1) as the kernel computes the new v scale
 * (a correction step that must equal IEEE division). */
void stq_host_div_code_range(const float *x, float *out, int64_t n, int bits);
/* The library's Philox4x32 round function run 10 times (Random123's default, whose
 * known-answer vectors pin it); the stochastic step runs the same rounds 7 times. */
void stq_host_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

#ifdef __cplusplus
}
#endif

#endif /* STQUANT_HIP_H */
