// mdq_capi.cpp -- C ABI of the fused MDQ AdamW step (declared in
// include/stquant_hip.h): argument checks, per-tensor AdamW constants,
// descriptor packing/upload and kernel dispatch.
//
// Replaces launch_fused_mdq_adamw (/root/reference/CUDA/stquant_kernel.cu:414-465)
// and its pybind shim (/root/reference/CUDA/stquant_core.cpp:3-14).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/stquant_hip.h"
#include "mdq_desc.h"
#include "mdq_launch.h"
#include "mdq_math.h"
#include "mdq_convert.h"
#include "mdq_stats.h"

namespace {

using mdq::MdqDesc;

thread_local std::string g_err;

int fail(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what)
{
    return fail(STQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

const char *dtype_name(int dt)
{
    switch (dt) {
    case STQ_FLOAT: return "Float";
    case STQ_BFLOAT16: return "BFloat16";
    case STQ_HALF: return "Half";
    case STQ_BYTE: return "Byte";
    case STQ_CHAR: return "Char";
    case STQ_SHORT: return "Short";
    case STQ_UINT16: return "UInt16";
    case STQ_INT: return "Int";
    case STQ_UINT32: return "UInt32";
    case STQ_LONG: return "Long";
    default: return "Unknown";
    }
}

// Storage dispatch of stquant_kernel.cu:430-464.  Returns the storage class or
// -1 (message set).  packed4 needs bits == 4, uint8 m codes, empty v codes.
int pick_storage(int bits, int ea_dt, int64_t ea_numel, int easq_dt, int64_t easq_numel, int64_t numel)
{
    if (bits == 4 && ea_dt == STQ_BYTE && easq_numel == 0) {
        if (ea_numel != numel) {
            fail(STQ_ERR_INVALID, "packed4: exp_avg numel must match parameters");
            return -1;
        }
        return mdq::ST_P4;
    }
    if (ea_dt == STQ_CHAR && easq_dt == STQ_BYTE) return mdq::ST_S8;
    if (ea_dt == STQ_SHORT && easq_dt == STQ_UINT16) return mdq::ST_S16;
    if (ea_dt == STQ_INT && easq_dt == STQ_UINT32) return mdq::ST_S32;
    fail(STQ_ERR_INVALID,
         "MDQ: state must be packed4 (uint8+empty), (int8,uint8), (int16,uint16) or (int32,uint32), got %s / %s bits=%d",
         dtype_name(ea_dt), dtype_name(easq_dt), bits);
    return -1;
}

int storage_width(int st)
{
    switch (st) {
    case mdq::ST_P4: return 4;
    case mdq::ST_S8: return 8;
    case mdq::ST_S16: return 16;
    default: return 32;
    }
}

int code_bytes(int st) { return st == mdq::ST_P4 ? 1 : storage_width(st) / 8; }

const char *storage_name(int st)
{
    switch (st) {
    case mdq::ST_P4: return "packed nibbles";
    case mdq::ST_S8: return "int8/uint8";
    case mdq::ST_S16: return "int16/uint16";
    default: return "int32/uint32";
    }
}


bool is_aligned(const void *ptr, int bytes) { return ((uintptr_t)ptr % (uintptr_t)bytes) == 0; }

// Checks one tensor and fills its descriptor (tile range filled by the caller).
int make_desc(const stq_tensor &t, int storage, int grad_dt, int B, MdqDesc &d)
{
    if (t.numel < 0) return fail(STQ_ERR_INVALID, "numel must be >= 0");
    if (t.grad_numel != t.numel)
        return fail(STQ_ERR_INVALID, "grad numel (%lld) must match parameters (%lld)",
                    (long long)t.grad_numel, (long long)t.numel);
    if (t.bits < 1 || t.bits > storage_width(storage))
        return fail(STQ_ERR_INVALID, "bits=%d does not fit the %d-bit code storage", t.bits,
                    storage_width(storage));
    if (storage == mdq::ST_P4) {
        if (t.exp_avg_numel != t.numel)
            return fail(STQ_ERR_INVALID, "packed4: exp_avg numel must match parameters");
    } else if (t.exp_avg_numel < t.numel || t.exp_avg_sq_numel < t.numel) {
        return fail(STQ_ERR_INVALID, "exp_avg / exp_avg_sq must hold numel (%lld) codes",
                    (long long)t.numel);
    }
    if (t.step < 1) return fail(STQ_ERR_INVALID, "step must be >= 1 (incremented by the caller), got %d", t.step);
    if (t.elem_offset < 0 || t.elem_offset % B != 0)
        return fail(STQ_ERR_INVALID, "elem_offset (%lld) must be >= 0 and a multiple of the block size %d",
                    (long long)t.elem_offset, B);
    const int64_t nb = (t.numel + B - 1) / B;
    if (t.scale_m_numel < nb || t.scale_v_numel < nb || t.v_min_numel < nb)
        return fail(STQ_ERR_INVALID, "scale_m / scale_v / v_min need ceil(numel / %d) = %lld elements", B,
                    (long long)nb);
    if (t.numel > 0 && (!t.p || !t.grad || !t.exp_avg || !t.scale_m || !t.scale_v || !t.v_min ||
                        (storage != mdq::ST_P4 && !t.exp_avg_sq)))
        return fail(STQ_ERR_INVALID, "null data pointer");
    const int gb = grad_dt == STQ_FLOAT ? 4 : 2;
    const int cb = code_bytes(storage);
    // Every array must start on a multiple of its element size (torch tensors always do): the
    // tile modes derive p's and the grads' place in their cache lines from element counts.
    if (t.numel > 0 && !(is_aligned(t.p, 4) && is_aligned(t.grad, gb) && is_aligned(t.exp_avg, cb) &&
                         (storage == mdq::ST_P4 || is_aligned(t.exp_avg_sq, cb)) && is_aligned(t.scale_m, 4) &&
                         is_aligned(t.scale_v, 4) && is_aligned(t.v_min, 4)))
        return fail(STQ_ERR_INVALID, "data pointers must be aligned to their element size");

    std::memset(&d, 0, sizeof d);
    d.p = t.p;
    d.g = t.grad;
    d.code_m = t.exp_avg;
    d.code_v = storage == mdq::ST_P4 ? nullptr : t.exp_avg_sq;
    d.scale_m = t.scale_m;
    d.scale_v = t.scale_v;
    d.v_min = t.v_min;
    d.numel = t.numel;
    // AdamW constants as stquant_kernel.cu:83-84,136-142 form them in fp32.
    d.b1 = t.beta1;
    d.omb1 = 1.0f - t.beta1;
    d.b2 = t.beta2;
    d.omb2 = 1.0f - t.beta2;
    d.eps = t.eps;
    const float bc1 = 1.0f - powf(t.beta1, (float)t.step);
    const float bc2 = 1.0f - powf(t.beta2, (float)t.step);
    d.step_size = t.lr / bc1;
    d.inv_sqrt_bc2 = 1.0f / sqrtf(bc2);
    d.decay = t.weight_decay != 0.0f ? 1.0f - t.lr * t.weight_decay : 1.0f;
    d.qm = ldexpf(1.0f, t.bits - 1);
    d.inv_qm = ldexpf(1.0f, -(t.bits - 1));
    d.qvf = (float)(std::ldexp(1.0, t.bits) - 1.0);
    d.inv_qvf = 1.0f / d.qvf;
    d.ep0_rn = mdq::mdq_rn_ep0(d.qvf);
    d.ep0_sr = mdq::mdq_sr_ep0(d.qvf);
    d.bits = (uint32_t)t.bits;
    d.step = (uint32_t)t.step;
    d.tensor_id = t.tensor_id;
    d.rng_origin = t.elem_offset;
    // full tiles move codes in 4-element quads (4 * cb bytes), 1-byte codes in 8-byte pairs
    const int ca = (storage == mdq::ST_S8 || storage == mdq::ST_P4) ? 8 : 4 * cb;
    const bool codes_al = is_aligned(t.exp_avg, ca) && (storage == mdq::ST_P4 || is_aligned(t.exp_avg_sq, ca));
    const bool pg_al = is_aligned(t.p, 16) && is_aligned(t.grad, 4 * gb);
    const bool pg_lines = is_aligned(t.p, 128) && is_aligned(t.grad, 128);
    // p and grads are always element-aligned (fp32 p, 2- or 4-byte grads): element accesses need no more
    d.flags = (codes_al ? mdq::DF_CODES_ALIGNED : 0u) | (codes_al && pg_al ? mdq::DF_ALIGNED : 0u) |
              (codes_al && pg_lines ? mdq::DF_LINES : 0u);
    return STQ_OK;
}

// ----------------------------------------------------- per-device resources
// A device buffer holding n MdqDesc followed by n int64 tile starts, and its
// pinned host staging copy.
struct Slot {
    char *dev = nullptr;
    char *host = nullptr;
    size_t cap = 0;   // bytes
    hipEvent_t done = nullptr;     // recorded behind the slot's last launch
    hipEvent_t copied = nullptr;   // recorded behind the slot's last upload
    bool pending = false;
    // A step table the device buffer holds (its first table_bytes bytes equal
    // host[0 .. table_bytes)), uploaded for launches on table_stream; 0 when
    // the buffer holds anything else.
    size_t table_bytes = 0;
    hipStream_t table_stream = nullptr;
};

struct DevCtx {
    std::mutex mu;
    int cus = 0;
    int next = 0;
    hipStream_t copy_stream = nullptr;   // descriptor uploads (default priority)
    int64_t table_uploads = 0;           // step tables uploaded (launches without a device copy)
    Slot slots[8];
};

std::mutex g_ctx_mu;
DevCtx *g_ctx[64] = {nullptr};

int get_ctx(DevCtx **out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(STQ_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_ctx_mu);
    if (!g_ctx[dev]) {
        DevCtx *c = new DevCtx();
        e = hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) { delete c; return hip_fail(e, "hipDeviceGetAttribute"); }
        g_ctx[dev] = c;
    }
    *out = g_ctx[dev];
    return STQ_OK;
}

// The next slot of the device's ring with at least `need` device bytes (and
// as many pinned staging bytes), after the work recorded behind its previous
// use has completed.  Called with ctx->mu held.
int take_slot(DevCtx *ctx, size_t need, Slot **out)
{
    Slot &s = ctx->slots[ctx->next];
    ctx->next = (ctx->next + 1) % 8;
    s.table_bytes = 0;
    hipError_t e;
    if (s.pending) {
        e = hipEventSynchronize(s.done);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
        s.pending = false;
    }
    if (s.cap < need) {
        if (s.dev) { (void)hipFree(s.dev); s.dev = nullptr; }
        if (s.host) { (void)hipHostFree(s.host); s.host = nullptr; }
        s.cap = 0;
        size_t cap = need < 16384 ? 16384 : need + need / 2;
        e = hipMalloc((void **)&s.dev, cap);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(descriptors)");
        e = hipHostMalloc((void **)&s.host, cap, hipHostMallocDefault);
        if (e != hipSuccess) return hip_fail(e, "hipHostMalloc(descriptors)");
        s.cap = cap;
    }
    if (!s.done) {
        e = hipEventCreateWithFlags(&s.done, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
    }
    if (!s.copied) {
        e = hipEventCreateWithFlags(&s.copied, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(e, "hipEventCreate");
    }
    *out = &s;
    return STQ_OK;
}

// Whether `stream` is capturing a HIP graph.
int is_capturing(hipStream_t stream, bool *capturing)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    *capturing = cs != hipStreamCaptureStatusNone;
    return STQ_OK;
}

// Descriptor tables are uploaded from a ring of staging slots that later
// calls refill, so a call captured into a HIP graph would, on replay, launch
// with whatever another call left in its slot.  Every entry point that uploads
// a table refuses a capturing stream before any slot, event or device work
// (a step over one tensor that keeps its storage uploads no table: its
// descriptor travels as a kernel argument, upload_and_launch).
int refuse_capture(hipStream_t stream)
{
    bool capturing = false;
    const int rc = is_capturing(stream, &capturing);
    if (rc != STQ_OK) return rc;
    if (capturing)
        return fail(STQ_ERR_INVALID,
                    "the stream is capturing a HIP graph: this library uploads each call's descriptor table "
                    "from staging buffers that later calls reuse, so a replay would step other tensors; "
                    "call it outside graph capture (a step over one tensor, as fused_mdq_adamw, can be "
                    "captured)");
    return STQ_OK;
}

// Copies the first `bytes` of the slot's staging buffer to its device buffer
// so that work queued next on `stream` sees them.  The copy goes on the
// device's copy stream and `stream` waits for it: a copy queued on `stream`
// itself would start only after the previous kernel there has finished, and
// the next kernel would wait for it, leaving the GPU idle between
// back-to-back steps.  The slot is free (take_slot waited for its last
// launch), so the copy cannot overwrite descriptors still in use.  A launch
// over fewer than SMALL_LAUNCH_ELEMS elements (a kernel of a few tens of
// microseconds) gets the copy on `stream` itself: there the cross-stream wait
// costs more than the overlap saves (flat 4M-element step 26.5 -> 17.7 us per
// call; GPT-2 small, 124M elements, 277 us per call with the copy stream, 286
// without; LLaMA-7B level).  Called with ctx->mu held.
constexpr int64_t SMALL_LAUNCH_ELEMS = int64_t(1) << 24;

int upload(DevCtx *ctx, Slot &s, size_t bytes, int64_t elems, hipStream_t stream)
{
    hipError_t e;
    const bool on_stream = elems < SMALL_LAUNCH_ELEMS;
    if (!on_stream && !ctx->copy_stream) {
        e = hipStreamCreateWithFlags(&ctx->copy_stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            ctx->copy_stream = nullptr;
            return hip_fail(e, "hipStreamCreate(descriptor copies)");
        }
    }
    if (on_stream) {
        e = hipMemcpyAsync(s.dev, s.host, bytes, hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(descriptors)");
        e = hipEventRecord(s.copied, stream);
        return e == hipSuccess ? STQ_OK : hip_fail(e, "hipEventRecord");
    }
    e = hipMemcpyAsync(s.dev, s.host, bytes, hipMemcpyHostToDevice, ctx->copy_stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(descriptors)");
    e = hipEventRecord(s.copied, ctx->copy_stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
    e = hipStreamWaitEvent(stream, s.copied, 0);
    return e == hipSuccess ? STQ_OK : hip_fail(e, "hipStreamWaitEvent");
}

// Marks the slot busy until the work queued so far on `stream` completes.
int release_slot(Slot *s, hipStream_t stream)
{
    hipError_t e = hipEventRecord(s->done, stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
    s->pending = true;
    return STQ_OK;
}

// Whether a launch over these descriptors needs the kernel variant with the staged tile
// modes: some tensor has whole tiles and aligned codes but p or grads off their 128-byte
// lines.  Launches without one take the variant that has only the vector and guarded
// tile modes (same-box A/B, LLaMA-7B 4-bit stochastic: 13.71 ms with the staged modes in
// the same kernel, 13.48 without).
bool launch_needs_views(const MdqDesc *descs, size_t n, int log2b)
{
    const int64_t te = mdq::tile_elems(1 << log2b);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t f = descs[i].flags;
        if ((f & mdq::DF_CODES_ALIGNED) && !(f & mdq::DF_LINES) && descs[i].numel >= te) return true;
    }
    return false;
}

// Launches the step kernel of (src_storage -> storage) over the nd
// descriptors at dd, which the tile starts follow in the same device buffer;
// one workgroup per tile (total_tiles).
hipError_t launch_step(const MdqDesc *dd, int nd, int src, int storage, int grad_dt, int log2b, bool sr,
                       int64_t total_tiles, unsigned long long *prof, const mdq::StepArgs &sa, bool views,
                       hipStream_t stream)
{
    if (src == storage) {
        switch (storage) {
        case mdq::ST_P4: return mdq::launch_p4(dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
        case mdq::ST_S8: return mdq::launch_s8(dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
        case mdq::ST_S16: return mdq::launch_s16(dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
        default: return mdq::launch_s32(dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
        }
    }
    switch (storage) {
    case mdq::ST_P4: return mdq::launch_tr_p4(src, dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
    case mdq::ST_S8: return mdq::launch_tr_s8(src, dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
    case mdq::ST_S16: return mdq::launch_tr_s16(src, dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
    default: return mdq::launch_tr_s32(src, dd, nd, total_tiles, grad_dt, log2b, sr, prof, sa, views, stream);
    }
}

// Launches the step kernel over one tensor whose descriptor d (tile_begin 0) travels as a
// kernel argument.
hipError_t launch_step_one(const MdqDesc &d, int storage, int grad_dt, int log2b, bool sr, int64_t total_tiles,
                           unsigned long long *prof, const mdq::StepArgs &sa, hipStream_t stream)
{
    switch (storage) {
    case mdq::ST_P4: return mdq::launch_one_p4(d, total_tiles, grad_dt, log2b, sr, prof, sa, stream);
    case mdq::ST_S8: return mdq::launch_one_s8(d, total_tiles, grad_dt, log2b, sr, prof, sa, stream);
    case mdq::ST_S16: return mdq::launch_one_s16(d, total_tiles, grad_dt, log2b, sr, prof, sa, stream);
    default: return mdq::launch_one_s32(d, total_tiles, grad_dt, log2b, sr, prof, sa, stream);
    }
}

// The same bits (so +0 / -0 and NaN patterns count as different).
bool same_bits(float a, float b) { return std::memcmp(&a, &b, sizeof a) == 0; }

// Launches the step kernel over n descriptors on `stream`.  The table (the
// descriptors, then their int64 tile starts) goes to the device through a
// slot of the ring; the slot's pinned staging buffer is reused only after the
// event recorded behind its previous launch has completed.  When every tensor
// has the same step_size, inv_sqrt_bc2 and step, those go in the kernel
// arguments and the table holds 0 in their place, so a fixed tensor set has
// the same table at every step: a slot whose device buffer already holds it,
// uploaded for a launch on this stream, is launched from again without an
// upload (the copy and, for large launches, the wait for the copy stream
// leave the GPU idle between back-to-back steps).  `storage` is the code
// storage the kernel writes; it reads `src_storage` (the same, except on a
// storage-changing step).  A step over one tensor that keeps its storage
// launches with its descriptor as a kernel argument instead (mdq_step_kernel_one:
// no table, no ring slot, no event; the flat 4,194,304-element step 14.6 -> 11.9
// us per call, same-allocation A/B), which also makes it capturable: on a stream
// that is capturing a HIP graph it records a plain kernel node that replays with
// the captured pointers and constants, as a captured launch of the reference's
// kernel would.  Other calls are refused under capture.
int upload_and_launch(const MdqDesc *descs, size_t n, int src_storage, int storage, int grad_dt, int log2b,
                      bool sr, int64_t total_tiles, unsigned long long *prof, uint64_t seed, hipStream_t stream)
{
    bool capturing = false;
    int rc = is_capturing(stream, &capturing);
    if (rc != STQ_OK) return rc;
    if (capturing && !(n == 1 && src_storage == storage)) return refuse_capture(stream);
    mdq::StepArgs sa{seed, 0.0f, 0.0f, 0u, 0u};
    bool uniform = n > 0;
    for (size_t i = 1; i < n && uniform; ++i)
        uniform = same_bits(descs[i].step_size, descs[0].step_size) &&
                  same_bits(descs[i].inv_sqrt_bc2, descs[0].inv_sqrt_bc2) && descs[i].step == descs[0].step;
    if (uniform) {
        sa.step_size = descs[0].step_size;
        sa.inv_sqrt_bc2 = descs[0].inv_sqrt_bc2;
        sa.step = descs[0].step;
        sa.uniform = 1u;
    }
    if (n == 1 && src_storage == storage) {
        const hipError_t e = launch_step_one(descs[0], storage, grad_dt, log2b, sr, total_tiles, prof, sa, stream);
        return e == hipSuccess ? STQ_OK : hip_fail(e, "kernel launch");
    }
    DevCtx *ctx = nullptr;
    rc = get_ctx(&ctx);
    if (rc != STQ_OK) return rc;
    const size_t need = n * (sizeof(MdqDesc) + sizeof(long long));
    thread_local std::vector<char> table;
    table.resize(need);
    MdqDesc *td = reinterpret_cast<MdqDesc *>(table.data());
    std::memcpy(td, descs, n * sizeof(MdqDesc));
    long long *tb = reinterpret_cast<long long *>(table.data() + n * sizeof(MdqDesc));
    for (size_t i = 0; i < n; ++i) {
        tb[i] = descs[i].tile_begin;
        if (uniform) {
            td[i].step_size = 0.0f;
            td[i].inv_sqrt_bc2 = 0.0f;
            td[i].step = 0u;
        }
    }
    const bool views = launch_needs_views(descs, n, log2b);
    std::lock_guard<std::mutex> lk(ctx->mu);
    Slot *sp = nullptr;
    for (Slot &c : ctx->slots)
        if (c.table_bytes == need && c.table_stream == stream && std::memcmp(c.host, table.data(), need) == 0) {
            sp = &c;
            break;
        }
    hipError_t e;
    if (sp) {
        // The upload was queued before the launch that last used the slot on this
        // stream, so it is complete or ahead of this launch in stream order; wait
        // explicitly only while it is pending (a stream handle can be recycled).
        e = hipEventQuery(sp->copied);
        if (e == hipErrorNotReady) e = hipStreamWaitEvent(stream, sp->copied, 0);
        if (e != hipSuccess) return hip_fail(e, "descriptor table upload");
    } else {
        rc = take_slot(ctx, need, &sp);
        if (rc != STQ_OK) return rc;
        std::memcpy(sp->host, table.data(), need);
        rc = upload(ctx, *sp, need, total_tiles * mdq::tile_elems(1 << log2b), stream);
        if (rc != STQ_OK) return rc;
        sp->table_bytes = need;
        sp->table_stream = stream;
        ++ctx->table_uploads;
    }
    e = launch_step(reinterpret_cast<const MdqDesc *>(sp->dev), (int)n, src_storage, storage, grad_dt, log2b, sr,
                    total_tiles, prof, sa, views, stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return release_slot(sp, stream);
}

// stq_multi_tensor_grad_stats: descriptors, tile starts and the fp64 partial
// sums share one ring slot.
int run_grad_stats(const void *const *grads, const int64_t *numels, int n, int grad_dt, float *stats,
                   hipStream_t stream)
{
    g_err.clear();
    if (grad_dt != STQ_FLOAT && grad_dt != STQ_BFLOAT16 && grad_dt != STQ_HALF)
        return fail(STQ_ERR_INVALID, "grad must be Float, BFloat16 or Half, got %s", dtype_name(grad_dt));
    if (n < 0 || (n > 0 && (!grads || !numels || !stats)))
        return fail(STQ_ERR_INVALID, "grad_stats: bad tensor list or output");
    if (n == 0) return STQ_OK;
    std::vector<mdq::StatDesc> d((size_t)n);
    int64_t tiles = 0;
    for (int i = 0; i < n; ++i) {
        if (numels[i] < 0) return fail(STQ_ERR_INVALID, "tensor %d: negative numel", i);
        if (numels[i] > 0 && !grads[i]) return fail(STQ_ERR_INVALID, "tensor %d: null grad", i);
        d[i].g = grads[i];
        d[i].numel = numels[i];
        d[i].tile_begin = tiles;
        tiles += (numels[i] + mdq::STAT_TILE - 1) / mdq::STAT_TILE;
        d[i].tile_end = tiles;
    }
    if (tiles > 0x7fffffffLL)
        return fail(STQ_ERR_INVALID, "too many tiles in one call (%lld); split the tensor list", (long long)tiles);
    int rc = refuse_capture(stream);
    if (rc != STQ_OK) return rc;
    DevCtx *ctx = nullptr;
    rc = get_ctx(&ctx);
    if (rc != STQ_OK) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const size_t up = (size_t)n * (sizeof(mdq::StatDesc) + sizeof(long long));
    const size_t part_off = (up + 255) / 256 * 256;
    Slot *s = nullptr;
    rc = take_slot(ctx, part_off + (size_t)tiles * mdq::STAT_PARTIALS * sizeof(double), &s);
    if (rc != STQ_OK) return rc;
    std::memcpy(s->host, d.data(), (size_t)n * sizeof(mdq::StatDesc));
    long long *tb = reinterpret_cast<long long *>(s->host + (size_t)n * sizeof(mdq::StatDesc));
    for (int i = 0; i < n; ++i) tb[i] = d[i].tile_begin;
    rc = upload(ctx, *s, up, tiles * mdq::STAT_TILE, stream);
    if (rc != STQ_OK) return rc;
    hipError_t e;
    const mdq::StatDesc *dd = reinterpret_cast<const mdq::StatDesc *>(s->dev);
    const long long *dtb = reinterpret_cast<const long long *>(s->dev + (size_t)n * sizeof(mdq::StatDesc));
    double *partials = reinterpret_cast<double *>(s->dev + part_off);
    e = mdq::launch_grad_stats(dd, dtb, n, tiles, grad_dt, partials, stats, stream);
    if (e != hipSuccess) return hip_fail(e, "grad_stats launch");
    return release_slot(s, stream);
}

int common_checks(int grad_dt, int block_size, int rounding, const int64_t *prof, int64_t prof_numel,
                  int *log2b)
{
    if (grad_dt != STQ_FLOAT && grad_dt != STQ_BFLOAT16 && grad_dt != STQ_HALF)
        return fail(STQ_ERR_INVALID, "grad must be Float, BFloat16 or Half, got %s", dtype_name(grad_dt));
    if (block_size < 1) return fail(STQ_ERR_INVALID, "block_size must be >= 1, got %d", block_size);
    const int B = block_size > 1024 ? 1024 : block_size;   // stquant_kernel.cu:421
    if (B & (B - 1))
        return fail(STQ_ERR_INVALID, "block_size must be a power of two (min(block_size, 1024) = %d)", B);
    int l = 0;
    while ((1 << l) < B) ++l;
    *log2b = l;
    if (rounding != STQ_ROUND_NEAREST && rounding != STQ_ROUND_STOCHASTIC)
        return fail(STQ_ERR_INVALID, "rounding must be 0 (nearest) or 1 (stochastic), got %d", rounding);
    if (prof && prof_numel < 5) return fail(STQ_ERR_INVALID, "profile_cycles needs >= 5 elements");
    return STQ_OK;
}

// Checks the tensors of a step launch and writes the descriptors of those with
// elements to out[0 .. *n_out) (at most cap; the caller checked n_tensors <= cap),
// with their tile ranges; *storage is the tensors' common code storage.
int build_step_descs(const stq_tensor *tensors, int n_tensors, int grad_dt, int ea_dt, int easq_dt, int B,
                     MdqDesc *out, int *n_out, int *storage, int64_t *tiles_out)
{
    const int64_t te = mdq::tile_elems(B);
    int st_all = -1, nd = 0;
    int64_t tiles = 0;
    for (int i = 0; i < n_tensors; ++i) {
        const stq_tensor &t = tensors[i];
        const int st = pick_storage(t.bits, ea_dt, t.exp_avg_numel, easq_dt, t.exp_avg_sq_numel, t.numel);
        if (st < 0) return STQ_ERR_INVALID;
        if (st_all >= 0 && st != st_all)
            return fail(STQ_ERR_INVALID, "all tensors of one call must share the code storage");
        st_all = st;
        MdqDesc d;
        const int rc = make_desc(t, st, grad_dt, B, d);
        if (rc != STQ_OK) {
            g_err = "tensor " + std::to_string(i) + ": " + g_err;
            return rc;
        }
        if (t.numel == 0) continue;
        d.tile_begin = tiles;
        tiles += (t.numel + te - 1) / te;
        d.tile_end = tiles;
        out[nd++] = d;
    }
    if (tiles > 0x7fffffffLL)
        return fail(STQ_ERR_INVALID, "too many tiles in one call (%lld); split the tensor list", (long long)tiles);
    *n_out = nd;
    *storage = st_all;
    *tiles_out = tiles;
    return STQ_OK;
}

int run(const stq_tensor *tensors, int n_tensors, int grad_dt, int ea_dt, int easq_dt, int block_size,
        int rounding, uint64_t seed, int64_t *prof, int64_t prof_numel, void *stream)
{
    g_err.clear();
    if (prof_numel == 0) prof = nullptr;   // empty profile buffer == off (stquant_kernel.cu:403-406)
    int log2b = 0;
    int rc = common_checks(grad_dt, block_size, rounding, prof, prof_numel, &log2b);
    if (rc != STQ_OK) return rc;
    if (n_tensors < 0 || (n_tensors > 0 && !tensors)) return fail(STQ_ERR_INVALID, "bad tensor list");
    std::vector<MdqDesc> descs((size_t)n_tensors);
    int nd = 0, storage = -1;
    int64_t tiles = 0;
    rc = build_step_descs(tensors, n_tensors, grad_dt, ea_dt, easq_dt, 1 << log2b, descs.data(), &nd, &storage,
                          &tiles);
    if (rc != STQ_OK || nd == 0) return rc;
    return upload_and_launch(descs.data(), (size_t)nd, storage, storage, grad_dt, log2b,
                             rounding == STQ_ROUND_STOCHASTIC, tiles, reinterpret_cast<unsigned long long *>(prof),
                             seed, reinterpret_cast<hipStream_t>(stream));
}

// The storage MDQAdamWSimple leaves a `bits`-wide tensor in after a step
// (stquant_opt_simple.py:140-210): nibbles at 4 bits, else int8 / int16 /
// int32 by width; -1 for widths it cannot store (17..31).
int final_storage(int bits)
{
    if (bits == 4) return mdq::ST_P4;
    if (bits >= 1 && bits <= 8) return mdq::ST_S8;
    if (bits >= 9 && bits <= 16) return mdq::ST_S16;
    if (bits == 32) return mdq::ST_S32;
    return -1;
}

bool ranges_overlap(const void *a, int64_t na, const void *b, int64_t nb)
{
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return na > 0 && nb > 0 && a0 < b0 + (uintptr_t)nb && b0 < a0 + (uintptr_t)na;
}

// stq_multi_tensor_mdq_adamw_restore: the step of `run` with source codes in
// src_storage and destination codes in dst_storage.
int run_restore(const stq_tensor *tensors, const stq_code_out *out, int n_tensors, int grad_dt, int src, int dst,
                int block_size, int rounding, uint64_t seed, int64_t *prof, int64_t prof_numel, void *stream)
{
    g_err.clear();
    if (prof_numel == 0) prof = nullptr;
    int log2b = 0;
    int rc = common_checks(grad_dt, block_size, rounding, prof, prof_numel, &log2b);
    if (rc != STQ_OK) return rc;
    if (n_tensors < 0 || (n_tensors > 0 && (!tensors || !out))) return fail(STQ_ERR_INVALID, "bad tensor list");
    if (src < STQ_STORE_P4 || src > STQ_STORE_S32 || dst < STQ_STORE_P4 || dst > STQ_STORE_S32)
        return fail(STQ_ERR_INVALID, "storage must be STQ_STORE_P4 .. STQ_STORE_S32");
    if (src == dst) return fail(STQ_ERR_INVALID, "restore: source and destination storage are the same");
    if (log2b < mdq::TRANSITION_LOG2B_MIN || log2b > mdq::TRANSITION_LOG2B_MAX)
        return fail(STQ_ERR_INVALID, "restore: block size must be 64, 128 or 256, got %d", 1 << log2b);
    const int B = 1 << log2b;
    const int64_t te = mdq::tile_elems(B);
    const int scb = code_bytes(src), dcb = code_bytes(dst);
    const int sca = (src == mdq::ST_S8 || src == mdq::ST_P4) ? 8 : 4 * scb;
    std::vector<MdqDesc> descs;
    descs.reserve((size_t)n_tensors);
    int64_t tiles = 0;
    for (int i = 0; i < n_tensors; ++i) {
        const stq_tensor &t = tensors[i];
        const stq_code_out &o = out[i];
        const std::string at = "tensor " + std::to_string(i) + ": ";
        if (final_storage(t.bits) != dst && !(dst == mdq::ST_S8 && t.bits == 4))
            return fail(STQ_ERR_INVALID, "%sbits=%d is not stored in destination storage %d (%s)", at.c_str(), t.bits,
                        dst, storage_name(dst));
        if (t.numel < 0) return fail(STQ_ERR_INVALID, "%snumel must be >= 0", at.c_str());
        if (src == mdq::ST_P4 ? t.exp_avg_numel != t.numel
                              : (t.exp_avg_numel < t.numel || t.exp_avg_sq_numel < t.numel))
            return fail(STQ_ERR_INVALID, "%ssource codes must hold numel (%lld) codes", at.c_str(), (long long)t.numel);
        if (t.numel > 0 && (!t.exp_avg || (src != mdq::ST_P4 && !t.exp_avg_sq)))
            return fail(STQ_ERR_INVALID, "%snull source code pointer", at.c_str());
        // the source codes are read with element-sized loads: as make_desc requires of the
        // destination's, each array starts on a multiple of its element size
        if (t.numel > 0 && !(is_aligned(t.exp_avg, scb) && (src == mdq::ST_P4 || is_aligned(t.exp_avg_sq, scb))))
            return fail(STQ_ERR_INVALID, "%sdata pointers must be aligned to their element size", at.c_str());
        // the destination arrays are checked as the step's own codes
        stq_tensor td = t;
        td.exp_avg = o.exp_avg;
        td.exp_avg_sq = o.exp_avg_sq;
        td.exp_avg_numel = o.exp_avg_numel;
        td.exp_avg_sq_numel = dst == mdq::ST_P4 ? 0 : o.exp_avg_sq_numel;
        MdqDesc d;
        rc = make_desc(td, dst, grad_dt, B, d);
        if (rc != STQ_OK) {
            g_err = at + g_err;
            return rc;
        }
        if (t.numel == 0) continue;
        const int64_t sb = t.numel * scb, db = t.numel * dcb;
        const void *sv = src == mdq::ST_P4 ? nullptr : t.exp_avg_sq;
        const void *dv = dst == mdq::ST_P4 ? nullptr : o.exp_avg_sq;
        if (ranges_overlap(t.exp_avg, sb, o.exp_avg, db) || (sv && ranges_overlap(sv, sb, o.exp_avg, db)) ||
            (dv && ranges_overlap(t.exp_avg, sb, dv, db)) || (sv && dv && ranges_overlap(sv, sb, dv, db)))
            return fail(STQ_ERR_INVALID, "%ssource and destination codes overlap", at.c_str());
        d.out_m = o.exp_avg;
        d.out_v = dst == mdq::ST_P4 ? nullptr : o.exp_avg_sq;
        d.code_m = t.exp_avg;
        d.code_v = src == mdq::ST_P4 ? nullptr : t.exp_avg_sq;
        if (!(is_aligned(d.code_m, sca) && (src == mdq::ST_P4 || is_aligned(d.code_v, sca))))
            d.flags &= ~(mdq::DF_ALIGNED | mdq::DF_CODES_ALIGNED | mdq::DF_LINES);
        d.tile_begin = tiles;
        tiles += (t.numel + te - 1) / te;
        d.tile_end = tiles;
        descs.push_back(d);
    }
    if (descs.empty()) return STQ_OK;
    if (tiles > 0x7fffffffLL)
        return fail(STQ_ERR_INVALID, "too many tiles in one call (%lld); split the tensor list", (long long)tiles);
    return upload_and_launch(descs.data(), descs.size(), src, dst, grad_dt, log2b, rounding == STQ_ROUND_STOCHASTIC,
                             tiles, reinterpret_cast<unsigned long long *>(prof), seed,
                             reinterpret_cast<hipStream_t>(stream));
}

// stq_multi_tensor_convert_codes: descriptors and tile starts in one ring slot.
int run_convert(const stq_code_convert *items, int n, hipStream_t stream)
{
    g_err.clear();
    if (n < 0 || (n > 0 && !items)) return fail(STQ_ERR_INVALID, "convert_codes: bad tensor list");
    std::vector<mdq::ConvDesc> d;
    d.reserve((size_t)n);
    int64_t tiles = 0;
    for (int i = 0; i < n; ++i) {
        const stq_code_convert &c = items[i];
        if (c.numel < 0) return fail(STQ_ERR_INVALID, "tensor %d: negative numel", i);
        if (c.src_storage < STQ_STORE_P4 || c.src_storage > STQ_STORE_S32 || c.dst_storage < STQ_STORE_P4 ||
            c.dst_storage > STQ_STORE_S32)
            return fail(STQ_ERR_INVALID, "tensor %d: storage must be STQ_STORE_P4 .. STQ_STORE_S32", i);
        if (c.numel == 0) continue;
        if (!c.src_exp_avg || !c.dst_exp_avg || (c.src_storage != STQ_STORE_P4 && !c.src_exp_avg_sq) ||
            (c.dst_storage != STQ_STORE_P4 && !c.dst_exp_avg_sq))
            return fail(STQ_ERR_INVALID, "tensor %d: null code pointer", i);
        mdq::ConvDesc e{};
        e.src_m = c.src_exp_avg;
        e.src_v = c.src_exp_avg_sq;
        e.dst_m = c.dst_exp_avg;
        e.dst_v = c.dst_exp_avg_sq;
        e.numel = c.numel;
        e.tile_begin = tiles;
        e.src = c.src_storage;
        e.dst = c.dst_storage;
        tiles += (c.numel + mdq::CONV_TILE - 1) / mdq::CONV_TILE;
        d.push_back(e);
    }
    if (d.empty()) return STQ_OK;
    if (tiles > 0x7fffffffLL)
        return fail(STQ_ERR_INVALID, "too many tiles in one call (%lld); split the tensor list", (long long)tiles);
    int rc = refuse_capture(stream);
    if (rc != STQ_OK) return rc;
    DevCtx *ctx = nullptr;
    rc = get_ctx(&ctx);
    if (rc != STQ_OK) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const size_t m = d.size();
    const size_t need = m * (sizeof(mdq::ConvDesc) + sizeof(long long));
    Slot *s = nullptr;
    rc = take_slot(ctx, need, &s);
    if (rc != STQ_OK) return rc;
    std::memcpy(s->host, d.data(), m * sizeof(mdq::ConvDesc));
    long long *tb = reinterpret_cast<long long *>(s->host + m * sizeof(mdq::ConvDesc));
    for (size_t i = 0; i < m; ++i) tb[i] = d[i].tile_begin;
    rc = upload(ctx, *s, need, tiles * mdq::CONV_TILE, stream);
    if (rc != STQ_OK) return rc;
    hipError_t e;
    e = mdq::launch_convert(reinterpret_cast<const mdq::ConvDesc *>(s->dev),
                            reinterpret_cast<const long long *>(s->dev + m * sizeof(mdq::ConvDesc)), (int)m,
                            tiles, stream);
    if (e != hipSuccess) return hip_fail(e, "convert launch");
    return release_slot(s, stream);
}

}  // namespace

// ------------------------------------------------- allocation-free entry point
// stq_multi_tensor_mdq_adamw_noalloc keeps its descriptor table (the MdqDesc of
// each tensor with elements, then their int64 tile starts: the layout the step
// kernel reads) in `scratch`, a file-scope device array that every GPU the
// library runs on holds once, until the process ends.  It is staged on the host
// in a static buffer, so a call allocates no device, pinned or heap memory.
// In host code the name `scratch` stands for the host-side shadow; its device
// address on each GPU comes from hipGetSymbolAddress (g_scratch_dev).
constexpr size_t NOALLOC_BYTES = (size_t)STQ_NOALLOC_MAX_TENSORS * (sizeof(mdq::MdqDesc) + sizeof(long long));
static __device__ __align__(256) char scratch[NOALLOC_BYTES];

namespace {

std::mutex g_noalloc_mu;                       // guards the staging buffer, g_scratch_dev and g_noalloc_done
char *g_scratch_dev[64] = {nullptr};           // scratch's device address, per device
hipEvent_t g_noalloc_done[64] = {nullptr};     // recorded behind each call's kernel, per device
alignas(256) char g_noalloc_stage[NOALLOC_BYTES];

int run_noalloc(const stq_tensor *tensors, int n_tensors, int grad_dt, int ea_dt, int easq_dt, int block_size,
                int rounding, uint64_t seed, int64_t *prof, int64_t prof_numel, hipStream_t stream)
{
    g_err.clear();
    if (prof_numel == 0) prof = nullptr;
    int log2b = 0;
    int rc = common_checks(grad_dt, block_size, rounding, prof, prof_numel, &log2b);
    if (rc != STQ_OK) return rc;
    if (n_tensors < 0 || (n_tensors > 0 && !tensors)) return fail(STQ_ERR_INVALID, "bad tensor list");
    if (n_tensors > STQ_NOALLOC_MAX_TENSORS)
        return fail(STQ_ERR_INVALID,
                    "noalloc: %d tensors in one call, more than its fixed descriptor space holds "
                    "(STQ_NOALLOC_MAX_TENSORS = %d); split the list or use stq_multi_tensor_mdq_adamw",
                    n_tensors, STQ_NOALLOC_MAX_TENSORS);
    rc = refuse_capture(stream);
    if (rc != STQ_OK) return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= 64) return fail(STQ_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    MdqDesc *descs = reinterpret_cast<MdqDesc *>(g_noalloc_stage);
    int nd = 0, storage = -1;
    int64_t tiles = 0;
    rc = build_step_descs(tensors, n_tensors, grad_dt, ea_dt, easq_dt, 1 << log2b, descs, &nd, &storage, &tiles);
    if (rc != STQ_OK || nd == 0) return rc;
    if (!g_scratch_dev[dev]) {
        // once per device, with that device current: its copy of the array, and the event
        // that orders each call's table copy after the previous call's kernel
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        hipEvent_t ev = nullptr;
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(e, "hipEventCreateWithFlags(noalloc)");
        g_noalloc_done[dev] = ev;
        g_scratch_dev[dev] = static_cast<char *>(ptr);
    }
    long long *tb = reinterpret_cast<long long *>(g_noalloc_stage + (size_t)nd * sizeof(MdqDesc));
    for (int i = 0; i < nd; ++i) tb[i] = descs[i].tile_begin;
    // Every call on this GPU shares `scratch`: the copy below waits (on the device) for the
    // kernel of the previous call, on whatever stream it ran, so it never overwrites a table
    // a kernel is still reading.  Calls on one stream are in stream order anyway.
    e = hipStreamWaitEvent(stream, g_noalloc_done[dev], 0);
    if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent(noalloc)");
    // The staging buffer is pageable host memory, and HIP performs a copy from pageable
    // memory synchronously (hip_runtime_api.h, hipMemcpyAsync: "If host or dst are not
    // pinned, the memory copy will be performed synchronously"): the buffer has been read
    // when the call returns, so the next call may refill it.
    e = hipMemcpyAsync(g_scratch_dev[dev], g_noalloc_stage, (size_t)nd * (sizeof(MdqDesc) + sizeof(long long)),
                       hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(descriptors -> scratch)");
    const mdq::StepArgs sa{seed, 0.0f, 0.0f, 0u, 0u};   // every descriptor carries its own step constants
    e = launch_step(reinterpret_cast<const MdqDesc *>(g_scratch_dev[dev]), nd, storage, storage, grad_dt, log2b,
                    rounding == STQ_ROUND_STOCHASTIC, tiles, reinterpret_cast<unsigned long long *>(prof), sa,
                    launch_needs_views(descs, (size_t)nd, log2b), stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    e = hipEventRecord(g_noalloc_done[dev], stream);
    return e == hipSuccess ? STQ_OK : hip_fail(e, "hipEventRecord(noalloc)");
}

}  // namespace

extern "C" {

int stq_multi_tensor_mdq_adamw_noalloc(const stq_tensor *tensors, int n_tensors, int grad_dtype, int exp_avg_dtype,
                                       int exp_avg_sq_dtype, int block_size, int rounding, uint64_t seed,
                                       int64_t *profile_cycles, int64_t profile_numel, void *stream)
{
    return run_noalloc(tensors, n_tensors, grad_dtype, exp_avg_dtype, exp_avg_sq_dtype, block_size, rounding, seed,
                       profile_cycles, profile_numel, reinterpret_cast<hipStream_t>(stream));
}

int stq_fused_mdq_adamw(float *p, const void *grad, int grad_dtype, int64_t grad_numel, int64_t numel,
                        void *exp_avg, int exp_avg_dtype, int64_t exp_avg_numel,
                        void *exp_avg_sq, int exp_avg_sq_dtype, int64_t exp_avg_sq_numel,
                        float *scale_m, int64_t scale_m_numel, float *scale_v, int64_t scale_v_numel,
                        float *v_min, int64_t v_min_numel,
                        float beta1, float beta2, float lr, float weight_decay, float eps,
                        int step, int bits, int block_size,
                        int64_t *profile_cycles, int64_t profile_numel,
                        int rounding, uint64_t seed, uint32_t tensor_id, void *stream)
{
    stq_tensor t;
    t.p = p;
    t.grad = grad;
    t.exp_avg = exp_avg;
    t.exp_avg_sq = exp_avg_sq;
    t.scale_m = scale_m;
    t.scale_v = scale_v;
    t.v_min = v_min;
    t.numel = numel;
    t.grad_numel = grad_numel;
    t.exp_avg_numel = exp_avg_numel;
    t.exp_avg_sq_numel = exp_avg_sq_numel;
    t.scale_m_numel = scale_m_numel;
    t.scale_v_numel = scale_v_numel;
    t.v_min_numel = v_min_numel;
    t.beta1 = beta1;
    t.beta2 = beta2;
    t.lr = lr;
    t.weight_decay = weight_decay;
    t.eps = eps;
    t.step = step;
    t.bits = bits;
    t.tensor_id = tensor_id;
    t.elem_offset = 0;
    return run(&t, 1, grad_dtype, exp_avg_dtype, exp_avg_sq_dtype, block_size, rounding, seed,
               profile_cycles, profile_numel, stream);
}

int stq_multi_tensor_mdq_adamw(const stq_tensor *tensors, int n_tensors, int grad_dtype, int exp_avg_dtype,
                               int exp_avg_sq_dtype, int block_size, int rounding, uint64_t seed,
                               int64_t *profile_cycles, int64_t profile_numel, void *stream)
{
    return run(tensors, n_tensors, grad_dtype, exp_avg_dtype, exp_avg_sq_dtype, block_size, rounding, seed,
               profile_cycles, profile_numel, stream);
}

int stq_multi_tensor_mdq_adamw_restore(const stq_tensor *tensors, const stq_code_out *out, int n_tensors,
                                       int grad_dtype, int src_storage, int dst_storage, int block_size,
                                       int rounding, uint64_t seed, int64_t *profile_cycles,
                                       int64_t profile_numel, void *stream)
{
    return run_restore(tensors, out, n_tensors, grad_dtype, src_storage, dst_storage, block_size, rounding, seed,
                       profile_cycles, profile_numel, stream);
}

int stq_multi_tensor_grad_stats(const void *const *grads, const int64_t *numels, int n_tensors,
                                int grad_dtype, float *stats, void *stream)
{
    return run_grad_stats(grads, numels, n_tensors, grad_dtype, stats, reinterpret_cast<hipStream_t>(stream));
}

int stq_multi_tensor_convert_codes(const stq_code_convert *items, int n_tensors, void *stream)
{
    return run_convert(items, n_tensors, reinterpret_cast<hipStream_t>(stream));
}

const char *stq_last_error(void) { return g_err.c_str(); }

int stq_abi_version(void) { return STQ_ABI_VERSION; }

int stq_step_table_uploads(int64_t *count)
{
    g_err.clear();
    if (!count) return fail(STQ_ERR_INVALID, "count must not be NULL");
    DevCtx *ctx = nullptr;
    const int rc = get_ctx(&ctx);
    if (rc != STQ_OK) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    *count = ctx->table_uploads;
    return STQ_OK;
}

int stq_device_math(int which, const float *x, float *y, int64_t n, void *stream)
{
    g_err.clear();
    if (which < 0 || which > 4)
        return fail(STQ_ERR_INVALID,
                    "which must be 0 (exp), 1 (log), 2 (v-code map), 3 (reciprocal) or 4 (stochastic fast v code)");
    if (n < 0 || (n > 0 && (!x || !y)) || (which == 2 && n % 2) || (which == 4 && n % 6))
        return fail(STQ_ERR_INVALID, "bad arrays");
    hipError_t e = mdq::launch_math(which, x, y, n, reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? STQ_OK : hip_fail(e, "math kernel launch");
}

int stq_device_log_approx_error(uint32_t first, uint32_t count, double slope, uint64_t *max_err_bits,
                                void *stream)
{
    g_err.clear();
    if ((uint64_t)first + count > 0x100000000ull) return fail(STQ_ERR_INVALID, "range exceeds 2^32");
    if (count > 0 && !max_err_bits) return fail(STQ_ERR_INVALID, "null output");
    if (!(slope >= 0.0)) return fail(STQ_ERR_INVALID, "slope must be >= 0");
    hipError_t e = mdq::launch_log_approx_err(first, count, slope,
                                              reinterpret_cast<unsigned long long *>(max_err_bits),
                                              reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? STQ_OK : hip_fail(e, "log error kernel launch");
}

int stq_device_hw_ulp_error(int which, uint32_t first, uint32_t count, uint32_t *max_ulps, void *stream)
{
    g_err.clear();
    if (which != 0 && which != 1) return fail(STQ_ERR_INVALID, "which must be 0 (sqrt) or 1 (reciprocal)");
    if ((uint64_t)first + count > 0x100000000ull) return fail(STQ_ERR_INVALID, "range exceeds 2^32");
    if (count > 0 && !max_ulps) return fail(STQ_ERR_INVALID, "null output");
    hipError_t e = mdq::launch_hw_ulp_err(which, first, count, max_ulps, reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? STQ_OK : hip_fail(e, "hardware ulp error kernel launch");
}

int stq_device_math_digests(int which, uint32_t first, uint32_t count, uint32_t chunk, uint64_t *digests,
                            void *stream)
{
    g_err.clear();
    if (which != 0 && which != 1 && which != 3)
        return fail(STQ_ERR_INVALID, "which must be 0 (exp), 1 (log) or 3 (reciprocal)");
    if (chunk == 0 || chunk % 64 != 0) return fail(STQ_ERR_INVALID, "chunk must be a positive multiple of 64");
    if ((uint64_t)first + count > 0x100000000ull) return fail(STQ_ERR_INVALID, "range exceeds 2^32");
    if (count > 0 && !digests) return fail(STQ_ERR_INVALID, "null digests");
    hipError_t e = mdq::launch_math_digests(which, first, count, chunk,
                                            reinterpret_cast<unsigned long long *>(digests),
                                            reinterpret_cast<hipStream_t>(stream));
    return e == hipSuccess ? STQ_OK : hip_fail(e, "math digest kernel launch");
}

void stq_host_math(int which, const float *x, float *y, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) y[i] = which == 0 ? mdq::mdq_expf(x[i]) : mdq::mdq_logf(x[i]);
}

void stq_host_round_half_away(const float *u, const float *d, float *out, int64_t n, int inv_ulps)
{
    for (int64_t i = 0; i < n; ++i) {
        const float inv = mdq::bits_f(mdq::f_bits(1.0f / d[i]) + (uint32_t)inv_ulps);
        out[i] = mdq::mdq_round_half_away(u[i], d[i], mdq::mdq_inv_lo(inv), 0.5f * d[i]);
    }
}

void stq_host_div_code_range(const float *x, float *out, int64_t n, int bits)
{
    const float D = (float)(std::ldexp(1.0, bits) - 1.0);
    const float y = 1.0f / D;
    for (int64_t i = 0; i < n; ++i) out[i] = mdq::mdq_div_code_range(x[i], D, y);
}

void stq_host_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4])
{
    mdq::U4 r = mdq::mdq_philox4x32_10(mdq::U4{ctr[0], ctr[1], ctr[2], ctr[3]}, key[0], key[1]);
    out[0] = r.x; out[1] = r.y; out[2] = r.z; out[3] = r.w;
}

}  // extern "C"
