// capi_driver.cpp -- a C++ caller of the C ABI (include/stquant_hip.h) with no
// torch and no Python: device buffers from hipMalloc, one stream from
// hipStreamCreate, steps through stq_multi_tensor_mdq_adamw and
// stq_fused_mdq_adamw, each checked against the CPU oracle (oracle/, test
// infrastructure) on the same inputs: codes and block scales bit-exact, params
// within 1e-6 of the step's scale (|dp| <= 1e-6 (|p| + |update|)).
//
// Built by __graft_entry__.build() into tests/capi_driver/capi_driver; run by
// tests/test_gpu_capi_driver.py.  Prints one line per checked step and "OK" at
// the end; exits nonzero on the first mismatch or error.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/stquant_hip.h"
#include "../../oracle/mdq_oracle.h"

#define HIP_OK(x)                                                                   \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,          \
                         hipGetErrorString(e_));                                    \
            std::exit(2);                                                           \
        }                                                                           \
    } while (0)

namespace {

uint16_t f2bf(float x)   // round to nearest even (finite inputs)
{
    uint32_t b;
    std::memcpy(&b, &x, 4);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

template <class T>
T *dev_copy(const std::vector<T> &h)
{
    T *d = nullptr;
    HIP_OK(hipMalloc((void **)&d, h.size() * sizeof(T) + 16));
    if (!h.empty()) HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <class T>
std::vector<T> host_copy(const T *d, size_t n)
{
    std::vector<T> h(n);
    if (n) HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

// One tensor: the oracle's host state and the device copy the library steps.
struct Tensor {
    int64_t n, nb;
    int storage;                 // MDQO_STORE_* (== the library's storage classes)
    size_t cb;                   // bytes per code
    std::vector<float> p;
    std::vector<uint8_t> cm, cv;     // codes as raw bytes
    std::vector<float> sm, sv, vm;
    float *dp;
    void *dg;
    uint8_t *dcm, *dcv;
    float *dsm, *dsv, *dvm;

    Tensor(int64_t n_, int B, int storage_, std::mt19937 &rng) : n(n_), nb((n_ + B - 1) / B), storage(storage_)
    {
        cb = storage == MDQO_STORE_S16 ? 2 : storage == MDQO_STORE_S32 ? 4 : 1;
        std::normal_distribution<float> nd(0.0f, 0.02f);
        p.resize(n);
        for (auto &x : p) x = nd(rng);
        cm.assign(n * cb, 0);
        if (storage == MDQO_STORE_P4) std::memset(cm.data(), 0x08, n);   // m code 0, v code 0
        else cv.assign(n * cb, 0);
        sm.assign(nb, 0.0f);
        sv.assign(nb, 0.0f);
        vm.assign(nb, -20.0f);
        dp = dev_copy(p);
        dg = nullptr;
        dcm = dev_copy(cm);
        dcv = cv.empty() ? nullptr : dev_copy(cv);
        dsm = dev_copy(sm);
        dsv = dev_copy(sv);
        dvm = dev_copy(vm);
    }
};

bool same_bytes(const void *a, const void *b, size_t n) { return n == 0 || std::memcmp(a, b, n) == 0; }

int check(const Tensor &t, const std::vector<float> &p_prev, const char *tag)
{
    auto cm = host_copy(t.dcm, t.cm.size());
    auto sm = host_copy(t.dsm, t.nb), sv = host_copy(t.dsv, t.nb), vm = host_copy(t.dvm, t.nb);
    auto p = host_copy(t.dp, (size_t)t.n);
    if (!same_bytes(cm.data(), t.cm.data(), cm.size())) return std::printf("%s: exp_avg codes differ\n", tag), 1;
    if (!t.cv.empty()) {
        auto cv = host_copy(t.dcv, t.cv.size());
        if (!same_bytes(cv.data(), t.cv.data(), cv.size())) return std::printf("%s: exp_avg_sq codes differ\n", tag), 1;
    }
    if (!same_bytes(sm.data(), t.sm.data(), 4 * sm.size()) || !same_bytes(sv.data(), t.sv.data(), 4 * sv.size()) ||
        !same_bytes(vm.data(), t.vm.data(), 4 * vm.size()))
        return std::printf("%s: block scales differ\n", tag), 1;
    for (int64_t i = 0; i < t.n; ++i) {
        const double ref = t.p[i], upd = std::fabs(ref - (double)p_prev[i]);
        if (std::fabs((double)p[i] - ref) > 1e-6 * (std::fabs(ref) + upd) + 1e-30)
            return std::printf("%s: param %lld got %.9g want %.9g\n", tag, (long long)i, p[i], t.p[i]), 1;
    }
    return 0;
}

struct HP {
    float beta1 = 0.9f, beta2 = 0.999f, lr = 1e-3f, wd = 0.01f, eps = 1e-8f;
};

// Steps of one multi-tensor launch each over `ts` (grads fp32 or bf16), the oracle alongside.
int run_multi(std::vector<Tensor> &ts, int B, int bits, int grad_bf16, int rounding, uint64_t seed, int steps,
              std::mt19937 &rng, hipStream_t stream, const char *name)
{
    const HP hp;
    std::normal_distribution<float> gd(0.0f, 1e-3f);
    for (int step = 1; step <= steps; ++step) {
        std::vector<stq_tensor> rows(ts.size());
        std::vector<std::vector<float>> prev(ts.size());
        std::vector<std::vector<uint16_t>> g16(ts.size());
        std::vector<std::vector<float>> g32(ts.size());
        for (size_t k = 0; k < ts.size(); ++k) {
            Tensor &t = ts[k];
            prev[k] = t.p;
            mdqo_tensor o{};
            if (grad_bf16) {
                g16[k].resize(t.n);
                for (auto &x : g16[k]) x = f2bf(gd(rng));
                if (t.dg) HIP_OK(hipFree(t.dg));
                t.dg = dev_copy(g16[k]);
                o.grad = g16[k].data();
            } else {
                g32[k].resize(t.n);
                for (auto &x : g32[k]) x = gd(rng);
                if (t.dg) HIP_OK(hipFree(t.dg));
                t.dg = dev_copy(g32[k]);
                o.grad = g32[k].data();
            }
            o.p = t.p.data();
            o.code_m = t.cm.data();
            o.code_v = t.cv.empty() ? nullptr : t.cv.data();
            o.scale_m = t.sm.data();
            o.scale_v = t.sv.data();
            o.v_min = t.vm.data();
            o.numel = t.n;
            o.storage = t.storage;
            o.grad_dtype = grad_bf16 ? MDQO_GRAD_BF16 : MDQO_GRAD_F32;
            o.block_size = B;
            o.bits = bits;
            o.step = step;
            o.tensor_id = (uint32_t)k;
            o.elem_offset = 0;
            const mdqo_hparams h{hp.beta1, hp.beta2, hp.lr, hp.wd, hp.eps, rounding, seed, 0};
            if (mdq_oracle_step(&o, &h) != 0) return std::printf("%s: oracle rejected tensor %zu\n", name, k), 1;

            stq_tensor &r = rows[k];
            std::memset(&r, 0, sizeof r);
            r.p = t.dp;
            r.grad = t.dg;
            r.exp_avg = t.dcm;
            r.exp_avg_sq = t.dcv;
            r.scale_m = t.dsm;
            r.scale_v = t.dsv;
            r.v_min = t.dvm;
            r.numel = r.grad_numel = r.exp_avg_numel = t.n;
            r.exp_avg_sq_numel = t.cv.empty() ? 0 : t.n;
            r.scale_m_numel = r.scale_v_numel = r.v_min_numel = t.nb;
            r.beta1 = hp.beta1;
            r.beta2 = hp.beta2;
            r.lr = hp.lr;
            r.weight_decay = hp.wd;
            r.eps = hp.eps;
            r.step = step;
            r.bits = bits;
            r.tensor_id = (uint32_t)k;
        }
        const int st = ts[0].storage;
        const int ea = st == MDQO_STORE_P4 ? STQ_BYTE : st == MDQO_STORE_S8 ? STQ_CHAR : st == MDQO_STORE_S16 ? STQ_SHORT : STQ_INT;
        const int easq = st == MDQO_STORE_P4 ? STQ_BYTE : st == MDQO_STORE_S8 ? STQ_BYTE : st == MDQO_STORE_S16 ? STQ_UINT16 : STQ_UINT32;
        const int rc = stq_multi_tensor_mdq_adamw(rows.data(), (int)rows.size(), grad_bf16 ? STQ_BFLOAT16 : STQ_FLOAT, ea, easq,
                                                  B, rounding, seed, nullptr, 0, stream);
        if (rc != STQ_OK) return std::printf("%s: step %d: %s\n", name, step, stq_last_error()), 1;
        HIP_OK(hipStreamSynchronize(stream));
        for (size_t k = 0; k < ts.size(); ++k) {
            char tag[128];
            std::snprintf(tag, sizeof tag, "%s step %d tensor %zu (n=%lld)", name, step, k, (long long)ts[k].n);
            if (check(ts[k], prev[k], tag)) return 1;
            // the next step starts from the oracle's params, so each step is judged alone
            HIP_OK(hipMemcpy(ts[k].dp, ts[k].p.data(), ts[k].p.size() * sizeof(float), hipMemcpyHostToDevice));
        }
        std::printf("%s: step %d of %zu tensors matches the oracle\n", name, step, ts.size());
    }
    return 0;
}

}  // namespace

int main()
{
    std::printf("C ABI version %d\n", stq_abi_version());
    if (stq_abi_version() != STQ_ABI_VERSION) return std::printf("ABI version mismatch\n"), 1;
    hipStream_t stream;
    HIP_OK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    std::mt19937 rng(2024);

    // packed 4-bit codes, fp32 grads, B = 128, nearest rounding: ragged sizes
    {
        std::vector<Tensor> ts;
        for (int64_t n : {1, 127, 4096, 70001, 262149}) ts.emplace_back(n, 128, MDQO_STORE_P4, rng);
        if (run_multi(ts, 128, 4, 0, STQ_ROUND_NEAREST, 0, 3, rng, stream, "packed4/f32/B128/nearest")) return 1;
    }
    // int16 / uint16 codes at 12 bits, bf16 grads, B = 64, stochastic rounding
    {
        std::vector<Tensor> ts;
        for (int64_t n : {64, 1000, 33333}) ts.emplace_back(n, 64, MDQO_STORE_S16, rng);
        if (run_multi(ts, 64, 12, 1, STQ_ROUND_STOCHASTIC, 0x1234abcdULL, 2, rng, stream, "int16/bf16/B64/stochastic"))
            return 1;
    }
    // int8 / uint8 codes, one tensor through the reference's single-tensor entry point
    {
        std::vector<Tensor> ts;
        ts.emplace_back(5000, 256, MDQO_STORE_S8, rng);
        Tensor &t = ts[0];
        std::normal_distribution<float> gd(0.0f, 1e-3f);
        std::vector<float> g(t.n);
        for (auto &x : g) x = gd(rng);
        t.dg = dev_copy(g);
        const std::vector<float> prev = t.p;
        const HP hp;
        mdqo_tensor o{t.p.data(), g.data(), t.cm.data(), t.cv.data(), t.sm.data(), t.sv.data(), t.vm.data(), t.n,
                      MDQO_STORE_S8, MDQO_GRAD_F32, 256, 8, 1, 0, 0};
        const mdqo_hparams h{hp.beta1, hp.beta2, hp.lr, hp.wd, hp.eps, MDQO_ROUND_NEAREST, 0, 0};
        if (mdq_oracle_step(&o, &h) != 0) return std::printf("oracle rejected the int8 tensor\n"), 1;
        const int rc = stq_fused_mdq_adamw(t.dp, t.dg, STQ_FLOAT, t.n, t.n, t.dcm, STQ_CHAR, t.n, t.dcv, STQ_BYTE, t.n,
                                           t.dsm, t.nb, t.dsv, t.nb, t.dvm, t.nb, hp.beta1, hp.beta2, hp.lr, hp.wd,
                                           hp.eps, 1, 8, 256, nullptr, 0, STQ_ROUND_NEAREST, 0, 0, stream);
        if (rc != STQ_OK) return std::printf("stq_fused_mdq_adamw: %s\n", stq_last_error()), 1;
        HIP_OK(hipStreamSynchronize(stream));
        if (check(t, prev, "int8/f32/B256 single tensor")) return 1;
        std::printf("int8/f32/B256: stq_fused_mdq_adamw matches the oracle\n");
        // an argument error is reported, nothing launched
        const int bad = stq_fused_mdq_adamw(t.dp, t.dg, STQ_FLOAT, t.n, t.n, t.dcm, STQ_CHAR, t.n, t.dcv, STQ_BYTE, t.n,
                                            t.dsm, t.nb, t.dsv, t.nb, t.dvm, t.nb, hp.beta1, hp.beta2, hp.lr, hp.wd,
                                            hp.eps, 0, 8, 256, nullptr, 0, STQ_ROUND_NEAREST, 0, 0, stream);
        if (bad != STQ_ERR_INVALID || !std::strstr(stq_last_error(), "step must be >= 1"))
            return std::printf("step 0 was not rejected: %d %s\n", bad, stq_last_error()), 1;
    }
    int64_t uploads = -1;
    if (stq_step_table_uploads(&uploads) != STQ_OK || uploads < 1) return std::printf("upload count %lld\n", (long long)uploads), 1;
    HIP_OK(hipStreamDestroy(stream));
    std::printf("OK\n");
    return 0;
}
