// kd_optim.hip - optimizer steps for gfx950: one launch per parameter tensor, or one launch per
// kManyTensors tensors for Adam.
//
// kael's optimizers (reference src/optim/optimizer.cpp:60-80 SGD, :93-120 Adam / AdamW) update
// a parameter through a chain of whole-tensor element ops: on the device Adam is 14 element
// launches and 7 scalar fills per tensor, SGD 3. Here the same chain runs per element in
// registers. Every step is rounded to the element type as kael's separate op rounds it (the
// *_sep helpers of kd_internal.h, so nothing is contracted into an FMA), and every scalar operand is
// the host-computed double converted to the element type, as kael's fill of a 0-d scalar tensor
// converts it (reference src/factory.cpp:68-79, include/kael/scalar.h:23-25). The bias
// corrections 1 - beta^step are computed on the host with std::pow, as kael computes them. The
// result therefore equals kael's composed device path bit for bit.
//
// Layout: p, g and the moments are contiguous, 16-byte aligned for the vector path (4 floats or
// 2 doubles per lane), scalar tail otherwise; HBM-bound (Adam moves 28 bytes per f32 element,
// SGD 12). Tensors of 32 MiB or more stream with nontemporal loads and stores: they are touched
// once per step and would only evict other data from the caches.
#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "kd_internal.h"

namespace kd {

namespace {

constexpr int kThreads = 256;

template <typename T> __device__ __forceinline__ T mul_rn(T a, T b) { return mul_sep(a, b); }
template <typename T> __device__ __forceinline__ T add_rn(T a, T b) { return add_sep(a, b); }
template <typename T> __device__ __forceinline__ T sub_rn(T a, T b) { return sub_sep(a, b); }
template <typename T> __device__ __forceinline__ T div_rn(T a, T b) { return div_sep(a, b); }
// std::sqrt is the correctly rounded square root here (v_sqrt_f32 plus a refinement step); the
// __fsqrt_rn intrinsic compiles to the bare v_sqrt_f32, which is not correctly rounded.
template <typename T> __device__ __forceinline__ T sqrt_rn(T a) { return std::sqrt(a); }

// Scalar operands in the element type, in the order kael uses them.
template <typename T> struct AdamScalars {
    T weight_decay;  // coupled: g + p * weight_decay
    T decay;         // decoupled: p * (1 - lr * weight_decay)
    T beta1, one_minus_beta1, beta2, one_minus_beta2;
    T first_correction, second_correction, epsilon, learning_rate;
    int mode;  // 0 no weight decay, 1 coupled (Adam), 2 decoupled (AdamW)
};

// One element of AdamBase::update (reference src/optim/optimizer.cpp:101-118).
template <typename T>
__device__ __forceinline__ void adam_element(T& p, T g, T& m, T& v, const AdamScalars<T>& s) {
    if (s.mode == 1) g = add_rn(g, mul_rn(p, s.weight_decay));   // gradient + parameter * wd
    else if (s.mode == 2) p = mul_rn(p, s.decay);                // parameter.mul_(1 - lr * wd)
    m = add_rn(mul_rn(m, s.beta1), mul_rn(g, s.one_minus_beta1));            // first.mul_(b1).add_(g * (1 - b1))
    v = add_rn(mul_rn(v, s.beta2), mul_rn(mul_rn(g, g), s.one_minus_beta2));  // second.mul_(b2).add_(g * g * (1 - b2))
    const T corrected_first = div_rn(m, s.first_correction);
    const T corrected_second = div_rn(v, s.second_correction);
    const T denominator = add_rn(sqrt_rn(corrected_second), s.epsilon);
    p = sub_rn(p, mul_rn(div_rn(corrected_first, denominator), s.learning_rate));
}

template <typename T> struct alignas(16) Vec {
    T v[16 / sizeof(T)];
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT, typename T> __device__ __forceinline__ Vec<T> ld(const Vec<T>* p) {
    if constexpr (!NT) {
        return *p;
    } else {
        const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        Vec<T> out;
        __builtin_memcpy(&out, &r, 16);
        return out;
    }
}

template <bool NT, typename T> __device__ __forceinline__ void st(Vec<T>* p, const Vec<T>& x) {
    if constexpr (!NT) {
        *p = x;
    } else {
        u32x4 r;
        __builtin_memcpy(&r, &x, 16);
        __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
    }
}

template <typename T, bool NT>
__global__ __launch_bounds__(kThreads) void adam_kernel(T* __restrict__ p, const T* __restrict__ g,
                                                        T* __restrict__ m, T* __restrict__ v, int64_t count,
                                                        bool vec, AdamScalars<T> s) {
    constexpr int V = 16 / sizeof(T);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    int64_t first_scalar = 0;
    if (vec) {
        const int64_t vectors = count / V;
        Vec<T>* pv = reinterpret_cast<Vec<T>*>(p);
        const Vec<T>* gv = reinterpret_cast<const Vec<T>*>(g);
        Vec<T>* mv = reinterpret_cast<Vec<T>*>(m);
        Vec<T>* vv = reinterpret_cast<Vec<T>*>(v);
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < vectors; i += stride) {
            Vec<T> a = ld<NT>(pv + i), b = ld<NT>(gv + i), c = ld<NT>(mv + i), d = ld<NT>(vv + i);
#pragma unroll
            for (int e = 0; e < V; ++e) adam_element(a.v[e], b.v[e], c.v[e], d.v[e], s);
            st<NT>(pv + i, a);
            st<NT>(mv + i, c);
            st<NT>(vv + i, d);
        }
        first_scalar = vectors * V;
    }
    for (int64_t i = first_scalar + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride)
        adam_element(p[i], g[i], m[i], v[i], s);
}

// ---- Adam over many tensors in one launch ----------------------------------------------------
//
// kael's AdamBase::update visits every parameter in turn; for a model of many small tensors the
// per-tensor launches, not the bytes, set the time. A table of up to kManyTensors tensors rides in
// the kernel arguments (no upload, nothing allocated); each tensor owns a contiguous run of
// workgroups, each workgroup kManyUnroll vectors per lane of one tensor. The element chain and
// scalars are those of adam_kernel, so the results are the same bits.
constexpr int kManyTensors = 32;
constexpr int kManyUnroll = 2;

template <typename T> struct AdamTable {
    T* p[kManyTensors];
    const T* g[kManyTensors];
    T* m[kManyTensors];
    T* v[kManyTensors];
    int64_t count[kManyTensors];
    uint32_t block_end[kManyTensors];  // running total of the tensors' workgroups
    uint32_t flags[kManyTensors];      // bit 0: 16-byte aligned (vector path), bit 1: nontemporal
    T first_correction[kManyTensors], second_correction[kManyTensors];
    int n;
};

template <bool NT, typename T>
__device__ __forceinline__ void adam_block(T* __restrict__ p, const T* __restrict__ g, T* __restrict__ m,
                                           T* __restrict__ v, int64_t count, bool vec, int64_t block,
                                           const AdamScalars<T>& s) {
    constexpr int V = 16 / sizeof(T);
    constexpr int64_t kPerBlock = int64_t{kThreads} * V * kManyUnroll;
    const int64_t begin = block * kPerBlock;
    if (vec) {
        const int64_t vectors = count / V;
        Vec<T>* pv = reinterpret_cast<Vec<T>*>(p);
        const Vec<T>* gv = reinterpret_cast<const Vec<T>*>(g);
        Vec<T>* mv = reinterpret_cast<Vec<T>*>(m);
        Vec<T>* vv = reinterpret_cast<Vec<T>*>(v);
#pragma unroll
        for (int u = 0; u < kManyUnroll; ++u) {
            const int64_t i = begin / V + u * kThreads + threadIdx.x;
            if (i < vectors) {
                Vec<T> a = ld<NT>(pv + i), b = ld<NT>(gv + i), c = ld<NT>(mv + i), d = ld<NT>(vv + i);
#pragma unroll
                for (int e = 0; e < V; ++e) adam_element(a.v[e], b.v[e], c.v[e], d.v[e], s);
                st<NT>(pv + i, a);
                st<NT>(mv + i, c);
                st<NT>(vv + i, d);
            }
        }
        // the last workgroup of the tensor takes the elements after the last whole vector
        const int64_t tail = vectors * V + threadIdx.x;
        if (begin + kPerBlock >= count && tail < count) adam_element(p[tail], g[tail], m[tail], v[tail], s);
        return;
    }
    for (int u = 0; u < V * kManyUnroll; ++u) {
        const int64_t i = begin + u * kThreads + threadIdx.x;
        if (i < count) adam_element(p[i], g[i], m[i], v[i], s);
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void adam_many_kernel(const AdamTable<T> table,
                                                             const AdamScalars<T> common) {
    int t = 0;
    while (t + 1 < table.n && blockIdx.x >= table.block_end[t]) ++t;
    const int64_t block = blockIdx.x - (t == 0 ? 0u : table.block_end[t - 1]);
    AdamScalars<T> s = common;
    s.first_correction = table.first_correction[t];
    s.second_correction = table.second_correction[t];
    const uint32_t flags = table.flags[t];
    if (flags & 2u)
        adam_block<true>(table.p[t], table.g[t], table.m[t], table.v[t], table.count[t], flags & 1u, block, s);
    else
        adam_block<false>(table.p[t], table.g[t], table.m[t], table.v[t], table.count[t], flags & 1u, block, s);
}

// One element of SGD::update without momentum (reference src/optim/optimizer.cpp:60-80):
// gradient = g (+ p * weight_decay); parameter.sub_(gradient * lr).
template <typename T>
__device__ __forceinline__ T sgd_element(T p, T g, T learning_rate, T weight_decay, bool decay) {
    if (decay) g = add_rn(g, mul_rn(p, weight_decay));
    return sub_rn(p, mul_rn(g, learning_rate));
}

template <typename T, bool NT>
__global__ __launch_bounds__(kThreads) void sgd_kernel(T* __restrict__ p, const T* __restrict__ g, int64_t count,
                                                       bool vec, T learning_rate, T weight_decay, bool decay) {
    constexpr int V = 16 / sizeof(T);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    int64_t first_scalar = 0;
    if (vec) {
        const int64_t vectors = count / V;
        Vec<T>* pv = reinterpret_cast<Vec<T>*>(p);
        const Vec<T>* gv = reinterpret_cast<const Vec<T>*>(g);
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < vectors; i += stride) {
            Vec<T> a = ld<NT>(pv + i);
            const Vec<T> b = ld<NT>(gv + i);
#pragma unroll
            for (int e = 0; e < V; ++e) a.v[e] = sgd_element(a.v[e], b.v[e], learning_rate, weight_decay, decay);
            st<NT>(pv + i, a);
        }
        first_scalar = vectors * V;
    }
    for (int64_t i = first_scalar + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride)
        p[i] = sgd_element(p[i], g[i], learning_rate, weight_decay, decay);
}

// Streaming threshold of the nontemporal variants (bytes of the parameter tensor).
constexpr int64_t kStreamBytes = int64_t{32} << 20;

bool aligned16(const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }

// One work item per thread up to 2^20 workgroups (the grid-stride loops cover larger tensors).
dim3 grid_for(int64_t work) {
    const int64_t blocks = (work + kThreads - 1) / kThreads;
    return dim3(static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>(blocks, int64_t{1} << 20))));
}

// The bias corrections of AdamBase::update (reference src/optim/optimizer.cpp:100-102), with the
// host's std::pow as kael computes them, converted to the element type.
template <typename T> void bias_corrections(double beta1, double beta2, int64_t step, T& first, T& second) {
    const double step_d = static_cast<double>(step);
    first = static_cast<T>(1.0 - std::pow(beta1, step_d));
    second = static_cast<T>(1.0 - std::pow(beta2, step_d));
}

template <typename T>
AdamScalars<T> adam_scalars(double learning_rate, double beta1, double beta2, double epsilon, double weight_decay,
                            int decoupled) {
    AdamScalars<T> s;
    s.mode = weight_decay > 0.0 ? (decoupled ? 2 : 1) : 0;
    s.weight_decay = static_cast<T>(weight_decay);
    s.decay = static_cast<T>(1.0 - learning_rate * weight_decay);
    s.beta1 = static_cast<T>(beta1);
    s.one_minus_beta1 = static_cast<T>(1.0 - beta1);
    s.beta2 = static_cast<T>(beta2);
    s.one_minus_beta2 = static_cast<T>(1.0 - beta2);
    s.first_correction = s.second_correction = T(1);
    s.epsilon = static_cast<T>(epsilon);
    s.learning_rate = static_cast<T>(learning_rate);
    return s;
}

template <typename T>
int adam_typed(void* param, const void* grad, void* first, void* second, int64_t count, double learning_rate,
               double beta1, double beta2, double epsilon, double weight_decay, int decoupled, int64_t step) {
    AdamScalars<T> s = adam_scalars<T>(learning_rate, beta1, beta2, epsilon, weight_decay, decoupled);
    bias_corrections(beta1, beta2, step, s.first_correction, s.second_correction);
    const bool vec = aligned16(param) && aligned16(grad) && aligned16(first) && aligned16(second);
    constexpr int V = 16 / sizeof(T);
    const dim3 grid = grid_for(vec ? (count + V - 1) / V : count);
    if (count * static_cast<int64_t>(sizeof(T)) >= kStreamBytes)
        hipLaunchKernelGGL((adam_kernel<T, true>), grid, dim3(kThreads), 0, stream(), static_cast<T*>(param),
                           static_cast<const T*>(grad), static_cast<T*>(first), static_cast<T*>(second), count, vec, s);
    else
        hipLaunchKernelGGL((adam_kernel<T, false>), grid, dim3(kThreads), 0, stream(), static_cast<T*>(param),
                           static_cast<const T*>(grad), static_cast<T*>(first), static_cast<T*>(second), count, vec, s);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <typename T>
int adam_many_typed(const kd_adam_tensor* tensors, int64_t n, double learning_rate, double beta1, double beta2,
                    double epsilon, double weight_decay, int decoupled) {
    constexpr int V = 16 / sizeof(T);
    constexpr int64_t kPerBlock = int64_t{kThreads} * V * kManyUnroll;
    const AdamScalars<T> common = adam_scalars<T>(learning_rate, beta1, beta2, epsilon, weight_decay, decoupled);
    AdamTable<T> table{};
    uint32_t blocks = 0;
    auto launch = [&]() -> int {
        if (table.n == 0) return KD_OK;
        hipLaunchKernelGGL((adam_many_kernel<T>), dim3(blocks), dim3(kThreads), 0, stream(), table, common);
        KD_LAUNCH_CHECK();
        table = AdamTable<T>{};
        blocks = 0;
        return KD_OK;
    };
    for (int64_t i = 0; i < n; ++i) {
        const kd_adam_tensor& x = tensors[i];
        if (x.count == 0) continue;
        const int64_t own = (x.count + kPerBlock - 1) / kPerBlock;
        if (table.n == kManyTensors || int64_t{blocks} + own > (int64_t{1} << 31) - 1)
            if (int rc = launch()) return rc;
        const int k = table.n++;
        table.p[k] = static_cast<T*>(x.param);
        table.g[k] = static_cast<const T*>(x.grad);
        table.m[k] = static_cast<T*>(x.first);
        table.v[k] = static_cast<T*>(x.second);
        table.count[k] = x.count;
        blocks += static_cast<uint32_t>(own);
        table.block_end[k] = blocks;
        const bool vec = aligned16(x.param) && aligned16(x.grad) && aligned16(x.first) && aligned16(x.second);
        table.flags[k] = (vec ? 1u : 0u) | (x.count * static_cast<int64_t>(sizeof(T)) >= kStreamBytes ? 2u : 0u);
        bias_corrections(beta1, beta2, x.step, table.first_correction[k], table.second_correction[k]);
    }
    return launch();
}

// Tensors updated by one kd_adam_step_many call may not share memory that one of them writes (the
// sequential calls it stands for would see each other's writes; one launch would race).
int check_adam_overlap(const kd_adam_tensor* tensors, int64_t n, size_t element) {
    struct Span {
        uintptr_t begin, end;
        int64_t tensor;
        bool written;
    };
    std::vector<Span> spans;
    spans.reserve(static_cast<size_t>(n) * 4);
    for (int64_t i = 0; i < n; ++i) {
        const kd_adam_tensor& x = tensors[i];
        if (x.count == 0) continue;
        const uintptr_t bytes = static_cast<uintptr_t>(x.count) * element;
        for (const void* ptr : {static_cast<const void*>(x.param), static_cast<const void*>(x.first), static_cast<const void*>(x.second)})
            spans.push_back({reinterpret_cast<uintptr_t>(ptr), reinterpret_cast<uintptr_t>(ptr) + bytes, i, true});
        spans.push_back({reinterpret_cast<uintptr_t>(x.grad), reinterpret_cast<uintptr_t>(x.grad) + bytes, i, false});
    }
    std::sort(spans.begin(), spans.end(), [](const Span& a, const Span& b) { return a.begin < b.begin; });
    std::vector<Span> open;
    for (const Span& s : spans) {
        open.erase(std::remove_if(open.begin(), open.end(), [&](const Span& o) { return o.end <= s.begin; }), open.end());
        for (const Span& o : open)
            if (o.tensor != s.tensor && (o.written || s.written))
                return fail(KD_E_INVALID, "kd_adam_step_many: tensors " + std::to_string(o.tensor) + " and " +
                                              std::to_string(s.tensor) + " overlap");
        open.push_back(s);
    }
    return KD_OK;
}

template <typename T>
int sgd_typed(void* param, const void* grad, int64_t count, double learning_rate, double weight_decay) {
    const bool vec = aligned16(param) && aligned16(grad);
    constexpr int V = 16 / sizeof(T);
    const dim3 grid = grid_for(vec ? (count + V - 1) / V : count);
    const T lr = static_cast<T>(learning_rate), wd = static_cast<T>(weight_decay);
    if (count * static_cast<int64_t>(sizeof(T)) >= kStreamBytes)
        hipLaunchKernelGGL((sgd_kernel<T, true>), grid, dim3(kThreads), 0, stream(), static_cast<T*>(param),
                           static_cast<const T*>(grad), count, vec, lr, wd, weight_decay > 0.0);
    else
        hipLaunchKernelGGL((sgd_kernel<T, false>), grid, dim3(kThreads), 0, stream(), static_cast<T*>(param),
                           static_cast<const T*>(grad), count, vec, lr, wd, weight_decay > 0.0);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

extern "C" int kd_adam_step(int dtype, void* param, const void* grad, void* first, void* second, int64_t count,
                            double learning_rate, double beta1, double beta2, double epsilon, double weight_decay,
                            int decoupled, int64_t step) {
    if (count < 0 || step < 1) return fail(KD_E_INVALID, "kd_adam_step: negative count or step < 1");
    if (dtype != KD_F32 && dtype != KD_F64) return fail(KD_E_INVALID, "kd_adam_step: dtype must be f32 or f64");
    if (count == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    return dtype == KD_F32 ? adam_typed<float>(param, grad, first, second, count, learning_rate, beta1, beta2, epsilon,
                                               weight_decay, decoupled, step)
                           : adam_typed<double>(param, grad, first, second, count, learning_rate, beta1, beta2,
                                                epsilon, weight_decay, decoupled, step);
}

extern "C" int kd_adam_step_many(int dtype, const kd_adam_tensor* tensors, int64_t n, double learning_rate,
                                 double beta1, double beta2, double epsilon, double weight_decay, int decoupled) {
    if (n < 0 || (n > 0 && tensors == nullptr)) return fail(KD_E_INVALID, "kd_adam_step_many: negative count or no table");
    if (dtype != KD_F32 && dtype != KD_F64) return fail(KD_E_INVALID, "kd_adam_step_many: dtype must be f32 or f64");
    bool work = false;
    for (int64_t i = 0; i < n; ++i) {
        if (tensors[i].count < 0 || tensors[i].step < 1)
            return fail(KD_E_INVALID, "kd_adam_step_many: tensor " + std::to_string(i) + " has a negative count or step < 1");
        work = work || tensors[i].count > 0;
    }
    if (!work) return KD_OK;
    if (int rc = check_adam_overlap(tensors, n, dtype == KD_F32 ? sizeof(float) : sizeof(double))) return rc;
    if (int rc = ensure_device()) return rc;
    return dtype == KD_F32 ? adam_many_typed<float>(tensors, n, learning_rate, beta1, beta2, epsilon, weight_decay, decoupled)
                           : adam_many_typed<double>(tensors, n, learning_rate, beta1, beta2, epsilon, weight_decay,
                                                     decoupled);
}

extern "C" int kd_sgd_step(int dtype, void* param, const void* grad, int64_t count, double learning_rate,
                           double weight_decay) {
    if (count < 0) return fail(KD_E_INVALID, "kd_sgd_step: negative count");
    if (dtype != KD_F32 && dtype != KD_F64) return fail(KD_E_INVALID, "kd_sgd_step: dtype must be f32 or f64");
    if (count == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    return dtype == KD_F32 ? sgd_typed<float>(param, grad, count, learning_rate, weight_decay)
                           : sgd_typed<double>(param, grad, count, learning_rate, weight_decay);
}
