// kd_rows.hip - fused row kernels: softmax / log_softmax, standardize (+ LayerNorm affine),
// cross-entropy loss and its gradient, for gfx950.
//
// The arithmetic restates kael's CPU row kernels (reference src/ops/nn.cpp:52-129 and
// 214-240): the row maximum is NaN-propagating, exponentials are evaluated in the element type,
// their sum is accumulated in double and rounded to the element type before the divide (or
// log); standardize takes mean and population variance in double. On the device the reference
// composes these from 5-12 separate elementwise/reduce launches (nn.cpp:153-160, 176-177,
// 185-187, 253-258); here each is one launch.
//
// Rows of up to 1024 elements are held in registers by one wave (one HBM read, one write);
// longer rows use a 256-lane workgroup per row and re-read the row (L2-resident) per pass.
#include <algorithm>

#include "kd_internal.h"

namespace kd {

namespace {

constexpr int kThreads = 256;

template <typename T> __device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int m = 32; m > 0; m /= 2) v = max_na(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int m = 32; m > 0; m /= 2) v += __shfl_xor(v, m, 64);
    return v;
}

// Multiply and add without contraction into FMA (kd_internal.h *_sep), so the LayerNorm affine
// rounds twice, as the reference's separate `* weight` and `+ bias` kernels do.
template <typename T> __device__ __forceinline__ T mul_rn(T a, T b) { return mul_sep(a, b); }
template <typename T> __device__ __forceinline__ T add_rn(T a, T b) { return add_sep(a, b); }
template <typename T> __device__ __forceinline__ T sub_rn(T a, T b) { return sub_sep(a, b); }
template <typename T> __device__ __forceinline__ T div_rn(T a, T b) { return div_sep(a, b); }

template <typename T> __device__ __forceinline__ T neg_inf() { return static_cast<T>(-INFINITY); }

enum RowOp { kSoftmax = 0, kLogSoftmax = 1, kCrossEntropy = 2, kCrossEntropyGrad = 3 };

// ---- softmax family, one wave per row ---------------------------------------------------------

template <typename T, int V, int Op>
__global__ __launch_bounds__(kThreads) void softmax_wave_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                                const int64_t* __restrict__ targets,
                                                                const T* __restrict__ weights, int64_t rows,
                                                                int64_t cols) {
    const int lane = threadIdx.x % 64;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const T* x = in + row * cols;
    T v[V];
    T largest = neg_inf<T>();
    bool first = true;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int64_t c = lane + 64 * j;
        v[j] = c < cols ? x[c] : neg_inf<T>();
        if (c < cols) {
            largest = first ? v[j] : max_na(largest, v[j]);
            first = false;
        }
    }
    // Lanes without elements hold -inf, the identity of the NaN-propagating max.
    largest = wave_max(largest);
    double total = 0.0;
    T e[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int64_t c = lane + 64 * j;
        e[j] = std::exp(sub_rn(v[j], largest));
        if (c < cols) total += static_cast<double>(e[j]);
    }
    total = wave_sum(total);
    const T denominator = static_cast<T>(total);
    if constexpr (Op == kSoftmax) {
        T* y = out + row * cols;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int64_t c = lane + 64 * j;
            if (c < cols) y[c] = div_rn(e[j], denominator);
        }
    } else if constexpr (Op == kLogSoftmax) {
        const T log_total = std::log(denominator);
        T* y = out + row * cols;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int64_t c = lane + 64 * j;
            if (c < cols) y[c] = sub_rn(sub_rn(v[j], largest), log_total);
        }
    } else if constexpr (Op == kCrossEntropy) {
        if (lane == 0) {
            const int64_t t = targets[row];
            out[row] = sub_rn(std::log(denominator), sub_rn(x[t], largest));
        }
    } else {
        const T w = weights[row];
        const int64_t t = targets[row];
        T* y = out + row * cols;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int64_t c = lane + 64 * j;
            if (c < cols) {
                T g = mul_rn(div_rn(e[j], denominator), w);
                if (c == t) g = sub_rn(g, w);
                y[c] = g;
            }
        }
    }
}

template <typename T> __device__ __forceinline__ T affine(T y, const T* w, const T* b, int64_t c);

// ---- vectorized wave-per-row variants (cols % 4 == 0, cols <= 1024) ----------------------------
//
// Same arithmetic as the scalar wave kernels; each lane holds V4 groups of 4 consecutive columns
// and moves them with 16-byte loads and stores (nontemporal for large tensors).

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Quad {
    T v[4];
};

template <bool NT, typename T> __device__ __forceinline__ Quad<T> ld4(const T* p) {
    Quad<T> q;
    if constexpr (NT && sizeof(T) == 4) {
        const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        __builtin_memcpy(&q, &r, 16);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) q.v[e] = p[e];
    }
    return q;
}

template <bool NT, typename T> __device__ __forceinline__ void st4(T* p, const Quad<T>& q) {
    if constexpr (NT && sizeof(T) == 4) {
        u32x4 r;
        __builtin_memcpy(&r, &q, 16);
        __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = q.v[e];
    }
}

template <typename T, int V4, int Op, bool NT>
__global__ __launch_bounds__(kThreads) void softmax_wave4_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                                 int64_t rows, int64_t cols) {
    const int lane = threadIdx.x % 64;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const T* x = in + row * cols;
    Quad<T> v[V4];
    T largest = neg_inf<T>();
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
            v[j] = ld4<NT>(x + c);
#pragma unroll
            for (int e = 0; e < 4; ++e) largest = max_na(largest, v[j].v[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j].v[e] = neg_inf<T>();
        }
    }
    largest = wave_max(largest);
    double total = 0.0;
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const T ex = std::exp(sub_rn(v[j].v[e], largest));
                if constexpr (Op == kSoftmax) v[j].v[e] = ex;
                total += static_cast<double>(ex);
            }
        }
    }
    total = wave_sum(total);
    const T denominator = static_cast<T>(total);
    const T log_total = Op == kLogSoftmax ? std::log(denominator) : T(0);
    T* y = out + row * cols;
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
            Quad<T> o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o.v[e] = Op == kSoftmax ? div_rn(v[j].v[e], denominator) : sub_rn(sub_rn(v[j].v[e], largest), log_total);
            st4<NT>(y + c, o);
        }
    }
}

template <typename T, int V4, bool NT>
__global__ __launch_bounds__(kThreads) void standardize_wave4_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                                     int64_t rows, int64_t cols, double eps,
                                                                     const T* __restrict__ w, const T* __restrict__ b,
                                                                     T* __restrict__ yhat) {
    const int lane = threadIdx.x % 64;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const T* x = in + row * cols;
    Quad<T> v[V4], wq[V4], bq[V4];
    double total = 0.0;
    // the affine weight and bias are loaded with the row, so that their latency overlaps the row's
    // instead of following the reductions
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
            v[j] = ld4<NT>(x + c);
            if (w != nullptr) {
                wq[j] = ld4<false>(w + c);
                bq[j] = ld4<false>(b + c);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
#pragma unroll
            for (int e = 0; e < 4; ++e) total += static_cast<double>(v[j].v[e]);
        }
    }
    const double center = wave_sum(total) / static_cast<double>(cols);
    double squares = 0.0;
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const double d = static_cast<double>(v[j].v[e]) - center;
                squares += d * d;
            }
        }
    }
    // (x - mean) * (1 / scale) in double: it differs from the reference's division by at most one
    // double ulp, which the rounding to T that follows absorbs (a per-element double divide made
    // this kernel compute-bound at a third of HBM bandwidth).
    const double rscale = 1.0 / std::sqrt(wave_sum(squares) / static_cast<double>(cols) + eps);
    T* y = out + row * cols;
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
            Quad<T> o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o.v[e] = static_cast<T>((static_cast<double>(v[j].v[e]) - center) * rscale);
            if (yhat != nullptr) st4<NT>(yhat + row * cols + c, o);
            if (w != nullptr) {
#pragma unroll
                for (int e = 0; e < 4; ++e) o.v[e] = add_rn(mul_rn(o.v[e], wq[j].v[e]), bq[j].v[e]);
            }
            st4<NT>(y + c, o);
        }
    }
}

// ---- softmax family, one workgroup per row (long rows) -------------------------------------------

template <typename T> __device__ __forceinline__ T block_max(T v, T* scratch) {
    v = wave_max(v);
    if (threadIdx.x % 64 == 0) scratch[threadIdx.x / 64] = v;
    __syncthreads();
    T r = scratch[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r = max_na(r, scratch[w]);
    __syncthreads();
    return r;
}

__device__ __forceinline__ double block_sum(double v, double* scratch) {
    v = wave_sum(v);
    if (threadIdx.x % 64 == 0) scratch[threadIdx.x / 64] = v;
    __syncthreads();
    double r = scratch[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) r += scratch[w];
    __syncthreads();
    return r;
}

template <typename T, int Op>
__global__ __launch_bounds__(kThreads) void softmax_block_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                                 const int64_t* __restrict__ targets,
                                                                 const T* __restrict__ weights, int64_t rows,
                                                                 int64_t cols) {
    __shared__ T tmax[kThreads / 64];
    __shared__ double tsum[kThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const T* x = in + row * cols;
        T largest = neg_inf<T>();
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) largest = max_na(largest, x[c]);
        largest = block_max(largest, tmax);
        double total = 0.0;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) total += static_cast<double>(std::exp(sub_rn(x[c], largest)));
        total = block_sum(total, tsum);
        const T denominator = static_cast<T>(total);
        if constexpr (Op == kSoftmax) {
            T* y = out + row * cols;
            for (int64_t c = threadIdx.x; c < cols; c += kThreads) y[c] = div_rn(std::exp(sub_rn(x[c], largest)), denominator);
        } else if constexpr (Op == kLogSoftmax) {
            const T log_total = std::log(denominator);
            T* y = out + row * cols;
            for (int64_t c = threadIdx.x; c < cols; c += kThreads) y[c] = sub_rn(sub_rn(x[c], largest), log_total);
        } else if constexpr (Op == kCrossEntropy) {
            if (threadIdx.x == 0) out[row] = sub_rn(std::log(denominator), sub_rn(x[targets[row]], largest));
        } else {
            const T w = weights[row];
            const int64_t t = targets[row];
            T* y = out + row * cols;
            for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
                T g = mul_rn(div_rn(std::exp(sub_rn(x[c], largest)), denominator), w);
                if (c == t) g = sub_rn(g, w);
                y[c] = g;
            }
        }
    }
}

template <typename T, int Op>
int softmax_family(T* out, const T* in, const int64_t* targets, const T* weights, int64_t rows, int64_t cols) {
    if (rows == 0 || cols == 0) return KD_OK;
    const dim3 block(kThreads);
    const bool quads = (Op == kSoftmax || Op == kLogSoftmax) && cols % 4 == 0 && cols <= 1024 &&
                       reinterpret_cast<uintptr_t>(in) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
    if (quads) {
        const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
        const bool nt = rows * cols * static_cast<int64_t>(sizeof(T)) >= (int64_t{16} << 20);
#define KD_WAVE4(V4)                                                                                                   \
    if (nt) hipLaunchKernelGGL((softmax_wave4_kernel<T, V4, Op, true>), grid, block, 0, stream(), out, in, rows, cols); \
    else hipLaunchKernelGGL((softmax_wave4_kernel<T, V4, Op, false>), grid, block, 0, stream(), out, in, rows, cols);
        if (cols <= 256) { KD_WAVE4(1) }
        else if (cols <= 512) { KD_WAVE4(2) }
        else { KD_WAVE4(4) }
#undef KD_WAVE4
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    if (cols <= 1024) {
        const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
        if (rows > int64_t{0xffffffff} * 4) return fail(KD_E_INVALID, "row kernel: too many rows");
#define KD_WAVE(V) hipLaunchKernelGGL((softmax_wave_kernel<T, V, Op>), grid, block, 0, stream(), out, in, targets, weights, rows, cols)
        if (cols <= 64) KD_WAVE(1);
        else if (cols <= 128) KD_WAVE(2);
        else if (cols <= 256) KD_WAVE(4);
        else if (cols <= 512) KD_WAVE(8);
        else KD_WAVE(16);
#undef KD_WAVE
    } else {
        const int64_t blocks = std::min<int64_t>(rows, int64_t{compute_units()} * 32);
        hipLaunchKernelGGL((softmax_block_kernel<T, Op>), dim3(static_cast<uint32_t>(blocks)), block, 0, stream(), out, in,
                           targets, weights, rows, cols);
    }
    KD_LAUNCH_CHECK();
    return KD_OK;
}

// ---- standardize -------------------------------------------------------------------------------------

// The LayerNorm affine step of a standardized value: y * w[c] + b[c], each op rounded.
template <typename T> __device__ __forceinline__ T affine(T y, const T* w, const T* b, int64_t c) {
    return w != nullptr ? add_rn(mul_rn(y, w[c]), b[c]) : y;
}

template <typename T, int V>
__global__ __launch_bounds__(kThreads) void standardize_wave_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                                    int64_t rows, int64_t cols, double eps,
                                                                    const T* __restrict__ w, const T* __restrict__ b,
                                                                    T* __restrict__ yhat) {
    const int lane = threadIdx.x % 64;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const T* x = in + row * cols;
    T v[V];
    double total = 0.0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int64_t c = lane + 64 * j;
        v[j] = c < cols ? x[c] : T(0);
        total += static_cast<double>(v[j]);
    }
    const double center = wave_sum(total) / static_cast<double>(cols);
    double squares = 0.0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < cols) {
            const double d = static_cast<double>(v[j]) - center;
            squares += d * d;
        }
    }
    const double scale = std::sqrt(wave_sum(squares) / static_cast<double>(cols) + eps);
    T* y = out + row * cols;
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < cols) {
            const T s = static_cast<T>((static_cast<double>(v[j]) - center) / scale);
            if (yhat != nullptr) yhat[row * cols + c] = s;
            y[c] = affine(s, w, b, c);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void standardize_block_kernel(T* __restrict__ out, const T* __restrict__ in,
                                                                     int64_t rows, int64_t cols, double eps,
                                                                     const T* __restrict__ w, const T* __restrict__ b,
                                                                     T* __restrict__ yhat) {
    __shared__ double tsum[kThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const T* x = in + row * cols;
        double total = 0.0;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) total += static_cast<double>(x[c]);
        const double center = block_sum(total, tsum) / static_cast<double>(cols);
        double squares = 0.0;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
            const double d = static_cast<double>(x[c]) - center;
            squares += d * d;
        }
        const double scale = std::sqrt(block_sum(squares, tsum) / static_cast<double>(cols) + eps);
        T* y = out + row * cols;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
            const T s = static_cast<T>((static_cast<double>(x[c]) - center) / scale);
            if (yhat != nullptr) yhat[row * cols + c] = s;
            y[c] = affine(s, w, b, c);
        }
    }
}

template <typename T>
int standardize_typed(T* out, const T* in, int64_t rows, int64_t cols, double eps, const T* w, const T* b,
                      T* yhat = nullptr) {
    if (rows == 0 || cols == 0) return KD_OK;
    const dim3 block(kThreads);
    const bool quads = cols % 4 == 0 && cols <= 1024 && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(out) % 16 == 0 && reinterpret_cast<uintptr_t>(yhat) % 16 == 0;
    if (quads) {
        const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
        const bool nt = rows * cols * static_cast<int64_t>(sizeof(T)) >= (int64_t{16} << 20);
#define KD_WAVE4(V4)                                                                                                    \
    if (nt) hipLaunchKernelGGL((standardize_wave4_kernel<T, V4, true>), grid, block, 0, stream(), out, in, rows, cols, eps, w, b, yhat); \
    else hipLaunchKernelGGL((standardize_wave4_kernel<T, V4, false>), grid, block, 0, stream(), out, in, rows, cols, eps, w, b, yhat);
        if (cols <= 256) { KD_WAVE4(1) }
        else if (cols <= 512) { KD_WAVE4(2) }
        else { KD_WAVE4(4) }
#undef KD_WAVE4
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    if (cols <= 1024) {
        const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
#define KD_WAVE(V) hipLaunchKernelGGL((standardize_wave_kernel<T, V>), grid, block, 0, stream(), out, in, rows, cols, eps, w, b, yhat)
        if (cols <= 64) KD_WAVE(1);
        else if (cols <= 128) KD_WAVE(2);
        else if (cols <= 256) KD_WAVE(4);
        else if (cols <= 512) KD_WAVE(8);
        else KD_WAVE(16);
#undef KD_WAVE
    } else {
        const int64_t blocks = std::min<int64_t>(rows, int64_t{compute_units()} * 32);
        hipLaunchKernelGGL((standardize_block_kernel<T>), dim3(static_cast<uint32_t>(blocks)), block, 0, stream(), out, in,
                           rows, cols, eps, w, b, yhat);
    }
    KD_LAUNCH_CHECK();
    return KD_OK;
}

// ---- backward passes of softmax, log_softmax and standardize ----------------------------------------
//
// kael composes each backward from whole-tensor device ops (reference
// src/autograd/functions_reduce.cpp:150-192), every op rounded to T and every row sum accumulated
// in double and rounded to T (src/ops/reduce.cpp:308-342):
//   softmax      y * (g - sum(g * y))
//   log_softmax  g - exp(y) * sum(g)
//   standardize  ((g - mean(g)) - y * mean(g * y)) / sqrt(var(x) + eps), mean = sum / T(n),
//                var = sum((x - mean(x))^2) / T(n) (population variance; each square rounded to T)
// These kernels keep that rounding sequence and fuse it into one pass over the row (plus a second
// pass over x in registers for the variance): only the order of the double sums differs.
enum BackOp { kSoftmaxBack = 0, kLogSoftmaxBack = 1, kStandardizeBack = 2 };

template <typename T> struct BackSums {
    double s1 = 0.0, s2 = 0.0, s3 = 0.0;  // softmax: sum(g*y); log_softmax: sum(g); standardize: sum(x), sum(g), sum(g*y)
};

template <int Op, typename T> __device__ __forceinline__ void back_accumulate(BackSums<T>& s, T x, T y, T g) {
    if constexpr (Op == kSoftmaxBack) {
        s.s1 += static_cast<double>(mul_rn(g, y));
    } else if constexpr (Op == kLogSoftmaxBack) {
        s.s1 += static_cast<double>(g);
    } else {
        s.s1 += static_cast<double>(x);
        s.s2 += static_cast<double>(g);
        s.s3 += static_cast<double>(mul_rn(g, y));
    }
}

// The per-row scalars of the output formula once the sums are complete.
template <typename T> struct BackScalars {
    T s;      // softmax: sum(g*y); log_softmax: sum(g); standardize: mean(x)
    T mg;     // standardize: mean(g)
    T mgy;    // standardize: mean(g*y)
    T scale;  // standardize: sqrt(var(x) + eps), set after the variance pass
};

template <int Op, typename T> __device__ __forceinline__ T back_output(const BackScalars<T>& k, T y, T g) {
    if constexpr (Op == kSoftmaxBack) {
        return mul_rn(y, sub_rn(g, k.s));
    } else if constexpr (Op == kLogSoftmaxBack) {
        return sub_rn(g, mul_rn(static_cast<T>(std::exp(y)), k.s));
    } else {
        return div_rn(sub_rn(sub_rn(g, k.mg), mul_rn(y, k.mgy)), k.scale);
    }
}

template <int Op, typename T> __device__ __forceinline__ BackScalars<T> back_scalars(const BackSums<T>& s, int64_t cols) {
    BackScalars<T> k{};
    k.s = static_cast<T>(s.s1);
    if constexpr (Op == kStandardizeBack) {
        const T n = static_cast<T>(cols);
        k.s = div_rn(static_cast<T>(s.s1), n);
        k.mg = div_rn(static_cast<T>(s.s2), n);
        k.mgy = div_rn(static_cast<T>(s.s3), n);
    }
    return k;
}

template <typename T> __device__ __forceinline__ T back_scale(double squares, int64_t cols, double eps) {
    const T var = div_rn(static_cast<T>(squares), static_cast<T>(cols));
    return static_cast<T>(std::sqrt(add_rn(var, static_cast<T>(eps))));
}

// One wave per row of cols <= 1024 (cols % 4 == 0, 16-byte aligned rows): the row's y, g (and x)
// are held in registers; one read of each input, one write.
template <typename T, int V4, int Op, bool NT>
__global__ __launch_bounds__(kThreads) void row_backward_wave4_kernel(T* __restrict__ out, const T* __restrict__ xin,
                                                                      const T* __restrict__ yin,
                                                                      const T* __restrict__ gin, int64_t rows,
                                                                      int64_t cols, double eps) {
    const int lane = threadIdx.x % 64;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    if (row >= rows) return;
    const int64_t base = row * cols;
    Quad<T> y[V4], g[V4], x[V4];
    BackSums<T> s;
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
            y[j] = ld4<NT>(yin + base + c);
            g[j] = ld4<NT>(gin + base + c);
            if constexpr (Op == kStandardizeBack) x[j] = ld4<NT>(xin + base + c);
#pragma unroll
            for (int e = 0; e < 4; ++e) back_accumulate<Op>(s, Op == kStandardizeBack ? x[j].v[e] : T(0), y[j].v[e], g[j].v[e]);
        }
    }
    s.s1 = wave_sum(s.s1);
    if constexpr (Op == kStandardizeBack) {
        s.s2 = wave_sum(s.s2);
        s.s3 = wave_sum(s.s3);
    }
    BackScalars<T> k = back_scalars<Op>(s, cols);
    if constexpr (Op == kStandardizeBack) {
        double squares = 0.0;
#pragma unroll
        for (int j = 0; j < V4; ++j) {
            const int64_t c = 4 * (lane + 64 * j);
            if (c < cols) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const T d = sub_rn(x[j].v[e], k.s);
                    squares += static_cast<double>(mul_rn(d, d));
                }
            }
        }
        k.scale = back_scale<T>(wave_sum(squares), cols, eps);
    }
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) {
            Quad<T> o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o.v[e] = back_output<Op>(k, y[j].v[e], g[j].v[e]);
            st4<NT>(out + base + c, o);
        }
    }
}

// Any row length and alignment: a workgroup per row, the row read from memory once per pass
// (later passes hit the L2 for rows that fit).
template <typename T, int Op>
__global__ __launch_bounds__(kThreads) void row_backward_block_kernel(T* __restrict__ out, const T* __restrict__ xin,
                                                                      const T* __restrict__ yin,
                                                                      const T* __restrict__ gin, int64_t rows,
                                                                      int64_t cols, double eps) {
    __shared__ double tsum[kThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int64_t base = row * cols;
        BackSums<T> s;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads)
            back_accumulate<Op>(s, Op == kStandardizeBack ? xin[base + c] : T(0), yin[base + c], gin[base + c]);
        s.s1 = block_sum(s.s1, tsum);
        if constexpr (Op == kStandardizeBack) {
            s.s2 = block_sum(s.s2, tsum);
            s.s3 = block_sum(s.s3, tsum);
        }
        BackScalars<T> k = back_scalars<Op>(s, cols);
        if constexpr (Op == kStandardizeBack) {
            double squares = 0.0;
            for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
                const T d = sub_rn(xin[base + c], k.s);
                squares += static_cast<double>(mul_rn(d, d));
            }
            k.scale = back_scale<T>(block_sum(squares, tsum), cols, eps);
        }
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) out[base + c] = back_output<Op>(k, yin[base + c], gin[base + c]);
    }
}

template <typename T, int Op>
int row_backward_typed(T* out, const T* x, const T* y, const T* g, int64_t rows, int64_t cols, double eps) {
    if (rows == 0 || cols == 0) return KD_OK;
    const dim3 block(kThreads);
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool quads = cols % 4 == 0 && cols <= 1024 && aligned(out) && aligned(y) && aligned(g) &&
                       (Op != kStandardizeBack || aligned(x));
    if (quads) {
        if ((rows + 3) / 4 > int64_t{0xffffffff}) return fail(KD_E_INVALID, "row backward: too many rows");
        const dim3 grid(static_cast<uint32_t>((rows + 3) / 4));
        const bool nt = rows * cols * static_cast<int64_t>(sizeof(T)) >= (int64_t{16} << 20);
#define KD_BACK4(V4)                                                                                                  \
    if (nt) hipLaunchKernelGGL((row_backward_wave4_kernel<T, V4, Op, true>), grid, block, 0, stream(), out, x, y, g, rows, cols, eps); \
    else hipLaunchKernelGGL((row_backward_wave4_kernel<T, V4, Op, false>), grid, block, 0, stream(), out, x, y, g, rows, cols, eps);
        if (cols <= 256) { KD_BACK4(1) }
        else if (cols <= 512) { KD_BACK4(2) }
        else { KD_BACK4(4) }
#undef KD_BACK4
    } else {
        const int64_t blocks = std::min<int64_t>(rows, int64_t{compute_units()} * 32);
        hipLaunchKernelGGL((row_backward_block_kernel<T, Op>), dim3(static_cast<uint32_t>(blocks)), block, 0, stream(), out,
                           x, y, g, rows, cols, eps);
    }
    KD_LAUNCH_CHECK();
    return KD_OK;
}

// ---- LayerNorm backward ---------------------------------------------------------------------------
//
// kael's LayerNorm::forward is standardize(x) * w + b (reference src/nn/layers.cpp:60-68); its
// backward is composed from AddBackward, MulBackward and StandardizeBackward
// (src/autograd/functions_math.cpp:54-72, functions_reduce.cpp:176-192). With y the standardized
// rows and g the gradient of the output:
//   grad_in     = the standardize backward (above) of gy = g * w (each product rounded),
//   grad_weight = sum over rows of g * y (each product rounded, summed in double),
//   grad_bias   = sum over rows of g (in double).
// ln_backward_wave4_kernel does all three in one pass for rows of <= 1024 (cols % 4 == 0): workgroup
// s of W waves takes the rows [s * rs, s * rs + rs), wave w the rows s * rs + w + W i in increasing
// order; each lane keeps the column sums of its columns in registers, the waves add theirs in LDS in
// wave order, and the workgroup writes its partials (double) for ln_combine_kernel, which adds the
// segments in order. Other shapes: ln_backward_block_kernel (a workgroup per row) for grad_in and
// ln_columns_kernel for the column partials.
template <typename T, int V4, bool NT, int Waves>
__global__ __launch_bounds__(Waves * 64) void ln_backward_wave4_kernel(T* __restrict__ grad_in, double* __restrict__ pw,
                                                                       double* __restrict__ pb, const T* __restrict__ xin,
                                                                       const T* __restrict__ yin, const T* __restrict__ gin,
                                                                       const T* __restrict__ w, int64_t rows, int64_t cols,
                                                                       int64_t rows_per_segment, double eps) {
    constexpr int kWaves = Waves;
    __shared__ double lds[kWaves][2][V4 * 4][64];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_segment;
    const int64_t r1 = std::min<int64_t>(rows, r0 + rows_per_segment);
    Quad<T> wq[V4];
    double cw[V4][4], cb[V4][4];
#pragma unroll
    for (int j = 0; j < V4; ++j) {
        const int64_t c = 4 * (lane + 64 * j);
        if (c < cols) wq[j] = ld4<false>(w + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) cw[j][e] = cb[j][e] = 0.0;
    }
    for (int64_t row = r0 + wave; row < r1; row += kWaves) {
        const int64_t base = row * cols;
        Quad<T> x[V4], y[V4], gy[V4];
        BackSums<T> s;
#pragma unroll
        for (int j = 0; j < V4; ++j) {
            const int64_t c = 4 * (lane + 64 * j);
            if (c < cols) {
                x[j] = ld4<NT>(xin + base + c);
                y[j] = ld4<NT>(yin + base + c);
                const Quad<T> g = ld4<NT>(gin + base + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cw[j][e] += static_cast<double>(mul_rn(g.v[e], y[j].v[e]));
                    cb[j][e] += static_cast<double>(g.v[e]);
                    gy[j].v[e] = mul_rn(g.v[e], wq[j].v[e]);
                    back_accumulate<kStandardizeBack>(s, x[j].v[e], y[j].v[e], gy[j].v[e]);
                }
            }
        }
        s.s1 = wave_sum(s.s1);
        s.s2 = wave_sum(s.s2);
        s.s3 = wave_sum(s.s3);
        BackScalars<T> k = back_scalars<kStandardizeBack>(s, cols);
        double squares = 0.0;
#pragma unroll
        for (int j = 0; j < V4; ++j) {
            const int64_t c = 4 * (lane + 64 * j);
            if (c < cols) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const T d = sub_rn(x[j].v[e], k.s);
                    squares += static_cast<double>(mul_rn(d, d));
                }
            }
        }
        k.scale = back_scale<T>(wave_sum(squares), cols, eps);
#pragma unroll
        for (int j = 0; j < V4; ++j) {
            const int64_t c = 4 * (lane + 64 * j);
            if (c < cols) {
                Quad<T> o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o.v[e] = back_output<kStandardizeBack>(k, y[j].v[e], gy[j].v[e]);
                st4<NT>(grad_in + base + c, o);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < V4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lds[wave][0][j * 4 + e][lane] = cw[j][e];
            lds[wave][1][j * 4 + e][lane] = cb[j][e];
        }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int j = 0; j < V4; ++j) {
            const int64_t c = 4 * (lane + 64 * j);
            if (c < cols) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    double sw = lds[0][0][j * 4 + e][lane], sb = lds[0][1][j * 4 + e][lane];
#pragma unroll
                    for (int v = 1; v < kWaves; ++v) {
                        sw += lds[v][0][j * 4 + e][lane];
                        sb += lds[v][1][j * 4 + e][lane];
                    }
                    pw[blockIdx.x * cols + c + e] = sw;
                    pb[blockIdx.x * cols + c + e] = sb;
                }
            }
        }
    }
}

// grad_in for any row length: a workgroup per row, gy = g * w recomputed in each pass.
template <typename T>
__global__ __launch_bounds__(kThreads) void ln_backward_block_kernel(T* __restrict__ grad_in, const T* __restrict__ xin,
                                                                     const T* __restrict__ yin, const T* __restrict__ gin,
                                                                     const T* __restrict__ w, int64_t rows, int64_t cols,
                                                                     double eps) {
    __shared__ double tsum[kThreads / 64];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int64_t base = row * cols;
        BackSums<T> s;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads)
            back_accumulate<kStandardizeBack>(s, xin[base + c], yin[base + c], mul_rn(gin[base + c], w[c]));
        s.s1 = block_sum(s.s1, tsum);
        s.s2 = block_sum(s.s2, tsum);
        s.s3 = block_sum(s.s3, tsum);
        BackScalars<T> k = back_scalars<kStandardizeBack>(s, cols);
        double squares = 0.0;
        for (int64_t c = threadIdx.x; c < cols; c += kThreads) {
            const T d = sub_rn(xin[base + c], k.s);
            squares += static_cast<double>(mul_rn(d, d));
        }
        k.scale = back_scale<T>(block_sum(squares, tsum), cols, eps);
        for (int64_t c = threadIdx.x; c < cols; c += kThreads)
            grad_in[base + c] = back_output<kStandardizeBack>(k, yin[base + c], mul_rn(gin[base + c], w[c]));
    }
}

// Column partials for any shape: workgroup (cb, s) sums the 64 columns [64 cb, 64 cb + 64) over the
// segment's rows, wave w the contiguous quarter [r0 + w q, r0 + w q + q), the waves in order.
template <typename T>
__global__ __launch_bounds__(kThreads) void ln_columns_kernel(double* __restrict__ pw, double* __restrict__ pb,
                                                              const T* __restrict__ yin, const T* __restrict__ gin,
                                                              int64_t rows, int64_t cols, int64_t rows_per_segment) {
    constexpr int kWaves = kThreads / 64;
    __shared__ double lds[kWaves][2][64];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * 64 + lane;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_segment;
    const int64_t r1 = std::min<int64_t>(rows, r0 + rows_per_segment);
    const int64_t q = (r1 - r0 + kWaves - 1) / kWaves;
    const int64_t w0 = std::min<int64_t>(r1, r0 + wave * q);
    const int64_t w1 = std::min<int64_t>(r1, w0 + q);
    double sw = 0.0, sb = 0.0;
    if (c < cols) {
        for (int64_t r = w0; r < w1; ++r) {
            const T g = gin[r * cols + c];
            sw += static_cast<double>(mul_rn(g, yin[r * cols + c]));
            sb += static_cast<double>(g);
        }
    }
    lds[wave][0][lane] = sw;
    lds[wave][1][lane] = sb;
    __syncthreads();
    if (wave == 0 && c < cols) {
        for (int v = 1; v < kWaves; ++v) {
            sw += lds[v][0][lane];
            sb += lds[v][1][lane];
        }
        pw[blockIdx.y * cols + c] = sw;
        pb[blockIdx.y * cols + c] = sb;
    }
}

// The weight and bias gradients from the segment partials: a workgroup of 16 waves per 16 columns
// (C4's 256 columns: 16 workgroups), lane i of wave w on column i % 16 and the contiguous segment
// range r = 4 w + i / 16 of 64 (8 loads of each array in flight per lane). Each range is summed in
// segment order, a wave's four ranges in order, then the 16 waves' sums in order: every column in
// the same fixed order.
constexpr int kCombineThreads = 1024;
constexpr int kCombineCols = 16;
template <typename T>
__global__ __launch_bounds__(kCombineThreads) void ln_combine_kernel(T* __restrict__ grad_w, T* __restrict__ grad_b,
                                                                     const double* __restrict__ pw,
                                                                     const double* __restrict__ pb, int64_t segments,
                                                                     int64_t cols) {
    constexpr int kWaves = kCombineThreads / 64;
    constexpr int kRanges = kWaves * (64 / kCombineCols);
    constexpr int kBatch = 8;
    __shared__ double ranges[2][kRanges][kCombineCols];
    __shared__ double waves[2][kWaves][kCombineCols];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int ci = lane % kCombineCols;
    const int r = wave * (64 / kCombineCols) + lane / kCombineCols;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kCombineCols + ci;
    const int64_t q = (segments + kRanges - 1) / kRanges;
    const int64_t s0 = std::min<int64_t>(segments, r * q);
    const int64_t s1 = std::min<int64_t>(segments, s0 + q);
    double sw = 0.0, sb = 0.0;
    if (c < cols) {
        for (int64_t s = s0; s < s1; s += kBatch) {
            double a[kBatch], b[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (s + u < s1) {
                    a[u] = pw[(s + u) * cols + c];
                    b[u] = pb[(s + u) * cols + c];
                }
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (s + u < s1) {
                    sw += a[u];
                    sb += b[u];
                }
        }
    }
    ranges[0][r][ci] = sw;
    ranges[1][r][ci] = sb;
    __syncthreads();
    if (lane < kCombineCols) {  // the wave's four ranges, in order
        double w4 = ranges[0][r][ci], b4 = ranges[1][r][ci];
#pragma unroll
        for (int k = 1; k < 64 / kCombineCols; ++k) {
            w4 += ranges[0][r + k][ci];
            b4 += ranges[1][r + k][ci];
        }
        waves[0][wave][ci] = w4;
        waves[1][wave][ci] = b4;
    }
    __syncthreads();
    if (wave == 0 && lane < kCombineCols && c < cols) {
        double tw = waves[0][0][ci], tb = waves[1][0][ci];
        for (int v = 1; v < kWaves; ++v) {
            tw += waves[0][v][ci];
            tb += waves[1][v][ci];
        }
        if (grad_w != nullptr) grad_w[c] = static_cast<T>(tw);
        if (grad_b != nullptr) grad_b[c] = static_cast<T>(tb);
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void zero_pair_kernel(T* a, T* b, int64_t n) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        if (a != nullptr) a[i] = T(0);
        if (b != nullptr) b[i] = T(0);
    }
}

template <typename T>
int ln_backward_typed(T* grad_in, T* grad_w, T* grad_b, const T* x, const T* y, const T* g, const T* w, int64_t rows,
                      int64_t cols, double eps) {
    const dim3 block(kThreads);
    const auto aligned = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool quads = cols % 4 == 0 && cols <= 1024 && aligned(grad_in) && aligned(x) && aligned(y) && aligned(g) &&
                       aligned(w);
    const bool columns = grad_w != nullptr || grad_b != nullptr;
    // segments of at least 16 rows, at most 4 per CU
    const int64_t segments = std::max<int64_t>(1, std::min<int64_t>((rows + 15) / 16, int64_t{compute_units()} * 4));
    const int64_t rows_per_segment = (rows + segments - 1) / segments;
    if (segments > 65535) return fail(KD_E_INVALID, "layer norm backward: too many rows");
    Workspace ws;  // the column partials, held until ln_combine_kernel is enqueued
    double* pw = nullptr;
    double* pb = nullptr;
    if (columns || quads) {
        if (int rc = workspace(ws, static_cast<size_t>(2 * segments * cols) * sizeof(double))) return rc;
        pw = static_cast<double*>(ws.ptr);
        pb = pw + segments * cols;
    }
    if (quads) {
        const bool nt = rows * cols * static_cast<int64_t>(sizeof(T)) >= (int64_t{16} << 20);
        const dim3 grid(static_cast<uint32_t>(segments));
#define KD_LN4(V4, W)                                                                                                   \
    if (nt) hipLaunchKernelGGL((ln_backward_wave4_kernel<T, V4, true, W>), grid, dim3(64 * W), 0, stream(), grad_in, pw, pb, \
                               x, y, g, w, rows, cols, rows_per_segment, eps);                                          \
    else hipLaunchKernelGGL((ln_backward_wave4_kernel<T, V4, false, W>), grid, dim3(64 * W), 0, stream(), grad_in, pw, pb, \
                            x, y, g, w, rows, cols, rows_per_segment, eps);
        // Rows of <= 256 columns: 16 waves per workgroup, so that a segment of 16 rows gives each
        // wave one row (C4's 4096 x 256: the row chains of the four waves of a 256-thread group ran
        // one after another, four rows each). Longer rows: 4 waves (their column partials in LDS
        // would not fit 16).
        if (cols <= 256) { KD_LN4(1, 16) }
        else if (cols <= 512) { KD_LN4(2, 4) }
        else { KD_LN4(4, 4) }
#undef KD_LN4
        KD_LAUNCH_CHECK();
    } else {
        const int64_t blocks = std::min<int64_t>(rows, int64_t{compute_units()} * 32);
        hipLaunchKernelGGL((ln_backward_block_kernel<T>), dim3(static_cast<uint32_t>(blocks)), block, 0, stream(), grad_in,
                           x, y, g, w, rows, cols, eps);
        KD_LAUNCH_CHECK();
        if (columns) {
            const int64_t col_blocks = (cols + 63) / 64;
            if (col_blocks > int64_t{0xffffffff}) return fail(KD_E_INVALID, "layer norm backward: too many columns");
            hipLaunchKernelGGL((ln_columns_kernel<T>), dim3(static_cast<uint32_t>(col_blocks), static_cast<uint32_t>(segments)),
                               block, 0, stream(), pw, pb, y, g, rows, cols, rows_per_segment);
            KD_LAUNCH_CHECK();
        }
    }
    if (columns) {
        const int64_t col_blocks = (cols + kCombineCols - 1) / kCombineCols;
        if (col_blocks > int64_t{0xffffffff}) return fail(KD_E_INVALID, "layer norm backward: too many columns");
        hipLaunchKernelGGL((ln_combine_kernel<T>), dim3(static_cast<uint32_t>(col_blocks)), dim3(kCombineThreads), 0,
                           stream(), grad_w, grad_b, static_cast<const double*>(pw), static_cast<const double*>(pb),
                           segments, cols);
        KD_LAUNCH_CHECK();
    }
    return KD_OK;
}

int check_rows(int dtype, int64_t rows, int64_t cols) {
    if (dtype != KD_F32 && dtype != KD_F64) return fail(KD_E_INVALID, "row kernel: dtype must be f32 or f64");
    if (rows < 0 || cols < 0) return fail(KD_E_INVALID, "row kernel: negative size");
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

extern "C" int kd_softmax_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols, int log_softmax) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (rows == 0 || cols == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32) {
        return log_softmax ? softmax_family<float, kLogSoftmax>(static_cast<float*>(out), static_cast<const float*>(in), nullptr, nullptr, rows, cols)
                           : softmax_family<float, kSoftmax>(static_cast<float*>(out), static_cast<const float*>(in), nullptr, nullptr, rows, cols);
    }
    return log_softmax ? softmax_family<double, kLogSoftmax>(static_cast<double*>(out), static_cast<const double*>(in), nullptr, nullptr, rows, cols)
                       : softmax_family<double, kSoftmax>(static_cast<double*>(out), static_cast<const double*>(in), nullptr, nullptr, rows, cols);
}

extern "C" int kd_standardize_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols, double eps,
                                   const void* weight, const void* bias) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if ((weight == nullptr) != (bias == nullptr)) return fail(KD_E_INVALID, "kd_standardize_rows: weight and bias go together");
    if (rows == 0 || cols == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32)
        return standardize_typed<float>(static_cast<float*>(out), static_cast<const float*>(in), rows, cols, eps,
                                        static_cast<const float*>(weight), static_cast<const float*>(bias));
    return standardize_typed<double>(static_cast<double*>(out), static_cast<const double*>(in), rows, cols, eps,
                                     static_cast<const double*>(weight), static_cast<const double*>(bias));
}

extern "C" int kd_cross_entropy_rows(int dtype, void* losses, const void* logits, const int64_t* targets, int64_t rows,
                                     int64_t cols) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (rows == 0) return KD_OK;
    if (cols == 0) return fail(KD_E_INVALID, "kd_cross_entropy_rows: no classes");
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32)
        return softmax_family<float, kCrossEntropy>(static_cast<float*>(losses), static_cast<const float*>(logits), targets, nullptr, rows, cols);
    return softmax_family<double, kCrossEntropy>(static_cast<double*>(losses), static_cast<const double*>(logits), targets, nullptr, rows, cols);
}

extern "C" int kd_cross_entropy_grad(int dtype, void* out, const void* logits, const int64_t* targets,
                                     const void* row_weights, int64_t rows, int64_t cols) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (rows == 0) return KD_OK;
    if (cols == 0) return fail(KD_E_INVALID, "kd_cross_entropy_grad: no classes");
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32)
        return softmax_family<float, kCrossEntropyGrad>(static_cast<float*>(out), static_cast<const float*>(logits), targets,
                                                        static_cast<const float*>(row_weights), rows, cols);
    return softmax_family<double, kCrossEntropyGrad>(static_cast<double*>(out), static_cast<const double*>(logits), targets,
                                                     static_cast<const double*>(row_weights), rows, cols);
}

extern "C" int kd_softmax_rows_backward(int dtype, void* out, const void* y, const void* grad, int64_t rows,
                                        int64_t cols, int log_softmax) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (rows == 0 || cols == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32) {
        auto* o = static_cast<float*>(out);
        const auto* yy = static_cast<const float*>(y);
        const auto* gg = static_cast<const float*>(grad);
        return log_softmax ? row_backward_typed<float, kLogSoftmaxBack>(o, nullptr, yy, gg, rows, cols, 0.0)
                           : row_backward_typed<float, kSoftmaxBack>(o, nullptr, yy, gg, rows, cols, 0.0);
    }
    auto* o = static_cast<double*>(out);
    const auto* yy = static_cast<const double*>(y);
    const auto* gg = static_cast<const double*>(grad);
    return log_softmax ? row_backward_typed<double, kLogSoftmaxBack>(o, nullptr, yy, gg, rows, cols, 0.0)
                       : row_backward_typed<double, kSoftmaxBack>(o, nullptr, yy, gg, rows, cols, 0.0);
}

extern "C" int kd_layer_norm_rows(int dtype, void* out, void* standardized, const void* in, int64_t rows, int64_t cols,
                                  double eps, const void* weight, const void* bias) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (rows == 0 || cols == 0) return KD_OK;
    if (out == nullptr || standardized == nullptr || in == nullptr || weight == nullptr || bias == nullptr)
        return fail(KD_E_INVALID, "kd_layer_norm_rows: null pointer");
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32)
        return standardize_typed<float>(static_cast<float*>(out), static_cast<const float*>(in), rows, cols, eps,
                                        static_cast<const float*>(weight), static_cast<const float*>(bias),
                                        static_cast<float*>(standardized));
    return standardize_typed<double>(static_cast<double*>(out), static_cast<const double*>(in), rows, cols, eps,
                                     static_cast<const double*>(weight), static_cast<const double*>(bias),
                                     static_cast<double*>(standardized));
}

extern "C" int kd_layer_norm_rows_backward(int dtype, void* grad_in, void* grad_weight, void* grad_bias, const void* x,
                                           const void* standardized, const void* grad, const void* weight, int64_t rows,
                                           int64_t cols, double eps) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (cols == 0) return KD_OK;
    if (grad_in == nullptr && rows > 0) return fail(KD_E_INVALID, "kd_layer_norm_rows_backward: null grad_in");
    if (rows > 0 && (x == nullptr || standardized == nullptr || grad == nullptr || weight == nullptr))
        return fail(KD_E_INVALID, "kd_layer_norm_rows_backward: null input");
    if (int rc = ensure_device()) return rc;
    if (rows == 0) {  // the column sums of no rows are zero (a kernel, not a memset: callers may capture this)
        const dim3 grid(static_cast<uint32_t>(std::min<int64_t>((cols + kThreads - 1) / kThreads, 65535)));
        if (dtype == KD_F32)
            hipLaunchKernelGGL((zero_pair_kernel<float>), grid, dim3(kThreads), 0, stream(), static_cast<float*>(grad_weight),
                               static_cast<float*>(grad_bias), cols);
        else
            hipLaunchKernelGGL((zero_pair_kernel<double>), grid, dim3(kThreads), 0, stream(),
                               static_cast<double*>(grad_weight), static_cast<double*>(grad_bias), cols);
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    if (dtype == KD_F32)
        return ln_backward_typed<float>(static_cast<float*>(grad_in), static_cast<float*>(grad_weight),
                                        static_cast<float*>(grad_bias), static_cast<const float*>(x),
                                        static_cast<const float*>(standardized), static_cast<const float*>(grad),
                                        static_cast<const float*>(weight), rows, cols, eps);
    return ln_backward_typed<double>(static_cast<double*>(grad_in), static_cast<double*>(grad_weight),
                                     static_cast<double*>(grad_bias), static_cast<const double*>(x),
                                     static_cast<const double*>(standardized), static_cast<const double*>(grad),
                                     static_cast<const double*>(weight), rows, cols, eps);
}

extern "C" int kd_standardize_rows_backward(int dtype, void* out, const void* x, const void* y, const void* grad,
                                            int64_t rows, int64_t cols, double eps) {
    if (int rc = check_rows(dtype, rows, cols)) return rc;
    if (rows == 0 || cols == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    if (dtype == KD_F32)
        return row_backward_typed<float, kStandardizeBack>(static_cast<float*>(out), static_cast<const float*>(x),
                                                          static_cast<const float*>(y), static_cast<const float*>(grad),
                                                          rows, cols, eps);
    return row_backward_typed<double, kStandardizeBack>(static_cast<double*>(out), static_cast<const double*>(x),
                                                       static_cast<const double*>(y), static_cast<const double*>(grad),
                                                       rows, cols, eps);
}
