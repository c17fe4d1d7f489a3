// kd_internal.h - shared pieces of the gfx950 backend: status/error plumbing, the backend
// stream, exact integer helpers, fast division and the element-op functors.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <type_traits>

#include "kd_api.h"

namespace kd {

// ---- status and errors ------------------------------------------------------------------

void set_error(const std::string& message);
int fail(int status, const std::string& message);
int hip_fail(hipError_t status, const char* call, const char* file, int line);

#define KD_HIP(call)                                                                         \
    do {                                                                                     \
        const hipError_t kd_status_ = (call);                                                \
        if (kd_status_ != hipSuccess) return ::kd::hip_fail(kd_status_, #call, __FILE__, __LINE__); \
    } while (0)

// Checks the launch that was just issued.
#define KD_LAUNCH_CHECK() KD_HIP(hipGetLastError())

// Probes the device once (gfx950 required); KD_OK when usable.
int ensure_device();
hipStream_t stream();
int device_ordinal();
int compute_units();

// A lease on the per-device workspace (scratch for split reductions and split-K partials,
// grown on demand, never shrunk). The lease holds the workspace lock from `workspace()` until
// it is destroyed, so a caller keeps it alive until every kernel that touches `ptr` has been
// enqueued: calls from several host threads then use the buffer one after another in stream
// order, and a growth (which frees the old block) never frees a block that a caller is about to
// hand to a kernel. When the backend stream differs from the one the previous lease used, the
// previous stream is drained first, so leases on different streams never overlap either.
struct Workspace {
    Workspace() = default;
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    ~Workspace();
    void* ptr = nullptr;
    bool held = false;
};
int workspace(Workspace& lease, size_t bytes);

// Split-K partial products for callers inside the library (the GPT-2 engine's prefill): with
// row-major A [M, K] (row stride lda) and B [K, N] (row stride ldb), parts[s][m][n] (row stride N,
// split stride M * N) is the product over K range [s * K / splits, (s + 1) * K / splits), on the
// 64x64 MFMA tiles, for s < splits. M and N multiples of 64, K a multiple of 32 * splits, lda and
// ldb multiples of 4 with 16-byte aligned operands; the caller adds the partials in split order.
int matmul_split_parts(const float* a, const float* b, float* parts, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, int64_t splits);

inline int64_t dtype_size(int dtype) {
    switch (dtype) {
    case KD_F32: return 4;
    case KD_F64: return 8;
    case KD_I64: return 8;
    case KD_BOOL: return 1;
    }
    return 0;
}

// ---- arithmetic rounded op by op -----------------------------------------------------------
//
// The compiler may contract a product and a following sum into one FMA, which rounds once;
// __fmul_rn / __fadd_rn do not prevent that on this target. Where a result must round as kael's
// separate element ops round it (each op rounded to the element type), these helpers are used:
// the pragma leaves their operations without the contraction flag, also after inlining.
template <typename T> __device__ __forceinline__ T mul_sep(T a, T b) {
#pragma clang fp contract(off)
    return a * b;
}
template <typename T> __device__ __forceinline__ T add_sep(T a, T b) {
#pragma clang fp contract(off)
    return a + b;
}
template <typename T> __device__ __forceinline__ T sub_sep(T a, T b) {
#pragma clang fp contract(off)
    return a - b;
}
template <typename T> __device__ __forceinline__ T div_sep(T a, T b) {
#pragma clang fp contract(off)
    return a / b;
}

// ---- exact integer arithmetic (reference src/internal/element_functions.h:45-119) --------

__host__ __device__ inline int64_t wrap_add(int64_t a, int64_t b) {
    return static_cast<int64_t>(static_cast<uint64_t>(a) + static_cast<uint64_t>(b));
}
__host__ __device__ inline int64_t wrap_sub(int64_t a, int64_t b) {
    return static_cast<int64_t>(static_cast<uint64_t>(a) - static_cast<uint64_t>(b));
}
__host__ __device__ inline int64_t wrap_mul(int64_t a, int64_t b) {
    return static_cast<int64_t>(static_cast<uint64_t>(a) * static_cast<uint64_t>(b));
}

// ---- fast unsigned division by a runtime constant --------------------------------------
//
// For a divisor 1 <= d < 2^31 choose s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1;
// then for every 0 <= n < 2^31, n / d = (n + mulhi32(n, m)) >> s (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, section 4).
struct FastDiv {
    uint32_t divisor;
    uint32_t multiplier;
    uint32_t shift;

    FastDiv() = default;
    explicit FastDiv(uint32_t d) : divisor(d), multiplier(0), shift(0) {
        while ((uint64_t{1} << shift) < d) ++shift;
        multiplier = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << shift) - d)) / d + 1);
    }
    __device__ inline uint32_t div(uint32_t n) const {
        const uint32_t hi = __umulhi(n, multiplier);
        return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> shift);
    }
};

// ---- element functors --------------------------------------------------------------------
//
// Each functor restates one reference functor of src/internal/element_functions.h with the
// same argument promotion, so bool (uint8) arithmetic promotes to int and is then
// normalised by the output cast, exactly as kernels.inl:5-13 does.

template <typename To, typename From> __device__ __forceinline__ To cast_value(From v) {
    if constexpr (std::is_same_v<To, uint8_t>) {
        return v != From(0) ? uint8_t{1} : uint8_t{0};
    } else if constexpr (std::is_integral_v<To> && std::is_floating_point_v<From>) {
        // saturating_cast: element_functions.h:76-90
        if (v != v) return To(0);
        if (v <= static_cast<From>(-9223372036854775808.0)) return INT64_MIN;
        if (v >= static_cast<From>(9223372036854775808.0)) return INT64_MAX;
        return static_cast<To>(v);
    } else {
        return static_cast<To>(v);
    }
}

template <typename T> __device__ __forceinline__ T max_na(T a, T b) {
    if constexpr (std::is_floating_point_v<T>) {
        if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    }
    return a < b ? b : a;
}
template <typename T> __device__ __forceinline__ T min_na(T a, T b) {
    if constexpr (std::is_floating_point_v<T>) {
        if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    }
    return b < a ? b : a;
}

__device__ inline int64_t int_power(int64_t base, int64_t exponent) {
    if (exponent < 0) {
        if (base == 1) return base;
        if (base == -1) return exponent % 2 == 0 ? 1 : base;
        return 0;
    }
    uint64_t result = 1;
    uint64_t factor = static_cast<uint64_t>(base);
    while (exponent > 0) {
        if (exponent % 2 == 1) result = result * factor;
        exponent /= 2;
        if (exponent > 0) factor = factor * factor;
    }
    return static_cast<int64_t>(result);
}

template <typename T> struct MathConst;
template <> struct MathConst<float> {
    static constexpr float sqrt2 = 1.41421356237309504880f;
    static constexpr float pi = 3.14159265358979323846f;
};
template <> struct MathConst<double> {
    static constexpr double sqrt2 = 1.41421356237309504880;
    static constexpr double pi = 3.14159265358979323846;
};

// Device math goes through ROCm's device library (ocml) via the HIP math headers.
template <typename T> __device__ __forceinline__ T d_exp(T x) { return std::exp(x); }
template <typename T> __device__ __forceinline__ T d_log(T x) { return std::log(x); }

// gelu_exact_slope / gelu_tanh_slope: reference src/autograd/functions_math.cpp:35-46.
template <typename T> __device__ __forceinline__ T gelu_slope(bool tanh_form, T x) {
    if (!tanh_form) {
        const T density = std::exp(-x * x / 2) / std::sqrt(2 * MathConst<T>::pi);
        return T(0.5) * (1 + std::erf(x / MathConst<T>::sqrt2)) + x * density;
    }
    const T scale = std::sqrt(2 / MathConst<T>::pi);
    const T c = T(0.044715);
    const T s = std::tanh(scale * (x + c * x * x * x));
    return T(0.5) * (1 + s) + T(0.5) * x * (1 - s * s) * scale * (1 + 3 * c * x * x);
}

// Op traits: inputs and output type for In = T (mirrors the dispatch of kernels.inl:333-424).
constexpr bool is_compare_op(int op) { return op >= KD_OP_EQUAL && op <= KD_OP_LOGICAL_XOR; }
constexpr bool is_floating_op(int op) {
    return (op >= KD_OP_EXP && op <= KD_OP_SIGMOID) || op == KD_OP_GELU_EXACT ||
           op == KD_OP_GELU_TANH || op == KD_OP_GELU_EXACT_BACKWARD ||
           op == KD_OP_GELU_TANH_BACKWARD;
}
constexpr int op_inputs(int op) {
    if (op <= KD_OP_LOGICAL_XOR) return 2;
    if (op == KD_OP_WHERE) return 3;
    if (op == KD_OP_MASKED_FILL || op == KD_OP_GELU_EXACT_BACKWARD ||
        op == KD_OP_GELU_TANH_BACKWARD)
        return 2;
    return 1;
}

template <int Op, typename T> struct OpOut { using type = T; };
template <int Op, typename T>
using op_out_t = std::conditional_t<is_compare_op(Op), uint8_t, T>;

// Scalar arguments of Clamp / MaskedFill (ElementParameters::get<T>, device_kernels.h:62-68).
template <typename T> struct Params {
    T p0;
    T p1;
    static Params make(const kd_element_parameters& p) {
        Params out;
        if constexpr (std::is_integral_v<T>) {
            out.p0 = static_cast<T>(p.integers[0]);
            out.p1 = static_cast<T>(p.integers[1]);
        } else {
            out.p0 = static_cast<T>(p.reals[0]);
            out.p1 = static_cast<T>(p.reals[1]);
        }
        return out;
    }
};

template <int Op, typename T>
__device__ __forceinline__ op_out_t<Op, T> apply_op(T a, T b, T c, const Params<T>& p) {
    using Out = op_out_t<Op, T>;
    constexpr bool wraps = std::is_same_v<T, int64_t>;
    constexpr bool is_bool = std::is_same_v<T, uint8_t>;
    (void)b;
    (void)c;
    (void)p;
    if constexpr (Op == KD_OP_PLUS) {
        if constexpr (wraps) return wrap_add(a, b);
        else return cast_value<Out>(a + b);
    } else if constexpr (Op == KD_OP_MINUS) {
        if constexpr (wraps) return wrap_sub(a, b);
        else return cast_value<Out>(a - b);
    } else if constexpr (Op == KD_OP_TIMES) {
        if constexpr (wraps) return wrap_mul(a, b);
        else return cast_value<Out>(a * b);
    } else if constexpr (Op == KD_OP_DIVIDES) {
        if constexpr (wraps) {
            // Undefined in the reference (the host traps); defined here as 0 and wrapping.
            if (b == 0) return int64_t{0};
            if (b == -1) return wrap_sub(0, a);
            return a / b;
        } else if constexpr (is_bool) {
            return cast_value<Out>(b == 0 ? 0 : int(a) / int(b));
        } else {
            return a / b;
        }
    } else if constexpr (Op == KD_OP_POWER) {
        if constexpr (std::is_floating_point_v<T>) return std::pow(a, b);
        else return static_cast<T>(int_power(a, b));
    } else if constexpr (Op == KD_OP_MAXIMUM) {
        return max_na(a, b);
    } else if constexpr (Op == KD_OP_MINIMUM) {
        return min_na(a, b);
    } else if constexpr (Op == KD_OP_EQUAL) {
        return a == b;
    } else if constexpr (Op == KD_OP_NOT_EQUAL) {
        return a != b;
    } else if constexpr (Op == KD_OP_LESS) {
        return a < b;
    } else if constexpr (Op == KD_OP_LESS_EQUAL) {
        return a <= b;
    } else if constexpr (Op == KD_OP_GREATER) {
        return a > b;
    } else if constexpr (Op == KD_OP_GREATER_EQUAL) {
        return a >= b;
    } else if constexpr (Op == KD_OP_LOGICAL_AND) {
        return a != T(0) && b != T(0);
    } else if constexpr (Op == KD_OP_LOGICAL_OR) {
        return a != T(0) || b != T(0);
    } else if constexpr (Op == KD_OP_LOGICAL_XOR) {
        return (a != T(0)) != (b != T(0));
    } else if constexpr (Op == KD_OP_IS_ZERO) {
        return cast_value<Out>(a == T(0));
    } else if constexpr (Op == KD_OP_NEGATE) {
        if constexpr (wraps) return wrap_sub(0, a);
        else if constexpr (is_bool) return cast_value<Out>(-int(a));
        else return -a;
    } else if constexpr (Op == KD_OP_ABSOLUTE) {
        if constexpr (is_bool) return a;
        else if constexpr (std::is_floating_point_v<T>) return std::fabs(a);
        else return a < 0 ? wrap_sub(0, a) : a;
    } else if constexpr (Op == KD_OP_SIGN) {
        if constexpr (is_bool) return a;
        else return static_cast<T>(a > T(0) ? 1 : (a < T(0) ? -1 : 0));
    } else if constexpr (Op == KD_OP_EXP) {
        return std::exp(a);
    } else if constexpr (Op == KD_OP_LOG) {
        return std::log(a);
    } else if constexpr (Op == KD_OP_LOG1P) {
        return std::log1p(a);
    } else if constexpr (Op == KD_OP_EXPM1) {
        return std::expm1(a);
    } else if constexpr (Op == KD_OP_SQRT) {
        return std::sqrt(a);
    } else if constexpr (Op == KD_OP_RSQRT) {
        return T(1) / std::sqrt(a);
    } else if constexpr (Op == KD_OP_SIN) {
        return std::sin(a);
    } else if constexpr (Op == KD_OP_COS) {
        return std::cos(a);
    } else if constexpr (Op == KD_OP_TANH) {
        return std::tanh(a);
    } else if constexpr (Op == KD_OP_SIGMOID) {
        if (a >= 0) return T(1) / (1 + std::exp(-a));
        const T e = std::exp(a);
        return e / (1 + e);
    } else if constexpr (Op == KD_OP_RELU) {
        return a < T(0) ? T(0) : a;
    } else if constexpr (Op == KD_OP_GELU_EXACT) {
        return T(0.5) * a * (1 + std::erf(a / MathConst<T>::sqrt2));
    } else if constexpr (Op == KD_OP_GELU_TANH) {
        const T scale = std::sqrt(2 / MathConst<T>::pi);
        return T(0.5) * a * (1 + std::tanh(scale * (a + T(0.044715) * a * a * a)));
    } else if constexpr (Op == KD_OP_CLAMP) {
        if constexpr (std::is_floating_point_v<T>) {
            if (isnan(p.p0) || isnan(p.p1)) return static_cast<T>(NAN);
        }
        const T raised = a < p.p0 ? p.p0 : a;
        return raised > p.p1 ? p.p1 : raised;
    } else if constexpr (Op == KD_OP_WHERE) {
        return a != T(0) ? b : c;
    } else if constexpr (Op == KD_OP_MASKED_FILL) {
        return b != T(0) ? p.p0 : a;
    } else if constexpr (Op == KD_OP_GELU_EXACT_BACKWARD) {
        return b * gelu_slope<T>(false, a);
    } else if constexpr (Op == KD_OP_GELU_TANH_BACKWARD) {
        return b * gelu_slope<T>(true, a);
    } else {
        return Out{};
    }
}

} // namespace kd
