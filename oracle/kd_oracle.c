/*
 * kd_oracle.c - TEST INFRASTRUCTURE ONLY: the checker, never the product.
 *
 * A plain-C CPU restatement of the reference device semantics (JetBerri/kael.cpp 1.0.1):
 *   - cast rules             src/cuda/kernels.inl:5-13, include/kael/dtype.h:130-155,
 *                            src/internal/element_functions.h:75-90
 *   - element ops (36)       src/internal/element_functions.h:27-323, dispatch kernels.inl:333-424
 *   - strided addressing     src/cuda/kernels.inl:15-28 (locate)
 *   - fill / convert         src/cuda/kernels.inl:53-57, 316-331
 *   - reduce                 src/cuda/kernels.inl:59-134, 278-307, 426-445
 *   - matmul                 src/cuda/kernels.inl:136-177
 *   - gather / scatter_add   src/cuda/kernels.inl:185-221, 447-465
 *   - row kernels            src/ops/nn.cpp:52-129, 214-240; src/nn/layers.cpp:60-68
 *   - GELU slopes            src/autograd/functions_math.cpp:35-46, 221-231
 *   - layout planning        src/iterator.cpp:12-63, 112-132, 152-172
 *   - host reductions        src/ops/reduce.cpp:24-83 (8 lanes, 16384-element blocks, pairwise
 *                            merge), :202-219 prod, :236-268 argmax/argmin, :285-295 all/any;
 *                            src/ops/sequence.cpp:95-117 cumsum (sequential, in the output dtype)
 *   - optimizer steps        src/optim/optimizer.cpp:60-80 SGD, :93-120 Adam / AdamW (the chain of
 *                            whole-tensor ops, each rounded to the element type)
 *   - random draws           src/random.cpp:66-84 rand (std::uniform_real_distribution<double> over
 *                            std::mt19937_64), :106-110 bernoulli; src/nn/functional.cpp:32-39
 *                            dropout. The engine is the C++ standard's mt19937_64 ([rand.predef])
 *                            in its sequential textbook form (Matsumoto & Nishimura); the draw is
 *                            libstdc++'s generate_canonical<double, 53> over a 64-bit engine.
 *
 * Deliberate choices where the reference is undefined: integer division by zero yields 0 and
 * INT64_MIN / -1 yields INT64_MIN (the reference host would trap). Floating ops on integer
 * dtypes, Max/Min of an empty chunk and bool scatter_add are errors (the reference host never
 * issues them).
 */
#include "kd_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static _Thread_local char g_error[256];

static int fail(const char* message) {
    snprintf(g_error, sizeof g_error, "%s", message);
    return KD_E_INVALID;
}

const char* oracle_last_error(void) { return g_error; }

typedef unsigned char u8;

/* ---- scalar helpers ----------------------------------------------------------------- */

/* wrapping_add / _subtract / _multiply: element_functions.h:48-73 */
static int64_t wadd(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
static int64_t wsub(int64_t a, int64_t b) { return (int64_t)((uint64_t)a - (uint64_t)b); }
static int64_t wmul(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }

/* saturating_cast<int64_t>: element_functions.h:76-90, dtype.h:132-144 */
static int64_t sat_i64(double v) {
    if (v != v) return 0;
    if (v <= -9223372036854775808.0) return INT64_MIN;
    if (v >= 9223372036854775808.0) return INT64_MAX;
    return (int64_t)v;
}

/* integer_power: element_functions.h:92-119 */
static int64_t ipow(int64_t base, int64_t exponent) {
    if (exponent < 0) {
        if (base == 1) return base;
        if (base == -1) return exponent % 2 == 0 ? 1 : base;
        return 0;
    }
    uint64_t result = 1, factor = (uint64_t)base;
    while (exponent > 0) {
        if (exponent % 2 == 1) result = result * factor;
        exponent /= 2;
        if (exponent > 0) factor = factor * factor;
    }
    return (int64_t)result;
}

static int64_t idiv(int64_t a, int64_t b) {
    if (b == 0) return 0;
    if (b == -1) return wsub(0, a);
    return a / b;
}

/* nan_aware_max / _min: element_functions.h:27-43 */
static double fmaxna(double a, double b) {
    if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    return a < b ? b : a;
}
static double fminna(double a, double b) {
    if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    return b < a ? b : a;
}
static float fmaxnaf(float a, float b) {
    if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    return a < b ? b : a;
}
static float fminnaf(float a, float b) {
    if (isnan(a) || isnan(b)) return isnan(a) ? a : b;
    return b < a ? b : a;
}

/* ---- element functors, evaluated per dtype ------------------------------------------ */

static const float kSqrt2F = 1.41421356237309504880f;
static const double kSqrt2 = 1.41421356237309504880;
static const float kPiF = 3.14159265358979323846f;
static const double kPi = 3.14159265358979323846;

/* Float unary ops (run_floating, kernels.inl:382-407) in float precision. */
static float unary_f32(int op, float x) {
    switch (op) {
    case KD_OP_EXP: return expf(x);
    case KD_OP_LOG: return logf(x);
    case KD_OP_LOG1P: return log1pf(x);
    case KD_OP_EXPM1: return expm1f(x);
    case KD_OP_SQRT: return sqrtf(x);
    case KD_OP_RSQRT: return 1 / sqrtf(x);
    case KD_OP_SIN: return sinf(x);
    case KD_OP_COS: return cosf(x);
    case KD_OP_TANH: return tanhf(x);
    case KD_OP_SIGMOID:
        if (x >= 0) return 1 / (1 + expf(-x));
        else {
            const float e = expf(x);
            return e / (1 + e);
        }
    case KD_OP_GELU_EXACT: return 0.5f * x * (1 + erff(x / kSqrt2F));
    case KD_OP_GELU_TANH: {
        const float scale = sqrtf(2 / kPiF);
        return 0.5f * x * (1 + tanhf(scale * (x + 0.044715f * x * x * x)));
    }
    }
    return 0.0f;
}

static double unary_f64(int op, double x) {
    switch (op) {
    case KD_OP_EXP: return exp(x);
    case KD_OP_LOG: return log(x);
    case KD_OP_LOG1P: return log1p(x);
    case KD_OP_EXPM1: return expm1(x);
    case KD_OP_SQRT: return sqrt(x);
    case KD_OP_RSQRT: return 1 / sqrt(x);
    case KD_OP_SIN: return sin(x);
    case KD_OP_COS: return cos(x);
    case KD_OP_TANH: return tanh(x);
    case KD_OP_SIGMOID:
        if (x >= 0) return 1 / (1 + exp(-x));
        else {
            const double e = exp(x);
            return e / (1 + e);
        }
    case KD_OP_GELU_EXACT: return 0.5 * x * (1 + erf(x / kSqrt2));
    case KD_OP_GELU_TANH: {
        const double scale = sqrt(2 / kPi);
        return 0.5 * x * (1 + tanh(scale * (x + 0.044715 * x * x * x)));
    }
    }
    return 0.0;
}

/* gelu_exact_slope / gelu_tanh_slope: functions_math.cpp:35-46 */
static float gelu_slope_f32(int tanh_form, float x) {
    if (!tanh_form) {
        const float density = expf(-x * x / 2) / sqrtf(2 * kPiF);
        return 0.5f * (1 + erff(x / kSqrt2F)) + x * density;
    }
    const float scale = sqrtf(2 / kPiF);
    const float c = 0.044715f;
    const float s = tanhf(scale * (x + c * x * x * x));
    return 0.5f * (1 + s) + 0.5f * x * (1 - s * s) * scale * (1 + 3 * c * x * x);
}

static double gelu_slope_f64(int tanh_form, double x) {
    if (!tanh_form) {
        const double density = exp(-x * x / 2) / sqrt(2 * kPi);
        return 0.5 * (1 + erf(x / kSqrt2)) + x * density;
    }
    const double scale = sqrt(2 / kPi);
    const double c = 0.044715;
    const double s = tanh(scale * (x + c * x * x * x));
    return 0.5 * (1 + s) + 0.5 * x * (1 - s * s) * scale * (1 + 3 * c * x * x);
}

static int is_compare(int op) { return op >= KD_OP_EQUAL && op <= KD_OP_LOGICAL_XOR; }
static int is_floating_only(int op) {
    return (op >= KD_OP_EXP && op <= KD_OP_SIGMOID) || op == KD_OP_GELU_EXACT ||
           op == KD_OP_GELU_TANH || op == KD_OP_GELU_EXACT_BACKWARD ||
           op == KD_OP_GELU_TANH_BACKWARD;
}
static int input_count(int op) {
    if (op <= KD_OP_LOGICAL_XOR) return 2;
    if (op == KD_OP_WHERE) return 3;
    if (op == KD_OP_MASKED_FILL || op == KD_OP_GELU_EXACT_BACKWARD ||
        op == KD_OP_GELU_TANH_BACKWARD)
        return 2;
    return 1;
}

/* Comparison (run_compare, kernels.inl:270-276): the functor returns bool. */
#define COMPARE_BODY(a, b)                                                                   \
    switch (op) {                                                                            \
    case KD_OP_EQUAL: return (a) == (b);                                                     \
    case KD_OP_NOT_EQUAL: return (a) != (b);                                                 \
    case KD_OP_LESS: return (a) < (b);                                                       \
    case KD_OP_LESS_EQUAL: return (a) <= (b);                                                \
    case KD_OP_GREATER: return (a) > (b);                                                    \
    case KD_OP_GREATER_EQUAL: return (a) >= (b);                                             \
    case KD_OP_LOGICAL_AND: return (a) != 0 && (b) != 0;                                     \
    case KD_OP_LOGICAL_OR: return (a) != 0 || (b) != 0;                                      \
    case KD_OP_LOGICAL_XOR: return ((a) != 0) != ((b) != 0);                                 \
    }                                                                                        \
    return 0;

static u8 compare_f32(int op, float a, float b) { COMPARE_BODY(a, b) }
static u8 compare_f64(int op, double a, double b) { COMPARE_BODY(a, b) }
static u8 compare_i64(int op, int64_t a, int64_t b) { COMPARE_BODY(a, b) }
static u8 compare_u8(int op, u8 a, u8 b) { COMPARE_BODY(a, b) }

/* Same-dtype ops on float (run_same, kernels.inl:254-260 + functors). */
static float same_f32(int op, const float* in, const kd_element_parameters* p) {
    const float x = in[0];
    switch (op) {
    case KD_OP_PLUS: return in[0] + in[1];
    case KD_OP_MINUS: return in[0] - in[1];
    case KD_OP_TIMES: return in[0] * in[1];
    case KD_OP_DIVIDES: return in[0] / in[1];
    case KD_OP_POWER: return powf(in[0], in[1]);
    case KD_OP_MAXIMUM: return fmaxnaf(in[0], in[1]);
    case KD_OP_MINIMUM: return fminnaf(in[0], in[1]);
    case KD_OP_IS_ZERO: return x == 0.0f ? 1.0f : 0.0f;
    case KD_OP_NEGATE: return -x;
    case KD_OP_ABSOLUTE: return fabsf(x);
    case KD_OP_SIGN: return (float)(x > 0 ? 1 : (x < 0 ? -1 : 0));
    case KD_OP_RELU: return x < 0 ? 0.0f : x;
    case KD_OP_CLAMP: {
        const float low = (float)p->reals[0], high = (float)p->reals[1];
        if (isnan(low) || isnan(high)) return NAN;
        const float raised = x < low ? low : x;
        return raised > high ? high : raised;
    }
    case KD_OP_WHERE: return in[0] != 0 ? in[1] : in[2];
    case KD_OP_MASKED_FILL: return in[1] != 0 ? (float)p->reals[0] : in[0];
    case KD_OP_GELU_EXACT_BACKWARD: return in[1] * gelu_slope_f32(0, in[0]);
    case KD_OP_GELU_TANH_BACKWARD: return in[1] * gelu_slope_f32(1, in[0]);
    }
    return unary_f32(op, x);
}

static double same_f64(int op, const double* in, const kd_element_parameters* p) {
    const double x = in[0];
    switch (op) {
    case KD_OP_PLUS: return in[0] + in[1];
    case KD_OP_MINUS: return in[0] - in[1];
    case KD_OP_TIMES: return in[0] * in[1];
    case KD_OP_DIVIDES: return in[0] / in[1];
    case KD_OP_POWER: return pow(in[0], in[1]);
    case KD_OP_MAXIMUM: return fmaxna(in[0], in[1]);
    case KD_OP_MINIMUM: return fminna(in[0], in[1]);
    case KD_OP_IS_ZERO: return x == 0.0 ? 1.0 : 0.0;
    case KD_OP_NEGATE: return -x;
    case KD_OP_ABSOLUTE: return fabs(x);
    case KD_OP_SIGN: return (double)(x > 0 ? 1 : (x < 0 ? -1 : 0));
    case KD_OP_RELU: return x < 0 ? 0.0 : x;
    case KD_OP_CLAMP: {
        const double low = p->reals[0], high = p->reals[1];
        if (isnan(low) || isnan(high)) return NAN;
        const double raised = x < low ? low : x;
        return raised > high ? high : raised;
    }
    case KD_OP_WHERE: return in[0] != 0 ? in[1] : in[2];
    case KD_OP_MASKED_FILL: return in[1] != 0 ? p->reals[0] : in[0];
    case KD_OP_GELU_EXACT_BACKWARD: return in[1] * gelu_slope_f64(0, in[0]);
    case KD_OP_GELU_TANH_BACKWARD: return in[1] * gelu_slope_f64(1, in[0]);
    }
    return unary_f64(op, x);
}

static int64_t same_i64(int op, const int64_t* in, const kd_element_parameters* p) {
    const int64_t x = in[0];
    switch (op) {
    case KD_OP_PLUS: return wadd(in[0], in[1]);
    case KD_OP_MINUS: return wsub(in[0], in[1]);
    case KD_OP_TIMES: return wmul(in[0], in[1]);
    case KD_OP_DIVIDES: return idiv(in[0], in[1]);
    case KD_OP_POWER: return ipow(in[0], in[1]);
    case KD_OP_MAXIMUM: return in[0] < in[1] ? in[1] : in[0];
    case KD_OP_MINIMUM: return in[1] < in[0] ? in[1] : in[0];
    case KD_OP_IS_ZERO: return x == 0;
    case KD_OP_NEGATE: return wsub(0, x);
    case KD_OP_ABSOLUTE: return x < 0 ? wsub(0, x) : x;
    case KD_OP_SIGN: return x > 0 ? 1 : (x < 0 ? -1 : 0);
    case KD_OP_RELU: return x < 0 ? 0 : x;
    case KD_OP_CLAMP: {
        const int64_t low = p->integers[0], high = p->integers[1];
        const int64_t raised = x < low ? low : x;
        return raised > high ? high : raised;
    }
    case KD_OP_WHERE: return in[0] != 0 ? in[1] : in[2];
    case KD_OP_MASKED_FILL: return in[1] != 0 ? p->integers[0] : in[0];
    }
    return 0;
}

/* bool (uint8) arithmetic: operands promote to int and the result is normalised
 * by cast_value<uint8_t> (kernels.inl:6-7). */
static u8 same_u8(int op, const u8* in, const kd_element_parameters* p) {
    const int a = in[0];
    int r = 0;
    switch (op) {
    case KD_OP_PLUS: r = in[0] + in[1]; break;
    case KD_OP_MINUS: r = in[0] - in[1]; break;
    case KD_OP_TIMES: r = in[0] * in[1]; break;
    case KD_OP_DIVIDES: r = in[1] == 0 ? 0 : in[0] / in[1]; break;
    case KD_OP_MAXIMUM: r = in[0] < in[1] ? in[1] : in[0]; break;
    case KD_OP_MINIMUM: r = in[1] < in[0] ? in[1] : in[0]; break;
    case KD_OP_IS_ZERO: r = a == 0; break;
    case KD_OP_NEGATE: r = -a; break;
    case KD_OP_ABSOLUTE: r = a; break;
    case KD_OP_SIGN: r = a; break;
    case KD_OP_RELU: r = a; break;
    case KD_OP_CLAMP: {
        const u8 low = (u8)p->integers[0], high = (u8)p->integers[1];
        const u8 raised = in[0] < low ? low : in[0];
        r = raised > high ? high : raised;
        break;
    }
    case KD_OP_WHERE: r = in[0] != 0 ? in[1] : in[2]; break;
    case KD_OP_MASKED_FILL: r = in[1] != 0 ? (u8)p->integers[0] : in[0]; break;
    }
    return r != 0;
}

/* ---- layouts -------------------------------------------------------------------------- */

static int64_t dtype_size(int dtype) {
    switch (dtype) {
    case KD_F32: return 4;
    case KD_F64: return 8;
    case KD_I64: return 8;
    case KD_BOOL: return 1;
    }
    return 0;
}

/* locate: kernels.inl:15-28 */
static void locate(const kd_element_layout* l, int64_t element, char** pointers) {
    int64_t offsets[KD_MAX_OPERANDS] = {0, 0, 0, 0};
    int64_t remaining = element;
    for (int dim = l->dims - 1; dim >= 0; --dim) {
        const int64_t position = remaining % l->shape[dim];
        remaining /= l->shape[dim];
        for (int op = 0; op < l->operands; ++op) offsets[op] += position * l->strides[op][dim];
    }
    for (int op = 0; op < l->operands; ++op) pointers[op] = (char*)l->base[op] + offsets[op];
}

static int check_layout(const kd_element_layout* l, int operands) {
    if (l->dims < 1 || l->dims > KD_MAX_DIMS) return fail("layout dims out of range");
    if (l->operands != operands) return fail("layout operand count does not match the op");
    return KD_OK;
}

static double read_as_double(int dtype, const char* p) {
    switch (dtype) {
    case KD_F32: return *(const float*)p;
    case KD_F64: return *(const double*)p;
    case KD_I64: return (double)*(const int64_t*)p;
    default: return *(const u8*)p;
    }
}

/* cast_value<Out, In>: kernels.inl:5-13 */
static void store_cast(int out_dtype, char* dst, int in_dtype, const char* src) {
    if (out_dtype == KD_BOOL) {
        *(u8*)dst = read_as_double(in_dtype, src) != 0.0 ||
                    (in_dtype == KD_I64 && *(const int64_t*)src != 0);
        return;
    }
    if (out_dtype == KD_I64) {
        if (in_dtype == KD_F32) *(int64_t*)dst = sat_i64(*(const float*)src);
        else if (in_dtype == KD_F64) *(int64_t*)dst = sat_i64(*(const double*)src);
        else if (in_dtype == KD_I64) *(int64_t*)dst = *(const int64_t*)src;
        else *(int64_t*)dst = *(const u8*)src;
        return;
    }
    if (out_dtype == KD_F32) {
        if (in_dtype == KD_I64) *(float*)dst = (float)*(const int64_t*)src;
        else if (in_dtype == KD_F64) *(float*)dst = (float)*(const double*)src;
        else *(float*)dst = (float)read_as_double(in_dtype, src);
        return;
    }
    if (in_dtype == KD_I64) *(double*)dst = (double)*(const int64_t*)src;
    else *(double*)dst = read_as_double(in_dtype, src);
}

int oracle_fill(int dtype, void* target, int64_t count, const void* value) {
    const int64_t size = dtype_size(dtype);
    if (size == 0) return fail("fill: unknown dtype");
    for (int64_t i = 0; i < count; ++i) memcpy((char*)target + i * size, value, (size_t)size);
    return KD_OK;
}

int oracle_convert(int out_dtype, int in_dtype, const kd_element_layout* l) {
    if (dtype_size(out_dtype) == 0 || dtype_size(in_dtype) == 0) return fail("convert: dtype");
    if (l->count == 0) return KD_OK;
    if (check_layout(l, 2)) return KD_E_INVALID;
    for (int64_t e = l->count; e-- > 0;) {
        char* ptr[KD_MAX_OPERANDS];
        locate(l, e, ptr);
        store_cast(out_dtype, ptr[0], in_dtype, ptr[1]);
    }
    return KD_OK;
}

int oracle_elementwise(int op, int out_dtype, int in_dtype, const kd_element_layout* l,
                       kd_element_parameters p) {
    (void)out_dtype; /* implied by the op, as at kernels.inl:335 */
    const int valid_op = (op >= KD_OP_PLUS && op <= KD_OP_MASKED_FILL) ||
                         op == KD_OP_GELU_EXACT_BACKWARD || op == KD_OP_GELU_TANH_BACKWARD;
    if (!valid_op) return fail("elementwise: unknown op");
    if (dtype_size(in_dtype) == 0) return fail("elementwise: unknown dtype");
    if (is_floating_only(op) && in_dtype != KD_F32 && in_dtype != KD_F64)
        return fail("elementwise: floating op on a non-floating dtype");
    if (op == KD_OP_POWER && in_dtype == KD_BOOL) return KD_OK; /* kernels.inl:345-351 */
    if (l->count == 0) return KD_OK;
    const int inputs = input_count(op);
    if (check_layout(l, inputs + 1)) return KD_E_INVALID;
    for (int64_t e = l->count; e-- > 0;) {
        char* ptr[KD_MAX_OPERANDS];
        locate(l, e, ptr);
        if (is_compare(op)) {
            u8 r = 0;
            switch (in_dtype) {
            case KD_F32: r = compare_f32(op, *(float*)ptr[1], *(float*)ptr[2]); break;
            case KD_F64: r = compare_f64(op, *(double*)ptr[1], *(double*)ptr[2]); break;
            case KD_I64: r = compare_i64(op, *(int64_t*)ptr[1], *(int64_t*)ptr[2]); break;
            default: r = compare_u8(op, *(u8*)ptr[1], *(u8*)ptr[2]); break;
            }
            *(u8*)ptr[0] = r;
            continue;
        }
        switch (in_dtype) {
        case KD_F32: {
            float in[3];
            for (int i = 0; i < inputs; ++i) in[i] = *(float*)ptr[i + 1];
            *(float*)ptr[0] = same_f32(op, in, &p);
            break;
        }
        case KD_F64: {
            double in[3];
            for (int i = 0; i < inputs; ++i) in[i] = *(double*)ptr[i + 1];
            *(double*)ptr[0] = same_f64(op, in, &p);
            break;
        }
        case KD_I64: {
            int64_t in[3];
            for (int i = 0; i < inputs; ++i) in[i] = *(int64_t*)ptr[i + 1];
            *(int64_t*)ptr[0] = same_i64(op, in, &p);
            break;
        }
        default: {
            u8 in[3];
            for (int i = 0; i < inputs; ++i) in[i] = *(u8*)ptr[i + 1];
            *(u8*)ptr[0] = same_u8(op, in, &p);
            break;
        }
        }
    }
    return KD_OK;
}

/* ---- reduce: kernels.inl:59-134, 278-307, 426-445 ----------------------------------------- */

#define KBLOCK 4096

static double reduce_range_f(int op, int in_dtype, const char* data, int64_t begin, int64_t end) {
    const int64_t size = dtype_size(in_dtype);
    if (op == KD_REDUCE_SUM) {
        double total = 0.0;
        for (int64_t i = begin; i < end; ++i) total += read_as_double(in_dtype, data + i * size);
        return total;
    }
    if (in_dtype == KD_F32) {
        const float* d = (const float*)data;
        float best = d[begin];
        for (int64_t i = begin + 1; i < end; ++i)
            best = op == KD_REDUCE_MAX ? fmaxnaf(best, d[i]) : fminnaf(best, d[i]);
        return best;
    }
    const double* d = (const double*)data;
    double best = d[begin];
    for (int64_t i = begin + 1; i < end; ++i)
        best = op == KD_REDUCE_MAX ? fmaxna(best, d[i]) : fminna(best, d[i]);
    return best;
}

static int64_t reduce_range_i(int op, int in_dtype, const char* data, int64_t begin, int64_t end) {
    const int64_t* d64 = (const int64_t*)data;
    const u8* d8 = (const u8*)data;
    const int wide = in_dtype == KD_I64;
    if (op == KD_REDUCE_SUM) {
        int64_t total = 0;
        for (int64_t i = begin; i < end; ++i) total = wadd(total, wide ? d64[i] : d8[i]);
        return total;
    }
    int64_t best = wide ? d64[begin] : d8[begin];
    for (int64_t i = begin + 1; i < end; ++i) {
        const int64_t v = wide ? d64[i] : d8[i];
        if (op == KD_REDUCE_MAX) best = best < v ? v : best;
        else best = v < best ? v : best;
    }
    return best;
}

/* ---- reductions kael runs on the host: prod, all / any, argmax / argmin, cumsum --------- */

#define CPU_BLOCK 16384 /* kReductionBlock, reduce.cpp:24 */
#define CPU_LANES 8     /* kLanes, reduce.cpp:25 */

/* fold_lanes (reduce.cpp:35-56) of the product over [first, last): double for floats. */
static double prod_lanes_f(int in_dtype, const char* row, int64_t first, int64_t last) {
    double lanes[CPU_LANES];
    for (int l = 0; l < CPU_LANES; ++l) lanes[l] = 1.0;
    int64_t i = first;
    for (; i + CPU_LANES <= last; i += CPU_LANES)
        for (int l = 0; l < CPU_LANES; ++l) lanes[l] = lanes[l] * read_as_double(in_dtype, row + (i + l) * dtype_size(in_dtype));
    double total = 1.0;
    for (int l = 0; l < CPU_LANES; ++l) total = total * lanes[l];
    for (; i < last; ++i) total = total * read_as_double(in_dtype, row + i * dtype_size(in_dtype));
    return total;
}

static int64_t read_as_i64(int in_dtype, const char* p) {
    if (in_dtype == KD_I64) {
        int64_t v;
        memcpy(&v, p, 8);
        return v;
    }
    return (int64_t)*(const u8*)p;
}

/* The same for integers: wrapping int64 products (element_functions.h:66-73). */
static int64_t prod_lanes_i(int in_dtype, const char* row, int64_t first, int64_t last) {
    int64_t lanes[CPU_LANES];
    for (int l = 0; l < CPU_LANES; ++l) lanes[l] = 1;
    int64_t i = first;
    for (; i + CPU_LANES <= last; i += CPU_LANES)
        for (int l = 0; l < CPU_LANES; ++l) lanes[l] = wmul(lanes[l], read_as_i64(in_dtype, row + (i + l) * dtype_size(in_dtype)));
    int64_t total = 1;
    for (int l = 0; l < CPU_LANES; ++l) total = wmul(total, lanes[l]);
    for (; i < last; ++i) total = wmul(total, read_as_i64(in_dtype, row + i * dtype_size(in_dtype)));
    return total;
}

/* reduce_in_blocks (reduce.cpp:58-83) of the product of one chunk. */
static int prod_chunk(int in_dtype, const char* row, int64_t size, double* fv, int64_t* iv) {
    const int floating = in_dtype == KD_F32 || in_dtype == KD_F64;
    if (size <= CPU_BLOCK) {
        if (floating) *fv = 1.0 * prod_lanes_f(in_dtype, row, 0, size);
        else *iv = wmul(1, prod_lanes_i(in_dtype, row, 0, size));
        return KD_OK;
    }
    const int64_t blocks = (size + CPU_BLOCK - 1) / CPU_BLOCK;
    double* fp = (double*)malloc((size_t)blocks * sizeof(double));
    int64_t* ip = (int64_t*)malloc((size_t)blocks * sizeof(int64_t));
    if (!fp || !ip) {
        free(fp);
        free(ip);
        return fail("prod: out of memory");
    }
    for (int64_t b = 0; b < blocks; ++b) {
        const int64_t begin = b * CPU_BLOCK;
        const int64_t end = begin + CPU_BLOCK < size ? begin + CPU_BLOCK : size;
        if (floating) fp[b] = prod_lanes_f(in_dtype, row, begin, end);
        else ip[b] = prod_lanes_i(in_dtype, row, begin, end);
    }
    for (int64_t width = blocks; width > 1; width = (width + 1) / 2) {
        for (int64_t i = 0; i < width / 2; ++i) {
            if (floating) fp[i] = fp[2 * i] * fp[2 * i + 1];
            else ip[i] = wmul(ip[2 * i], ip[2 * i + 1]);
        }
        if (width % 2 == 1) {
            if (floating) fp[width / 2] = fp[width - 1];
            else ip[width / 2] = ip[width - 1];
        }
    }
    if (floating) *fv = 1.0 * fp[0];
    else *iv = wmul(1, ip[0]);
    free(fp);
    free(ip);
    return KD_OK;
}

static int host_reduce(int op, int in_dtype, void* results, const void* data, int64_t chunk, int64_t rows) {
    const int64_t esize = dtype_size(in_dtype);
    for (int64_t r = 0; r < rows; ++r) {
        const char* row = (const char*)data + r * chunk * esize;
        if (op == KD_REDUCE_PROD) {
            double fv = 0;
            int64_t iv = 0;
            if (prod_chunk(in_dtype, row, chunk, &fv, &iv) != KD_OK) return KD_E_INVALID;
            if (in_dtype == KD_F32) ((float*)results)[r] = (float)fv;
            else if (in_dtype == KD_F64) ((double*)results)[r] = fv;
            else ((int64_t*)results)[r] = iv;
        } else {
            /* all / any: the first zero (all) or nonzero (any) decides; NaN != 0 (reduce.cpp:295) */
            u8 v = op == KD_REDUCE_ALL ? 1 : 0;
            for (int64_t i = 0; i < chunk; ++i) {
                const int nonzero = read_as_double(in_dtype, row + i * esize) != 0.0 ||
                                    (in_dtype == KD_I64 && read_as_i64(in_dtype, row + i * esize) != 0);
                if (op == KD_REDUCE_ALL && !nonzero) {
                    v = 0;
                    break;
                }
                if (op == KD_REDUCE_ANY && nonzero) {
                    v = 1;
                    break;
                }
            }
            ((u8*)results)[r] = v;
        }
    }
    return KD_OK;
}

/* best_position (reduce.cpp:236-254) with std::greater (argmax) or std::less (argmin). */
int oracle_arg_reduce(int largest, int in_dtype, int64_t* results, const void* data, int64_t chunk,
                      int64_t rows) {
    if (dtype_size(in_dtype) == 0) return fail("arg_reduce: unknown dtype");
    if (chunk < 0 || rows < 0) return fail("arg_reduce: negative size");
    if (rows == 0) return KD_OK;
    if (chunk == 0) return fail("arg_reduce: argmax/argmin of an empty chunk");
    const int64_t esize = dtype_size(in_dtype);
    const int floating = in_dtype == KD_F32 || in_dtype == KD_F64;
    for (int64_t r = 0; r < rows; ++r) {
        const char* row = (const char*)data + r * chunk * esize;
        int64_t best = 0;
        for (int64_t i = 1; i < chunk; ++i) {
            if (floating) {
                const double b = read_as_double(in_dtype, row + best * esize);
                const double c = read_as_double(in_dtype, row + i * esize);
                if (b != b) break;
                if (c != c) {
                    best = i;
                    continue;
                }
                if (largest ? c > b : c < b) best = i;
            } else {
                const int64_t b = read_as_i64(in_dtype, row + best * esize);
                const int64_t c = read_as_i64(in_dtype, row + i * esize);
                if (largest ? c > b : c < b) best = i;
            }
        }
        results[r] = best;
    }
    return KD_OK;
}

/* cumsum (sequence.cpp:95-117): the input converted to the output dtype (In for floats, I64
 * otherwise), then results[i] = results[i-1] + data[i] in that dtype (wrapping for I64). */
int oracle_cumsum(int in_dtype, void* out, const void* in, int64_t size, int64_t rows) {
    if (dtype_size(in_dtype) == 0) return fail("cumsum: unknown dtype");
    if (size < 0 || rows < 0) return fail("cumsum: negative size");
    const int64_t esize = dtype_size(in_dtype);
    for (int64_t r = 0; r < rows; ++r) {
        const char* row = (const char*)in + r * size * esize;
        if (in_dtype == KD_F32) {
            float* o = (float*)out + r * size;
            for (int64_t i = 0; i < size; ++i) o[i] = i == 0 ? ((const float*)row)[0] : o[i - 1] + ((const float*)row)[i];
        } else if (in_dtype == KD_F64) {
            double* o = (double*)out + r * size;
            for (int64_t i = 0; i < size; ++i) o[i] = i == 0 ? ((const double*)row)[0] : o[i - 1] + ((const double*)row)[i];
        } else {
            int64_t* o = (int64_t*)out + r * size;
            for (int64_t i = 0; i < size; ++i) {
                const int64_t v = read_as_i64(in_dtype, row + i * esize);
                o[i] = i == 0 ? v : wadd(o[i - 1], v);
            }
        }
    }
    return KD_OK;
}

int oracle_reduce(int op, int out_dtype, int in_dtype, void* results, const void* data,
                  int64_t chunk, int64_t rows) {
    (void)out_dtype;
    if (op == KD_REDUCE_PROD || op == KD_REDUCE_ALL || op == KD_REDUCE_ANY) {
        if (dtype_size(in_dtype) == 0) return fail("reduce: unknown dtype");
        if (chunk < 0 || rows < 0) return fail("reduce: negative size");
        return host_reduce(op, in_dtype, results, data, chunk, rows);
    }
    if (op < KD_REDUCE_SUM || op > KD_REDUCE_MIN) return fail("reduce: unknown op");
    if (dtype_size(in_dtype) == 0) return fail("reduce: unknown dtype");
    if (rows == 0) return KD_OK;
    if (chunk == 0 && op != KD_REDUCE_SUM) return fail("reduce: max/min of an empty chunk");
    const int floating = in_dtype == KD_F32 || in_dtype == KD_F64;
    const int64_t esize = dtype_size(in_dtype);
    const int64_t blocks = chunk <= KBLOCK ? 1 : (chunk + KBLOCK - 1) / KBLOCK;
    double* fpart = (double*)malloc((size_t)(2 * blocks) * sizeof(double));
    int64_t* ipart = (int64_t*)malloc((size_t)(2 * blocks) * sizeof(int64_t));
    for (int64_t r = 0; r < rows; ++r) {
        const char* row = (const char*)data + r * chunk * esize;
        double fv;
        int64_t iv;
        if (chunk <= KBLOCK) {
            fv = floating ? reduce_range_f(op, in_dtype, row, 0, chunk) : 0;
            iv = floating ? 0 : reduce_range_i(op, in_dtype, row, 0, chunk);
        } else {
            /* ReduceBlocks then the MergePairs tree, kernels.inl:108-128, 286-303 */
            double* fs = fpart;
            double* ft = fpart + blocks;
            int64_t* is = ipart;
            int64_t* it = ipart + blocks;
            for (int64_t b = 0; b < blocks; ++b) {
                const int64_t begin = b * KBLOCK;
                const int64_t end = begin + KBLOCK < chunk ? begin + KBLOCK : chunk;
                if (floating) fs[b] = reduce_range_f(op, in_dtype, row, begin, end);
                else is[b] = reduce_range_i(op, in_dtype, row, begin, end);
            }
            for (int64_t width = blocks; width > 1; width = (width + 1) / 2) {
                for (int64_t i = 0; i < (width + 1) / 2; ++i) {
                    if (2 * i + 1 < width) {
                        if (floating) {
                            const double a = fs[2 * i], b = fs[2 * i + 1];
                            ft[i] = op == KD_REDUCE_SUM ? a + b
                                    : op == KD_REDUCE_MAX ? (in_dtype == KD_F32 ? fmaxnaf((float)a, (float)b) : fmaxna(a, b))
                                                          : (in_dtype == KD_F32 ? fminnaf((float)a, (float)b) : fminna(a, b));
                        } else {
                            const int64_t a = is[2 * i], b = is[2 * i + 1];
                            it[i] = op == KD_REDUCE_SUM ? wadd(a, b)
                                    : op == KD_REDUCE_MAX ? (a < b ? b : a)
                                                          : (b < a ? b : a);
                        }
                    } else {
                        if (floating) ft[i] = fs[2 * i];
                        else it[i] = is[2 * i];
                    }
                }
                double* ftmp = fs; fs = ft; ft = ftmp;
                int64_t* itmp = is; is = it; it = itmp;
            }
            fv = fs[0];
            iv = is[0];
        }
        if (floating) {
            if (in_dtype == KD_F32) ((float*)results)[r] = (float)fv;
            else ((double*)results)[r] = fv;
        } else if (op == KD_REDUCE_SUM || in_dtype == KD_I64) {
            ((int64_t*)results)[r] = iv;
        } else {
            ((u8*)results)[r] = (u8)iv;
        }
    }
    free(fpart);
    free(ipart);
    return KD_OK;
}

/* kd_reduce_columns: column j of the [outer, inner] matrix copied out and reduced as one chunk by
 * oracle_reduce, exactly as kael's plan_reduction copy followed by device::reduce computes it
 * (reference src/ops/reduce.cpp:118-153, 309-314). */
int oracle_reduce_columns(int op, int out_dtype, int in_dtype, void* results, const void* data,
                          int64_t outer, int64_t inner) {
    if (outer < 0 || inner < 0) return fail("reduce_columns: negative size");
    const int64_t esize = dtype_size(in_dtype);
    if (esize == 0) return fail("reduce_columns: unknown dtype");
    if (inner == 0) return KD_OK;
    const int64_t osize = dtype_size(op == KD_REDUCE_ALL || op == KD_REDUCE_ANY ? KD_BOOL
                                     : (op == KD_REDUCE_SUM || op == KD_REDUCE_PROD) && in_dtype != KD_F32 && in_dtype != KD_F64
                                         ? KD_I64 : in_dtype);
    char* column = (char*)malloc((size_t)(outer > 0 ? outer : 1) * (size_t)esize);
    int rc = KD_OK;
    for (int64_t j = 0; j < inner && rc == KD_OK; ++j) {
        for (int64_t i = 0; i < outer; ++i)
            memcpy(column + i * esize, (const char*)data + (i * inner + j) * esize, (size_t)esize);
        rc = oracle_reduce(op, out_dtype, in_dtype, (char*)results + j * osize, column, outer, 1);
    }
    free(column);
    return rc;
}

/* kd_index_bounds: bounds[0] = min, bounds[1] = max of indices[i * stride], i < count: the two
 * reductions kael reads back before a device gather / scatter_add (reference
 * src/internal/index_checks.h:37-43: max(indices).item(), min(indices).item()) and on
 * cross-entropy targets (src/ops/nn.cpp:97-98, src/nn/loss.cpp:27-28). */
int oracle_index_bounds(const int64_t* indices, int64_t count, int64_t stride, int64_t* bounds) {
    if (indices == NULL || bounds == NULL || count <= 0) return fail("index_bounds: needs indices and count > 0");
    int64_t lo = indices[0], hi = indices[0];
    for (int64_t i = 1; i < count; ++i) {
        const int64_t v = indices[i * stride];
        if (v < lo) lo = v;
        if (v > hi) hi = v;
    }
    bounds[0] = lo;
    bounds[1] = hi;
    return KD_OK;
}

/* ---- causal self-attention: kael's composed chain -------------------------------------------
 *
 * kael's CausalSelfAttention::forward without a cache or dropout (reference
 * src/nn/transformer.cpp:114-136), each op as kael's device path computes it, per (batch, head):
 * Q, K, V = the head's rows of the fused projection qkv [B, T, 3, H, D] (select + transpose);
 * S = Q . K^T (oracle_matmul, the device kernel's order); S / sqrt(D) rounded to f32 (the scalar
 * division); masked_fill of key > query with -inf (the triu(ones, 1) mask, :25-27); softmax rows
 * (oracle_softmax_rows); O = P . V; out[b, t, h, :] = O[t] (transpose(1, 2).contiguous()). lse
 * is the log-sum-exp of each scaled, masked row in double (not a kael value: the input of the
 * fused backward, which recomputes P from it). The backward restates kael's autograd for the
 * same chain: MatmulBackward of O = P . V (dP = dO . V^T, dV = P^T . dO), SoftmaxBackward
 * (oracle_softmax_rows_backward), MaskedFillBackward (masked -> 0), the division's backward
 * (dS / sqrt(D)), MatmulBackward of S = Q . K^T (dQ = dS . K, dK = dS^T . Q), and the select /
 * transpose backward into dqkv. f32 only. */
static int64_t attention_index(int64_t b, int64_t t, int64_t part, int64_t h, int64_t d, int64_t length,
                               int64_t heads, int64_t head_dim) {
    return (((b * length + t) * 3 + part) * heads + h) * head_dim + d;
}

static int attention_args(int dtype, int64_t batch, int64_t length, int64_t heads, int64_t head_dim) {
    if (dtype != KD_F32) return fail("causal_attention: f32 only");
    if (batch < 1 || length < 1 || heads < 1 || head_dim < 1) return fail("causal_attention: empty shape");
    return KD_OK;
}

/* a [rows, cols] row-major copy of the head's `part` (0 q, 1 k, 2 v) rows, or its transpose */
static void head_matrix(float* dst, const float* qkv, int64_t b, int64_t part, int64_t h, int64_t length,
                        int64_t heads, int64_t head_dim, int transposed) {
    for (int64_t t = 0; t < length; ++t)
        for (int64_t d = 0; d < head_dim; ++d) {
            const float v = qkv[attention_index(b, t, part, h, d, length, heads, head_dim)];
            if (transposed) dst[d * length + t] = v;
            else dst[t * head_dim + d] = v;
        }
}

static void transpose_f32(float* dst, const float* src, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) dst[c * rows + r] = src[r * cols + c];
}

/* P (the softmax of the scaled, masked scores) of one head and, when lse != NULL, its rows' lse */
static int attention_weights(float* p, float* scores, double* lse, const float* q, const float* kt, int64_t length,
                             int64_t head_dim) {
    kd_matmul_sizes s = {1, length, head_dim, length};
    int rc = oracle_matmul(KD_F32, q, kt, scores, &s, 0);
    if (rc != KD_OK) return rc;
    const float scale = (float)sqrt((double)head_dim);
    for (int64_t i = 0; i < length; ++i)
        for (int64_t j = 0; j < length; ++j) {
            const float x = scores[i * length + j] / scale;
            scores[i * length + j] = j > i ? -INFINITY : x;
        }
    if (lse != NULL)
        for (int64_t i = 0; i < length; ++i) {
            double m = -INFINITY, sum = 0.0;
            for (int64_t j = 0; j <= i; ++j) m = fmax(m, (double)scores[i * length + j]);
            for (int64_t j = 0; j <= i; ++j) sum += exp((double)scores[i * length + j] - m);
            lse[i] = m + log(sum);
        }
    return oracle_softmax_rows(KD_F32, p, scores, length, length, 0);
}

int oracle_causal_attention(int dtype, void* out, void* lse, const void* qkv, int64_t batch, int64_t length,
                            int64_t heads, int64_t head_dim) {
    int rc = attention_args(dtype, batch, length, heads, head_dim);
    if (rc != KD_OK) return rc;
    const float* x = (const float*)qkv;
    const size_t tt = (size_t)(length * length), td = (size_t)(length * head_dim);
    float* q = (float*)malloc(td * 4);
    float* kt = (float*)malloc(td * 4);
    float* v = (float*)malloc(td * 4);
    float* scores = (float*)malloc(tt * 4);
    float* p = (float*)malloc(tt * 4);
    float* o = (float*)malloc(td * 4);
    double* row_lse = (double*)malloc((size_t)length * 8);
    for (int64_t b = 0; b < batch && rc == KD_OK; ++b)
        for (int64_t h = 0; h < heads && rc == KD_OK; ++h) {
            head_matrix(q, x, b, 0, h, length, heads, head_dim, 0);
            head_matrix(kt, x, b, 1, h, length, heads, head_dim, 1);
            head_matrix(v, x, b, 2, h, length, heads, head_dim, 0);
            rc = attention_weights(p, scores, row_lse, q, kt, length, head_dim);
            if (rc != KD_OK) break;
            kd_matmul_sizes s = {1, length, length, head_dim};
            rc = oracle_matmul(KD_F32, p, v, o, &s, 0);
            for (int64_t t = 0; t < length; ++t) {
                for (int64_t d = 0; d < head_dim; ++d)
                    ((float*)out)[((b * length + t) * heads + h) * head_dim + d] = o[t * head_dim + d];
                ((float*)lse)[(b * heads + h) * length + t] = (float)row_lse[t];
            }
        }
    free(q); free(kt); free(v); free(scores); free(p); free(o); free(row_lse);
    return rc;
}

int oracle_causal_attention_backward(int dtype, void* dqkv, const void* dout, const void* qkv, const void* out,
                                     const void* lse, int64_t batch, int64_t length, int64_t heads, int64_t head_dim) {
    (void)out;
    (void)lse;
    int rc = attention_args(dtype, batch, length, heads, head_dim);
    if (rc != KD_OK) return rc;
    const float* x = (const float*)qkv;
    const size_t tt = (size_t)(length * length), td = (size_t)(length * head_dim);
    float* q = (float*)malloc(td * 4);
    float* k = (float*)malloc(td * 4);
    float* kt = (float*)malloc(td * 4);
    float* v = (float*)malloc(td * 4);
    float* vt = (float*)malloc(td * 4);
    float* go = (float*)malloc(td * 4);
    float* scores = (float*)malloc(tt * 4);
    float* p = (float*)malloc(tt * 4);
    float* pt = (float*)malloc(tt * 4);
    float* dp = (float*)malloc(tt * 4);
    float* ds = (float*)malloc(tt * 4);
    float* dst = (float*)malloc(tt * 4);
    float* grad = (float*)malloc(td * 4);
    const float scale = (float)sqrt((double)head_dim);
    for (int64_t b = 0; b < batch && rc == KD_OK; ++b)
        for (int64_t h = 0; h < heads && rc == KD_OK; ++h) {
            head_matrix(q, x, b, 0, h, length, heads, head_dim, 0);
            head_matrix(k, x, b, 1, h, length, heads, head_dim, 0);
            head_matrix(kt, x, b, 1, h, length, heads, head_dim, 1);
            head_matrix(v, x, b, 2, h, length, heads, head_dim, 0);
            head_matrix(vt, x, b, 2, h, length, heads, head_dim, 1);
            for (int64_t t = 0; t < length; ++t)
                for (int64_t d = 0; d < head_dim; ++d)
                    go[t * head_dim + d] = ((const float*)dout)[((b * length + t) * heads + h) * head_dim + d];
            rc = attention_weights(p, scores, NULL, q, kt, length, head_dim);
            if (rc != KD_OK) break;
            kd_matmul_sizes s_dp = {1, length, head_dim, length};  /* dP = dO . V^T */
            rc = oracle_matmul(KD_F32, go, vt, dp, &s_dp, 0);
            transpose_f32(pt, p, length, length);
            kd_matmul_sizes s_dv = {1, length, length, head_dim};  /* dV = P^T . dO */
            if (rc == KD_OK) rc = oracle_matmul(KD_F32, pt, go, grad, &s_dv, 0);
            for (int64_t t = 0; t < length; ++t)
                for (int64_t d = 0; d < head_dim; ++d)
                    ((float*)dqkv)[attention_index(b, t, 2, h, d, length, heads, head_dim)] = grad[t * head_dim + d];
            if (rc == KD_OK) rc = oracle_softmax_rows_backward(KD_F32, ds, p, dp, length, length, 0);
            for (int64_t i = 0; i < length; ++i)
                for (int64_t j = 0; j < length; ++j) {
                    const float g = j > i ? 0.0f : ds[i * length + j];
                    ds[i * length + j] = g / scale;
                }
            kd_matmul_sizes s_dq = {1, length, length, head_dim};  /* dQ = dS . K, dK = dS^T . Q */
            if (rc == KD_OK) rc = oracle_matmul(KD_F32, ds, k, grad, &s_dq, 0);
            for (int64_t t = 0; t < length; ++t)
                for (int64_t d = 0; d < head_dim; ++d)
                    ((float*)dqkv)[attention_index(b, t, 0, h, d, length, heads, head_dim)] = grad[t * head_dim + d];
            transpose_f32(dst, ds, length, length);
            if (rc == KD_OK) rc = oracle_matmul(KD_F32, dst, q, grad, &s_dq, 0);
            for (int64_t t = 0; t < length; ++t)
                for (int64_t d = 0; d < head_dim; ++d)
                    ((float*)dqkv)[attention_index(b, t, 1, h, d, length, heads, head_dim)] = grad[t * head_dim + d];
        }
    free(q); free(k); free(kt); free(v); free(vt); free(go); free(scores); free(p); free(pt); free(dp); free(ds);
    free(dst); free(grad);
    return rc;
}

/* ---- causal self-attention with a KV cache ----------------------------------------------------
 *
 * kael's CausalSelfAttention::forward with a cache (reference src/nn/transformer.cpp:103-138): the
 * new queries Q [T, D] of positions past .. past + T - 1 (past = keys - T), the keys and values
 * K, V [keys, D] of positions 0 .. keys - 1 (the cache's cat with the new rows, :119-126), each
 * per (batch, head) a strided view read element by element; S = Q . K^T (oracle_matmul); S / sqrt(D)
 * rounded to f32; masked_fill with -inf where key > past + query (the future mask's rows past ..
 * past + T, :131); softmax rows; O = P . V; out[b, t, h, :] = O[t]. With past = 0 this is the
 * uncached chain above, op for op. */
int oracle_cached_attention(int dtype, void* out, const void* q, const int64_t* q_strides, const void* k,
                            const int64_t* k_strides, const void* v, const int64_t* v_strides, int64_t batch,
                            int64_t heads, int64_t length, int64_t keys, int64_t head_dim) {
    if (dtype != KD_F32) return fail("cached_attention: f32 only");
    if (batch < 1 || heads < 1 || length < 1 || head_dim < 1 || keys < length)
        return fail("cached_attention: needs batch, heads, length, head_dim >= 1 and keys >= length");
    const float* qf = (const float*)q;
    const float* kf = (const float*)k;
    const float* vf = (const float*)v;
    const int64_t past = keys - length;
    float* qm = (float*)malloc((size_t)(length * head_dim) * 4);
    float* kt = (float*)malloc((size_t)(head_dim * keys) * 4);
    float* vm = (float*)malloc((size_t)(keys * head_dim) * 4);
    float* scores = (float*)malloc((size_t)(length * keys) * 4);
    float* p = (float*)malloc((size_t)(length * keys) * 4);
    float* o = (float*)malloc((size_t)(length * head_dim) * 4);
    const float scale = (float)sqrt((double)head_dim);
    int rc = KD_OK;
    for (int64_t b = 0; b < batch && rc == KD_OK; ++b)
        for (int64_t h = 0; h < heads && rc == KD_OK; ++h) {
            for (int64_t t = 0; t < length; ++t)
                for (int64_t d = 0; d < head_dim; ++d)
                    qm[t * head_dim + d] = qf[b * q_strides[0] + h * q_strides[1] + t * q_strides[2] + d];
            for (int64_t j = 0; j < keys; ++j)
                for (int64_t d = 0; d < head_dim; ++d) {
                    kt[d * keys + j] = kf[b * k_strides[0] + h * k_strides[1] + j * k_strides[2] + d];
                    vm[j * head_dim + d] = vf[b * v_strides[0] + h * v_strides[1] + j * v_strides[2] + d];
                }
            kd_matmul_sizes s_qk = {1, length, head_dim, keys};
            rc = oracle_matmul(KD_F32, qm, kt, scores, &s_qk, 0);
            if (rc != KD_OK) break;
            for (int64_t i = 0; i < length; ++i)
                for (int64_t j = 0; j < keys; ++j) {
                    const float x = scores[i * keys + j] / scale;
                    scores[i * keys + j] = j > past + i ? -INFINITY : x;
                }
            rc = oracle_softmax_rows(KD_F32, p, scores, length, keys, 0);
            kd_matmul_sizes s_pv = {1, length, keys, head_dim};
            if (rc == KD_OK) rc = oracle_matmul(KD_F32, p, vm, o, &s_pv, 0);
            for (int64_t t = 0; t < length && rc == KD_OK; ++t)
                for (int64_t d = 0; d < head_dim; ++d)
                    ((float*)out)[((b * length + t) * heads + h) * head_dim + d] = o[t * head_dim + d];
        }
    free(qm); free(kt); free(vm); free(scores); free(p); free(o);
    return rc;
}

/* ---- sampled next token: kael's sample_next with a top-k -------------------------------------
 *
 * Reference src/nn/transformer.cpp:39-50 for one row of `vocab` logits with temperature > 0:
 * x = logits / temperature (kael's scalar converted to f32, one f32 division); for
 * 0 < top_k < vocab, topk(x, k) (src/ops/sequence.cpp:124-128) gives the k-th largest value t and
 * x < t is masked_fill'ed with -inf (top_k 0 or >= vocab: nothing is masked); softmax's CPU row kernel (src/ops/nn.cpp:60-71: largest, f32
 * exponentials of x - largest, their sum in double in index order rounded to f32, each divided
 * by it); multinomial of one sample with the draw u (src/random.cpp:117-155: the weights as
 * double, partial_sum, point = u * total, upper_bound, the end mapped to the last entry, then
 * back to a positive weight). Finite logits only. */
static int descending_float(const void* a, const void* b) {
    const float x = *(const float*)a, y = *(const float*)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}

int oracle_sample_topk(const float* logits, int64_t vocab, double temperature, int64_t top_k, double uniform,
                       int64_t* token) {
    if (logits == NULL || token == NULL || vocab < 2 || top_k < 0 || !(temperature > 0.0))
        return fail("sample_topk: needs vocab >= 2, top_k >= 0 and temperature > 0");
    /* kael masks below the k-th largest only for 0 < top_k < vocab (top_k 0 is its default) */
    const int masked = top_k > 0 && top_k < vocab;
    if (!(uniform >= 0.0 && uniform < 1.0)) return fail("sample_topk: the draw must lie in [0, 1)");
    const float t = (float)temperature;
    float* x = (float*)malloc((size_t)vocab * sizeof(float));
    float* sorted = (float*)malloc((size_t)vocab * sizeof(float));
    double* cumulative = (double*)malloc((size_t)vocab * sizeof(double));
    int rc = KD_OK;
    for (int64_t i = 0; i < vocab && rc == KD_OK; ++i) {
        x[i] = logits[i] / t;
        if (!isfinite(x[i])) rc = fail("sample_topk: non-finite logit");
        sorted[i] = x[i];
    }
    if (rc == KD_OK) {
        qsort(sorted, (size_t)vocab, sizeof(float), descending_float);
        const float kth = masked ? sorted[top_k - 1] : sorted[vocab - 1];
        float largest = -INFINITY;
        for (int64_t i = 0; i < vocab; ++i) {
            if (x[i] < kth) x[i] = -INFINITY;
            if (x[i] > largest) largest = x[i];
        }
        double total = 0.0;
        for (int64_t i = 0; i < vocab; ++i) {
            x[i] = expf(x[i] - largest);
            total += (double)x[i];
        }
        const float denominator = (float)total;
        double run = 0.0;
        for (int64_t i = 0; i < vocab; ++i) {
            x[i] /= denominator;
            run += (double)x[i];
            cumulative[i] = run;
        }
        const double point = uniform * cumulative[vocab - 1];
        int64_t picked = vocab - 1;
        for (int64_t i = 0; i < vocab; ++i)
            if (cumulative[i] > point) {
                picked = i;
                break;
            }
        while (x[picked] <= 0.0f && picked > 0) --picked;
        *token = picked;
    }
    free(x); free(sorted); free(cumulative);
    return rc;
}

/* ---- matmul: kernels.inl:136-177 -------------------------------------------------------------- */

int oracle_matmul(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* s,
                  int exact) {
    kd_matmul_strides st;
    st.a[0] = s->rows * s->inner; st.a[1] = s->inner; st.a[2] = 1;
    st.b[0] = s->inner * s->columns; st.b[1] = s->columns; st.b[2] = 1;
    st.out[0] = s->rows * s->columns; st.out[1] = s->columns; st.out[2] = 1;
    if (exact && dtype == KD_F32) {
        const float* A = (const float*)a;
        const float* B = (const float*)b;
        float* C = (float*)out;
        for (int64_t bt = 0; bt < s->batches; ++bt)
            for (int64_t i = 0; i < s->rows; ++i)
                for (int64_t j = 0; j < s->columns; ++j) {
                    double acc = 0.0;
                    for (int64_t k = 0; k < s->inner; ++k)
                        acc += (double)A[bt * st.a[0] + i * s->inner + k] *
                               (double)B[bt * st.b[0] + k * s->columns + j];
                    C[bt * st.out[0] + i * s->columns + j] = (float)acc;
                }
        return KD_OK;
    }
    return oracle_matmul_strided(dtype, a, b, out, s, &st);
}

int oracle_matmul_strided(int dtype, const void* a, const void* b, void* out,
                          const kd_matmul_sizes* s, const kd_matmul_strides* t) {
    if (dtype == KD_BOOL) return fail("matmul does not support dtype bool");
    if (dtype_size(dtype) == 0) return fail("matmul: unknown dtype");
    for (int64_t bt = 0; bt < s->batches; ++bt)
        for (int64_t i = 0; i < s->rows; ++i)
            for (int64_t j = 0; j < s->columns; ++j) {
                const int64_t ao = bt * t->a[0] + i * t->a[1];
                const int64_t bo = bt * t->b[0] + j * t->b[2];
                const int64_t oo = bt * t->out[0] + i * t->out[1] + j * t->out[2];
                if (dtype == KD_F32) {
                    float acc = 0.0f;
                    for (int64_t k = 0; k < s->inner; ++k)
                        acc = acc + ((const float*)a)[ao + k * t->a[2]] *
                                        ((const float*)b)[bo + k * t->b[1]];
                    ((float*)out)[oo] = acc;
                } else if (dtype == KD_F64) {
                    double acc = 0.0;
                    for (int64_t k = 0; k < s->inner; ++k)
                        acc = acc + ((const double*)a)[ao + k * t->a[2]] *
                                        ((const double*)b)[bo + k * t->b[1]];
                    ((double*)out)[oo] = acc;
                } else {
                    int64_t acc = 0;
                    for (int64_t k = 0; k < s->inner; ++k)
                        acc = wadd(acc, wmul(((const int64_t*)a)[ao + k * t->a[2]],
                                             ((const int64_t*)b)[bo + k * t->b[1]]));
                    ((int64_t*)out)[oo] = acc;
                }
            }
    return KD_OK;
}

/* kd_matmul_strided_bias: oracle_matmul_strided, then kael's `product + bias` (src/nn/layers.cpp:42-44)
 * as a separate rounded add per element (wrapping for i64). */
int oracle_matmul_strided_bias(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* s,
                               const kd_matmul_strides* t, const void* bias) {
    const int rc = oracle_matmul_strided(dtype, a, b, out, s, t);
    if (rc != KD_OK) return rc;
    for (int64_t bt = 0; bt < s->batches; ++bt)
        for (int64_t i = 0; i < s->rows; ++i)
            for (int64_t j = 0; j < s->columns; ++j) {
                const int64_t o = bt * t->out[0] + i * t->out[1] + j * t->out[2];
                if (dtype == KD_F32) ((float*)out)[o] = ((float*)out)[o] + ((const float*)bias)[j];
                else if (dtype == KD_F64) ((double*)out)[o] = ((double*)out)[o] + ((const double*)bias)[j];
                else ((int64_t*)out)[o] = wadd(((int64_t*)out)[o], ((const int64_t*)bias)[j]);
            }
    return KD_OK;
}

/* kd_matmul_strided_heads: batch i = o * heads + h at o * strides->X[0] + h * heads->X, i.e.
 * oracle_matmul_strided over the `heads` batches of each outer index o. */
int oracle_matmul_strided_heads(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* s,
                                const kd_matmul_strides* t, const kd_matmul_heads* h) {
    if (h->heads < 1) return fail("matmul_strided_heads: heads must be >= 1");
    if (s->batches % h->heads != 0) return fail("matmul_strided_heads: batches is not a multiple of heads");
    const int64_t esize = dtype_size(dtype);
    if (esize == 0) return fail("matmul: unknown dtype");
    kd_matmul_sizes inner = *s;
    inner.batches = h->heads;
    kd_matmul_strides st = *t;
    st.a[0] = h->a;
    st.b[0] = h->b;
    st.out[0] = h->out;
    for (int64_t o = 0; o < s->batches / h->heads; ++o) {
        const int rc = oracle_matmul_strided(dtype, (const char*)a + o * t->a[0] * esize,
                                             (const char*)b + o * t->b[0] * esize, (char*)out + o * t->out[0] * esize,
                                             &inner, &st);
        if (rc != KD_OK) return rc;
    }
    return KD_OK;
}

/* ---- gather / scatter_add: kernels.inl:179-221 --------------------------------------------------- */

typedef struct {
    int64_t data, index, source;
} position_t;

static position_t locate_index(const kd_index_layout* l, const int64_t* indices, int64_t e) {
    position_t p = {0, 0, 0};
    int64_t remaining = e;
    for (int dim = l->dims - 1; dim >= 0; --dim) {
        const int64_t c = remaining % l->shape[dim];
        remaining /= l->shape[dim];
        p.index += c * l->index_strides[dim];
        p.source += c * l->source_strides[dim];
        if (dim != l->axis) p.data += c * l->data_strides[dim];
    }
    p.data += indices[p.index] * l->data_strides[l->axis];
    return p;
}

int oracle_gather(int dtype, void* out, const void* data, const int64_t* indices,
                  const kd_index_layout* l) {
    const int64_t size = dtype_size(dtype);
    if (size == 0) return fail("gather: unknown dtype");
    for (int64_t e = l->count; e-- > 0;) {
        const position_t p = locate_index(l, indices, e);
        memcpy((char*)out + e * size, (const char*)data + p.data * size, (size_t)size);
    }
    return KD_OK;
}

int oracle_scatter_add(int dtype, void* data, const int64_t* indices, const void* source,
                       const kd_index_layout* l) {
    if (dtype != KD_F32 && dtype != KD_F64 && dtype != KD_I64)
        return fail("scatter_add: dtype must be f32, f64 or i64");
    for (int64_t e = 0; e < l->count; ++e) {
        const position_t p = locate_index(l, indices, e);
        if (dtype == KD_F32) ((float*)data)[p.data] += ((const float*)source)[p.source];
        else if (dtype == KD_F64) ((double*)data)[p.data] += ((const double*)source)[p.source];
        else ((int64_t*)data)[p.data] = wadd(((int64_t*)data)[p.data], ((const int64_t*)source)[p.source]);
    }
    return KD_OK;
}

/* ---- row kernels: nn.cpp:52-129, 214-240 ------------------------------------------------------ */

#define ROW_KERNELS(T, SUFFIX, EXPF, LOGF, MAXF)                                                     \
    static T row_max_##SUFFIX(const T* row, int64_t n) {                                        \
        T largest = row[0];                                                                     \
        for (int64_t i = 1; i < n; ++i) largest = MAXF(largest, row[i]);                         \
        return largest;                                                                         \
    }                                                                                           \
    static void softmax_row_##SUFFIX(const T* row, T* out, int64_t n) {                          \
        const T largest = row_max_##SUFFIX(row, n);                                             \
        double total = 0.0;                                                                     \
        for (int64_t i = 0; i < n; ++i) {                                                       \
            out[i] = EXPF(row[i] - largest);                                                    \
            total += (double)out[i];                                                            \
        }                                                                                       \
        const T denominator = (T)total;                                                         \
        for (int64_t i = 0; i < n; ++i) out[i] /= denominator;                                  \
    }                                                                                           \
    static void log_softmax_row_##SUFFIX(const T* row, T* out, int64_t n) {                      \
        const T largest = row_max_##SUFFIX(row, n);                                             \
        double total = 0.0;                                                                     \
        for (int64_t i = 0; i < n; ++i) {                                                       \
            out[i] = row[i] - largest;                                                          \
            total += (double)EXPF(out[i]);                                                      \
        }                                                                                       \
        const T log_total = LOGF((T)total);                                                     \
        for (int64_t i = 0; i < n; ++i) out[i] -= log_total;                                    \
    }                                                                                           \
    static T cross_entropy_row_##SUFFIX(const T* row, int64_t target, int64_t n) {              \
        const T largest = row_max_##SUFFIX(row, n);                                             \
        double total = 0.0;                                                                     \
        for (int64_t i = 0; i < n; ++i) total += (double)EXPF(row[i] - largest);                \
        return LOGF((T)total) - (row[target] - largest);                                        \
    }                                                                                           \
    static void standardize_row_##SUFFIX(const T* row, T* out, int64_t n, double eps,           \
                                         const T* w, const T* b) {                              \
        double total = 0.0;                                                                     \
        for (int64_t i = 0; i < n; ++i) total += (double)row[i];                                \
        const double center = total / (double)n;                                                \
        double squares = 0.0;                                                                   \
        for (int64_t i = 0; i < n; ++i) {                                                       \
            const double d = (double)row[i] - center;                                           \
            squares += d * d;                                                                   \
        }                                                                                       \
        const double scale = sqrt(squares / (double)n + eps);                                   \
        for (int64_t i = 0; i < n; ++i) {                                                       \
            T y = (T)(((double)row[i] - center) / scale);                                       \
            if (w) {                                                                            \
                y = y * w[i];                                                                   \
                y = y + b[i];                                                                   \
            }                                                                                   \
            out[i] = y;                                                                         \
        }                                                                                       \
    }

ROW_KERNELS(float, f32, expf, logf, fmaxnaf)
ROW_KERNELS(double, f64, exp, log, fmaxna)

static int check_floating(int dtype) {
    return dtype == KD_F32 || dtype == KD_F64 ? KD_OK : fail("row kernel: dtype must be f32 or f64");
}

int oracle_softmax_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols,
                        int log_softmax) {
    if (check_floating(dtype)) return KD_E_INVALID;
    if (cols == 0) return KD_OK;
    for (int64_t r = 0; r < rows; ++r) {
        if (dtype == KD_F32) {
            const float* x = (const float*)in + r * cols;
            float* y = (float*)out + r * cols;
            if (log_softmax) log_softmax_row_f32(x, y, cols);
            else softmax_row_f32(x, y, cols);
        } else {
            const double* x = (const double*)in + r * cols;
            double* y = (double*)out + r * cols;
            if (log_softmax) log_softmax_row_f64(x, y, cols);
            else softmax_row_f64(x, y, cols);
        }
    }
    return KD_OK;
}

int oracle_standardize_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols,
                            double eps, const void* weight, const void* bias) {
    if (check_floating(dtype)) return KD_E_INVALID;
    if ((weight == NULL) != (bias == NULL)) return fail("standardize: weight and bias go together");
    if (cols == 0) return KD_OK;
    for (int64_t r = 0; r < rows; ++r) {
        if (dtype == KD_F32)
            standardize_row_f32((const float*)in + r * cols, (float*)out + r * cols, cols, eps,
                                (const float*)weight, (const float*)bias);
        else
            standardize_row_f64((const double*)in + r * cols, (double*)out + r * cols, cols, eps,
                                (const double*)weight, (const double*)bias);
    }
    return KD_OK;
}

int oracle_cross_entropy_rows(int dtype, void* losses, const void* logits, const int64_t* targets,
                              int64_t rows, int64_t cols) {
    if (check_floating(dtype)) return KD_E_INVALID;
    for (int64_t r = 0; r < rows; ++r) {
        if (targets[r] < 0 || targets[r] >= cols) return fail("cross_entropy: target out of range");
        if (dtype == KD_F32)
            ((float*)losses)[r] = cross_entropy_row_f32((const float*)logits + r * cols, targets[r], cols);
        else
            ((double*)losses)[r] = cross_entropy_row_f64((const double*)logits + r * cols, targets[r], cols);
    }
    return KD_OK;
}

int oracle_cross_entropy_grad(int dtype, void* out, const void* logits, const int64_t* targets,
                              const void* weights, int64_t rows, int64_t cols) {
    if (check_floating(dtype)) return KD_E_INVALID;
    for (int64_t r = 0; r < rows; ++r) {
        if (targets[r] < 0 || targets[r] >= cols) return fail("cross_entropy: target out of range");
        if (dtype == KD_F32) {
            float* y = (float*)out + r * cols;
            const float w = ((const float*)weights)[r];
            softmax_row_f32((const float*)logits + r * cols, y, cols);
            for (int64_t i = 0; i < cols; ++i) y[i] *= w;
            y[targets[r]] -= w;
        } else {
            double* y = (double*)out + r * cols;
            const double w = ((const double*)weights)[r];
            softmax_row_f64((const double*)logits + r * cols, y, cols);
            for (int64_t i = 0; i < cols; ++i) y[i] *= w;
            y[targets[r]] -= w;
        }
    }
    return KD_OK;
}

/* ---- row backward passes: src/autograd/functions_reduce.cpp:150-192 ----------------------------
 *
 * kael composes them from whole-tensor device ops; each element op rounds to T (ISO C: no
 * contraction), each row sum is device::reduce Sum: double accumulation in the order of
 * kernels.inl:278-307 (sequential for rows of <= 4096 elements, else sequential 4096-element
 * blocks merged pairwise), rounded to T. mean = sum / T(n) (src/ops/reduce.cpp:330-335);
 * var = sum((x - mean)^2) / T(n) with correction 0 (:337-343). */

#define ROW_BACKWARD(T, SUFFIX, EXPF, SQRTF)                                                        \
    static double device_row_sum_##SUFFIX(const T* v, int64_t n) {                               \
        if (n <= 4096) {                                                                         \
            double total = 0.0;                                                                  \
            for (int64_t i = 0; i < n; ++i) total += (double)v[i];                               \
            return total;                                                                        \
        }                                                                                        \
        const int64_t blocks = (n + 4095) / 4096;                                                \
        double* partial = (double*)malloc((size_t)blocks * sizeof(double));                      \
        for (int64_t b = 0; b < blocks; ++b) {                                                   \
            const int64_t end = (b + 1) * 4096 < n ? (b + 1) * 4096 : n;                         \
            double total = 0.0;                                                                  \
            for (int64_t i = b * 4096; i < end; ++i) total += (double)v[i];                      \
            partial[b] = total;                                                                  \
        }                                                                                        \
        for (int64_t width = blocks; width > 1; width = (width + 1) / 2)                         \
            for (int64_t i = 0; i < (width + 1) / 2; ++i)                                        \
                partial[i] = 2 * i + 1 < width ? partial[2 * i] + partial[2 * i + 1] : partial[2 * i]; \
        const double total = partial[0];                                                         \
        free(partial);                                                                           \
        return total;                                                                            \
    }                                                                                            \
    /* y * (g - sum(g * y)) or g - exp(y) * sum(g); `tmp` holds n elements */                    \
    static void softmax_backward_row_##SUFFIX(const T* y, const T* g, T* out, T* tmp, int64_t n, \
                                              int log_softmax) {                                 \
        if (log_softmax) {                                                                       \
            const T s = (T)device_row_sum_##SUFFIX(g, n);                                        \
            for (int64_t i = 0; i < n; ++i) {                                                    \
                const T t = EXPF(y[i]) * s;                                                      \
                out[i] = g[i] - t;                                                               \
            }                                                                                    \
        } else {                                                                                 \
            for (int64_t i = 0; i < n; ++i) tmp[i] = g[i] * y[i];                                \
            const T s = (T)device_row_sum_##SUFFIX(tmp, n);                                      \
            for (int64_t i = 0; i < n; ++i) {                                                    \
                const T d = g[i] - s;                                                            \
                out[i] = y[i] * d;                                                               \
            }                                                                                    \
        }                                                                                        \
    }                                                                                            \
    /* ((g - mean(g)) - y * mean(g * y)) / sqrt(var(x) + eps) */                                 \
    static void standardize_backward_row_##SUFFIX(const T* x, const T* y, const T* g, T* out,    \
                                                  T* tmp, int64_t n, double eps) {               \
        const T count = (T)n;                                                                    \
        const T mean = (T)device_row_sum_##SUFFIX(x, n) / count;                                 \
        for (int64_t i = 0; i < n; ++i) {                                                        \
            const T d = x[i] - mean;                                                             \
            tmp[i] = d * d;                                                                      \
        }                                                                                        \
        const T var = (T)device_row_sum_##SUFFIX(tmp, n) / count;                                \
        const T shifted = var + (T)eps;                                                          \
        const T scale = SQRTF(shifted);                                                          \
        const T mg = (T)device_row_sum_##SUFFIX(g, n) / count;                                   \
        for (int64_t i = 0; i < n; ++i) tmp[i] = g[i] * y[i];                                    \
        const T mgy = (T)device_row_sum_##SUFFIX(tmp, n) / count;                                \
        for (int64_t i = 0; i < n; ++i) {                                                        \
            const T centered = g[i] - mg;                                                        \
            const T along = y[i] * mgy;                                                          \
            const T diff = centered - along;                                                     \
            out[i] = diff / scale;                                                               \
        }                                                                                        \
    }

ROW_BACKWARD(float, f32, expf, sqrtf)
ROW_BACKWARD(double, f64, exp, sqrt)

int oracle_softmax_rows_backward(int dtype, void* out, const void* y, const void* grad, int64_t rows,
                                 int64_t cols, int log_softmax) {
    if (check_floating(dtype)) return KD_E_INVALID;
    if (rows < 0 || cols < 0) return fail("softmax backward: negative size");
    if (rows == 0 || cols == 0) return KD_OK;
    void* tmp = malloc((size_t)cols * 8);
    for (int64_t r = 0; r < rows; ++r) {
        if (dtype == KD_F32)
            softmax_backward_row_f32((const float*)y + r * cols, (const float*)grad + r * cols,
                                     (float*)out + r * cols, (float*)tmp, cols, log_softmax);
        else
            softmax_backward_row_f64((const double*)y + r * cols, (const double*)grad + r * cols,
                                     (double*)out + r * cols, (double*)tmp, cols, log_softmax);
    }
    free(tmp);
    return KD_OK;
}

int oracle_standardize_rows_backward(int dtype, void* out, const void* x, const void* y, const void* grad,
                                     int64_t rows, int64_t cols, double eps) {
    if (check_floating(dtype)) return KD_E_INVALID;
    if (rows < 0 || cols < 0) return fail("standardize backward: negative size");
    if (rows == 0 || cols == 0) return KD_OK;
    void* tmp = malloc((size_t)cols * 8);
    for (int64_t r = 0; r < rows; ++r) {
        if (dtype == KD_F32)
            standardize_backward_row_f32((const float*)x + r * cols, (const float*)y + r * cols,
                                         (const float*)grad + r * cols, (float*)out + r * cols, (float*)tmp,
                                         cols, eps);
        else
            standardize_backward_row_f64((const double*)x + r * cols, (const double*)y + r * cols,
                                         (const double*)grad + r * cols, (double*)out + r * cols,
                                         (double*)tmp, cols, eps);
    }
    free(tmp);
    return KD_OK;
}

/* kd_layer_norm_rows: LayerNorm::forward (src/nn/layers.cpp:60-68), standardize(x) * w + b:
 * oracle_standardize_rows, then the product and the sum each rounded (kael's two element ops). */
int oracle_layer_norm_rows(int dtype, void* out, void* standardized, const void* in, int64_t rows, int64_t cols,
                           double eps, const void* weight, const void* bias) {
    if (weight == NULL || bias == NULL) return fail("layer norm: weight and bias are required");
    const int rc = oracle_standardize_rows(dtype, standardized, in, rows, cols, eps, NULL, NULL);
    if (rc != KD_OK) return rc;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) {
            if (dtype == KD_F32) {
                const float t = ((const float*)standardized)[r * cols + c] * ((const float*)weight)[c];
                ((float*)out)[r * cols + c] = t + ((const float*)bias)[c];
            } else {
                const double t = ((const double*)standardized)[r * cols + c] * ((const double*)weight)[c];
                ((double*)out)[r * cols + c] = t + ((const double*)bias)[c];
            }
        }
    return KD_OK;
}

/* kd_layer_norm_rows_backward: the backward of LayerNorm::forward as kael composes it from
 * AddBackward and MulBackward (src/autograd/functions_math.cpp:54-72: the bias gradient is g summed
 * over the rows, the weight gradient (g * y) summed over the rows, the standardized rows' gradient
 * g * w) and StandardizeBackward (functions_reduce.cpp:176-192) of g * w; the row sums are
 * sum_to_shape's device sums (oracle_reduce_columns: the reference's reduce over the transposed
 * copy). */
int oracle_layer_norm_rows_backward(int dtype, void* grad_in, void* grad_weight, void* grad_bias, const void* x,
                                    const void* standardized, const void* grad, const void* weight, int64_t rows,
                                    int64_t cols, double eps) {
    if (check_floating(dtype)) return KD_E_INVALID;
    if (rows < 0 || cols < 0) return fail("layer norm backward: negative size");
    const size_t n = (size_t)(rows * cols > 0 ? rows * cols : 1);
    char* gy = (char*)malloc(n * 8);
    char* gyy = (char*)malloc(n * 8);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) {
            const int64_t i = r * cols + c;
            if (dtype == KD_F32) {
                ((float*)gy)[i] = ((const float*)grad)[i] * ((const float*)weight)[c];
                ((float*)gyy)[i] = ((const float*)grad)[i] * ((const float*)standardized)[i];
            } else {
                ((double*)gy)[i] = ((const double*)grad)[i] * ((const double*)weight)[c];
                ((double*)gyy)[i] = ((const double*)grad)[i] * ((const double*)standardized)[i];
            }
        }
    int rc = oracle_standardize_rows_backward(dtype, grad_in, x, standardized, gy, rows, cols, eps);
    if (rc == KD_OK && grad_weight != NULL)
        rc = oracle_reduce_columns(KD_REDUCE_SUM, dtype, dtype, grad_weight, gyy, rows, cols);
    if (rc == KD_OK && grad_bias != NULL)
        rc = oracle_reduce_columns(KD_REDUCE_SUM, dtype, dtype, grad_bias, grad, rows, cols);
    free(gy);
    free(gyy);
    return rc;
}

/* ---- optimizer steps: src/optim/optimizer.cpp:60-80 (SGD), :93-120 (AdamBase::update) ------ */

/* Each statement is one of kael's whole-tensor ops, rounded to the element type (ISO C: no
 * contraction into FMA); scalars are the doubles kael computes, converted to the element type as
 * its scalar fill converts them (src/factory.cpp:68-79). */
#define ADAM_BODY(T, SQRT)                                                                          \
    do {                                                                                            \
        T* p = (T*)param;                                                                           \
        const T* g = (const T*)grad;                                                                \
        T* m = (T*)first;                                                                           \
        T* v = (T*)second;                                                                          \
        const T wd = (T)weight_decay, decay = (T)(1.0 - learning_rate * weight_decay);              \
        const T b1 = (T)beta1, omb1 = (T)(1.0 - beta1), b2 = (T)beta2, omb2 = (T)(1.0 - beta2);     \
        const T c1 = (T)(1.0 - pow(beta1, (double)step)), c2 = (T)(1.0 - pow(beta2, (double)step)); \
        const T eps = (T)epsilon, lr = (T)learning_rate;                                            \
        for (int64_t i = 0; i < count; ++i) {                                                       \
            T gi = g[i];                                                                            \
            if (weight_decay > 0.0 && !decoupled) {                                                 \
                const T t = p[i] * wd; /* gradient + parameter * weight_decay */                    \
                gi = gi + t;                                                                        \
            } else if (weight_decay > 0.0) {                                                        \
                p[i] = p[i] * decay; /* parameter.mul_(1 - lr * weight_decay) */                    \
            }                                                                                       \
            const T m1 = m[i] * b1; /* first.mul_(beta1) */                                         \
            const T t1 = gi * omb1; /* gradient * (1 - beta1) */                                    \
            m[i] = m1 + t1;         /* .add_(...) */                                                \
            const T v1 = v[i] * b2;                                                                 \
            const T gg = gi * gi;                                                                   \
            const T t2 = gg * omb2;                                                                 \
            v[i] = v1 + t2;                                                                         \
            const T cf = m[i] / c1; /* first / first_correction */                                  \
            const T cs = v[i] / c2;                                                                 \
            const T sq = SQRT(cs);                                                                  \
            const T den = sq + eps;                                                                 \
            const T q = cf / den;                                                                   \
            const T u = q * lr;                                                                     \
            p[i] = p[i] - u; /* parameter.sub_(...) */                                              \
        }                                                                                           \
    } while (0)

int oracle_adam_step(int dtype, void* param, const void* grad, void* first, void* second, int64_t count,
                     double learning_rate, double beta1, double beta2, double epsilon, double weight_decay,
                     int decoupled, int64_t step) {
    if (count < 0 || step < 1) return fail("adam_step: negative count or step < 1");
    if (check_floating(dtype)) return KD_E_INVALID;
    if (dtype == KD_F32) ADAM_BODY(float, sqrtf);
    else ADAM_BODY(double, sqrt);
    return KD_OK;
}

#undef ADAM_BODY

/* kd_adam_step_many: oracle_adam_step over the table in order, as the loop of AdamBase::update
 * (reference src/optim/optimizer.cpp:93-120) visits the parameters. */
int oracle_adam_step_many(int dtype, const kd_adam_tensor* tensors, int64_t n, double learning_rate, double beta1,
                          double beta2, double epsilon, double weight_decay, int decoupled) {
    if (n < 0 || (n > 0 && tensors == NULL)) return fail("adam_step_many: negative count or no table");
    for (int64_t i = 0; i < n; ++i) {
        const kd_adam_tensor* x = &tensors[i];
        const int rc = oracle_adam_step(dtype, x->param, x->grad, x->first, x->second, x->count, learning_rate, beta1,
                                        beta2, epsilon, weight_decay, decoupled, x->step);
        if (rc != KD_OK) return rc;
    }
    return KD_OK;
}

int oracle_sgd_step(int dtype, void* param, const void* grad, int64_t count, double learning_rate,
                    double weight_decay) {
    if (count < 0) return fail("sgd_step: negative count");
    if (check_floating(dtype)) return KD_E_INVALID;
    for (int64_t i = 0; i < count; ++i) {
        if (dtype == KD_F32) {
            float* p = (float*)param;
            float gi = ((const float*)grad)[i];
            if (weight_decay > 0.0) {
                const float t = p[i] * (float)weight_decay;
                gi = gi + t;
            }
            const float u = gi * (float)learning_rate;
            p[i] = p[i] - u;
        } else {
            double* p = (double*)param;
            double gi = ((const double*)grad)[i];
            if (weight_decay > 0.0) {
                const double t = p[i] * weight_decay;
                gi = gi + t;
            }
            const double u = gi * learning_rate;
            p[i] = p[i] - u;
        }
    }
    return KD_OK;
}

/* ---- layout planning: iterator.cpp:12-63, 152-172 ------------------------------------------- */

int oracle_layout_build(kd_element_layout* out, int operands, const int* ranks,
                        const int64_t* shapes, const int64_t* strides, const int* element_sizes,
                        void* const* bases) {
    if (operands < 1 || operands > KD_MAX_OPERANDS) return fail("layout: operand count");
    const int ndim = ranks[0];
    if (ndim < 0 || ndim > KD_MAX_DIMS) return fail("layout: rank");
    int64_t shape[KD_MAX_DIMS];
    int64_t st[KD_MAX_OPERANDS][KD_MAX_DIMS];
    int64_t count = 1;
    for (int d = 0; d < ndim; ++d) {
        shape[d] = shapes[d];
        count *= shape[d];
        st[0][d] = strides[d] * element_sizes[0];
    }
    /* broadcast_strides: align trailing dims; size-1 or missing dims get stride 0 */
    for (int op = 1; op < operands; ++op) {
        const int r = ranks[op];
        if (r > ndim) return fail("layout: input rank exceeds the output rank");
        for (int d = 0; d < ndim; ++d) {
            const int src = d - (ndim - r);
            if (src < 0) {
                st[op][d] = 0;
                continue;
            }
            const int64_t size = shapes[op * KD_MAX_DIMS + src];
            if (size == shape[d]) st[op][d] = strides[op * KD_MAX_DIMS + src] * element_sizes[op];
            else if (size == 1) st[op][d] = 0;
            else return fail("layout: shapes do not broadcast");
        }
    }
    /* coalesce_dims: drop size-1 dims, then merge from the innermost outward */
    int n = 0;
    int64_t ms[KD_MAX_DIMS];
    int64_t mst[KD_MAX_OPERANDS][KD_MAX_DIMS];
    for (int d = 0; d < ndim; ++d) {
        if (shape[d] == 1) continue;
        ms[n] = shape[d];
        for (int op = 0; op < operands; ++op) mst[op][n] = st[op][d];
        ++n;
    }
    for (int inner = n - 1; inner >= 1; --inner) {
        const int outer = inner - 1;
        int mergeable = 1;
        for (int op = 0; op < operands; ++op)
            if (mst[op][outer] != mst[op][inner] * ms[inner]) mergeable = 0;
        if (!mergeable) continue;
        ms[outer] *= ms[inner];
        for (int k = inner; k < n - 1; ++k) ms[k] = ms[k + 1];
        for (int op = 0; op < operands; ++op) {
            mst[op][outer] = mst[op][inner];
            for (int k = inner; k < n - 1; ++k) mst[op][k] = mst[op][k + 1];
        }
        --n;
    }
    memset(out, 0, sizeof *out);
    if (n == 0) {
        n = 1;
        ms[0] = 1;
        for (int op = 0; op < operands; ++op) mst[op][0] = 0;
    }
    out->dims = n;
    out->operands = operands;
    out->count = count;
    for (int d = 0; d < n; ++d) {
        out->shape[d] = ms[d];
        for (int op = 0; op < operands; ++op) out->strides[op][d] = mst[op][d];
    }
    for (int op = 0; op < operands; ++op) out->base[op] = bases ? bases[op] : NULL;
    return KD_OK;
}


/* ---- random draws ----------------------------------------------------------------------------
 * std::mt19937_64, sequentially: state words x[0..311] and the position of the next word; at
 * position 312 the whole state is regenerated in place (k = 0..311, each new word from x[k],
 * x[k+1 mod 312] and x[k+156 mod 312], the later ones already new), then tempered word by word. */

#define MT_N 312
#define MT_M 156

void oracle_mt19937_64_seed(uint64_t* state, uint64_t seed) {
    state[0] = seed;
    for (int i = 1; i < MT_N; ++i)
        state[i] = 6364136223846793005ULL * (state[i - 1] ^ (state[i - 1] >> 62)) + (uint64_t)i;
    state[MT_N] = MT_N;
}

static uint64_t mt_next(uint64_t* state) {
    if (state[MT_N] >= MT_N) {
        for (int k = 0; k < MT_N; ++k) {
            const uint64_t y = (state[k] & 0xFFFFFFFF80000000ULL) | (state[(k + 1) % MT_N] & 0x7FFFFFFFULL);
            state[k] = state[(k + MT_M) % MT_N] ^ (y >> 1) ^ ((y & 1) ? 0xB5026F5AA96619E9ULL : 0);
        }
        state[MT_N] = 0;
    }
    uint64_t x = state[state[MT_N]++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

int oracle_mt19937_64_draws(uint64_t* state, int64_t count, uint64_t* out) {
    if (count < 0 || state[MT_N] > MT_N) return fail("oracle_mt19937_64_draws: bad count or state");
    for (int64_t i = 0; i < count; ++i) out[i] = mt_next(state);
    return KD_OK;
}

/* std::uniform_real_distribution<double>(0, 1): generate_canonical<double, 53> takes one 64-bit
 * word, converts it to double (rounded to nearest) and divides by 2^64; a result of 1 becomes the
 * largest double below 1. */
static double uniform01(uint64_t* state) {
    const double u = (double)mt_next(state) / 18446744073709551616.0;
    return u >= 1.0 ? nextafter(1.0, 0.0) : u;
}

int oracle_bernoulli(int dtype, void* out, int64_t count, double probability, uint64_t* state) {
    if (count < 0 || !(probability >= 0.0 && probability <= 1.0) || state[MT_N] > MT_N)
        return fail("oracle_bernoulli: bad arguments");
    for (int64_t i = 0; i < count; ++i) {
        const int hit = uniform01(state) < probability;
        switch (dtype) {
        case KD_F32: ((float*)out)[i] = hit ? 1.0f : 0.0f; break;
        case KD_F64: ((double*)out)[i] = hit ? 1.0 : 0.0; break;
        case KD_I64: ((int64_t*)out)[i] = hit; break;
        case KD_BOOL: ((uint8_t*)out)[i] = (uint8_t)hit; break;
        default: return fail("oracle_bernoulli: unknown dtype");
        }
    }
    return KD_OK;
}

/* dropout: input * bernoulli(keep) / keep, the multiply and the divide each rounded to the element
 * type, keep converted to it (kael's scalar operand). */
int oracle_dropout(int dtype, void* out, void* mask, const void* in, int64_t count, double keep, uint64_t* state) {
    if (count < 0 || !(keep > 0.0 && keep <= 1.0) || state[MT_N] > MT_N) return fail("oracle_dropout: bad arguments");
    if (dtype == KD_F32) {
        const float k = (float)keep;
        for (int64_t i = 0; i < count; ++i) {
            const float m = uniform01(state) < keep ? 1.0f : 0.0f;
            const float product = ((const float*)in)[i] * m;
            ((float*)out)[i] = product / k;
            if (mask) ((float*)mask)[i] = m;
        }
    } else if (dtype == KD_F64) {
        for (int64_t i = 0; i < count; ++i) {
            const double m = uniform01(state) < keep ? 1.0 : 0.0;
            const double product = ((const double*)in)[i] * m;
            ((double*)out)[i] = product / keep;
            if (mask) ((double*)mask)[i] = m;
        }
    } else {
        return fail("oracle_dropout: dtype must be f32 or f64");
    }
    return KD_OK;
}
