/*
 * kd_api.h - C ABI of the MI355X (gfx950) device backend for kael.
 *
 * Every entry point replaces one function of kael's device boundary,
 * `namespace kael::device` in include/kael/device_kernels.h:96-116 of the reference
 * (JetBerri/kael.cpp 1.0.1). The C++ adapter kael.cpp_amd/host/backend_hip.cpp
 * implements those `kael::device::*` symbols on top of this header and turns a
 * non-zero status into `kael::Error` carrying kd_last_error().
 *
 * Conventions
 *  - Plain C: pointers, sizes and POD structs only. No C++ or torch types.
 *  - Every call returns KD_OK (0) or a negative KD_E_* status; the message of the
 *    last failure on the calling thread is returned by kd_last_error().
 *  - All device work is issued on one in-order HIP stream (kd_set_stream; default
 *    is the null stream), so kernels run in issue order, exactly like the
 *    reference's default-stream backend (reference src/cuda/backend.cu:45-53).
 *  - kd_copy_h2d and kd_copy_d2h return only after the bytes have landed, as the
 *    synchronous cudaMemcpy of reference src/cuda/backend.cu:92-100 does.
 *  - count == 0 (or an empty matrix) is a no-op for every operation.
 *  - Pointers inside layouts already include the tensor offset (reference
 *    src/tensor.cpp:37-41); strides in kd_element_layout are in BYTES, strides in
 *    kd_index_layout are in ELEMENTS (reference device_kernels.h:70-87).
 */
#ifndef KD_API_H
#define KD_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KD_MAX_DIMS 8     /* reference device_kernels.h:12 kMaxDims */
#define KD_MAX_OPERANDS 4 /* reference device_kernels.h:13 kMaxOperands */

/* Status codes. */
#define KD_OK 0
#define KD_E_INVALID (-1)     /* bad argument (dtype, op, sizes, layout) */
#define KD_E_RUNTIME (-2)     /* a HIP runtime call failed */
#define KD_E_NO_DEVICE (-3)   /* no usable gfx950 device */
#define KD_E_UNSUPPORTED (-4) /* combination the reference also rejects */

/* dtype tags; same order as `enum class DType { F32, F64, I64, Bool }`
 * (reference include/kael/dtype.h:22). Bool is stored as one byte 0/1. */
typedef enum kd_dtype { KD_F32 = 0, KD_F64 = 1, KD_I64 = 2, KD_BOOL = 3 } kd_dtype;

/* Element operations; values 0..35 are `enum class ElementOp` in the order of
 * reference include/kael/device_kernels.h:15-52. Values from 64 on are this
 * backend's extensions (no reference counterpart; they replace host round trips
 * or composed launches of the reference, see each comment). */
typedef enum kd_element_op {
    KD_OP_PLUS = 0,
    KD_OP_MINUS,
    KD_OP_TIMES,
    KD_OP_DIVIDES,
    KD_OP_POWER,
    KD_OP_MAXIMUM,
    KD_OP_MINIMUM,
    KD_OP_EQUAL,
    KD_OP_NOT_EQUAL,
    KD_OP_LESS,
    KD_OP_LESS_EQUAL,
    KD_OP_GREATER,
    KD_OP_GREATER_EQUAL,
    KD_OP_LOGICAL_AND,
    KD_OP_LOGICAL_OR,
    KD_OP_LOGICAL_XOR,
    KD_OP_IS_ZERO,
    KD_OP_NEGATE,
    KD_OP_ABSOLUTE,
    KD_OP_SIGN,
    KD_OP_EXP,
    KD_OP_LOG,
    KD_OP_LOG1P,
    KD_OP_EXPM1,
    KD_OP_SQRT,
    KD_OP_RSQRT,
    KD_OP_SIN,
    KD_OP_COS,
    KD_OP_TANH,
    KD_OP_SIGMOID,
    KD_OP_RELU,
    KD_OP_GELU_EXACT,
    KD_OP_GELU_TANH,
    KD_OP_CLAMP,
    KD_OP_WHERE,
    KD_OP_MASKED_FILL,
    /* out = grad * d/dx gelu(x), operands (out, x, grad). Replaces the untagged
     * host lambda of reference src/autograd/functions_math.cpp:221-231, which
     * round-trips a device tensor through the host (include/kael/kernels.h:130-133).
     * Slopes follow functions_math.cpp:35-46. Floating dtypes only. */
    KD_OP_GELU_EXACT_BACKWARD = 64,
    KD_OP_GELU_TANH_BACKWARD = 65
} kd_element_op;

/* `enum class ReduceOp { Sum, Max, Min }` (reference device_kernels.h:54), plus three
 * extensions for reductions that kael computes on the host today (src/ops/reduce.cpp:362-369
 * `prod`, :442-469 `all` / `any`); they use the same contiguous-chunk contract. */
typedef enum kd_reduce_op {
    KD_REDUCE_SUM = 0,
    KD_REDUCE_MAX = 1,
    KD_REDUCE_MIN = 2,
    KD_REDUCE_PROD = 16, /* f32/f64: double accumulation, stores In; i64/bool: wrapping int64 */
    KD_REDUCE_ALL = 17,  /* bool: every element nonzero (NaN counts as nonzero); empty -> 1 */
    KD_REDUCE_ANY = 18   /* bool: some element nonzero; empty -> 0 */
} kd_reduce_op;

/* Mirror of `struct ElementParameters` (reference device_kernels.h:57-68): integer
 * arguments travel apart from real ones so that every int64 survives. */
typedef struct kd_element_parameters {
    double reals[2];
    int64_t integers[2];
} kd_element_parameters;

/* Mirror of `struct ElementLayout` (reference device_kernels.h:70-77), same field
 * order and size (368 bytes). Operand 0 is the output; strides are bytes. */
typedef struct kd_element_layout {
    int32_t dims;
    int32_t operands;
    int64_t count;
    int64_t shape[KD_MAX_DIMS];
    int64_t strides[KD_MAX_OPERANDS][KD_MAX_DIMS];
    void* base[KD_MAX_OPERANDS];
} kd_element_layout;

/* Mirror of `struct IndexLayout` (reference device_kernels.h:79-87); strides are
 * elements. */
typedef struct kd_index_layout {
    int32_t dims;
    int32_t axis;
    int64_t count;
    int64_t shape[KD_MAX_DIMS];
    int64_t data_strides[KD_MAX_DIMS];
    int64_t index_strides[KD_MAX_DIMS];
    int64_t source_strides[KD_MAX_DIMS];
} kd_index_layout;

/* Mirror of `struct MatmulSizes` (reference device_kernels.h:89-94). */
typedef struct kd_matmul_sizes {
    int64_t batches;
    int64_t rows;
    int64_t inner;
    int64_t columns;
} kd_matmul_sizes;

/* ---- errors and runtime ------------------------------------------------ */

/* Message of the last failed call on this thread ("" if none). */
const char* kd_last_error(void);

/* reference device_kernels.h:96 `bool available()`: 1 if a gfx950 device is usable. */
int kd_available(void);
/* reference device_kernels.h:97 `void synchronize()`: drains the backend stream. */
int kd_synchronize(void);
/* Selects the stream every later call issues on (hipStream_t; NULL = null stream).
 * No reference counterpart: the reference always uses the default stream. */
int kd_set_stream(void* stream);
void* kd_get_stream(void);

/* reference device_kernels.h:99 `std::byte* allocate(int64 bytes)`. */
int kd_malloc(void** out, int64_t bytes);
/* reference device_kernels.h:100 `void release(std::byte*) noexcept`: never fails. */
void kd_free(void* block);
/* reference device_kernels.h:101-103 copy_to_device / copy_to_host / copy_within_device. */
int kd_copy_h2d(void* target, const void* source, int64_t bytes);
int kd_copy_d2h(void* target, const void* source, int64_t bytes);
int kd_copy_d2d(void* target, const void* source, int64_t bytes);

/* ---- the hot path ------------------------------------------------------ */

/* reference device_kernels.h:105 `fill(DType, std::byte*, int64 count, const void* value)`:
 * `value` is a host pointer to one element of `dtype`, read during the call. */
int kd_fill(int dtype, void* target, int64_t count, const void* value);

/* reference device_kernels.h:106 `convert(DType out, DType in, const ElementLayout&)`:
 * strided copy with the cast rules of reference src/cuda/kernels.inl:5-13
 * (bool normalisation, saturating float->int). Operands: (out, in). */
int kd_convert(int out_dtype, int in_dtype, const kd_element_layout* layout);

/* reference device_kernels.h:107-108 `elementwise(ElementOp, DType out, DType in,
 * const ElementLayout&, ElementParameters)`. As in the reference, the output dtype
 * is implied by the op (In for arithmetic, Bool for comparisons) and `out_dtype` is
 * ignored (kernels.inl:335). */
int kd_elementwise(int op, int out_dtype, int in_dtype, const kd_element_layout* layout,
                   kd_element_parameters parameters);

/* reference device_kernels.h:109-110 `reduce(ReduceOp, DType out, DType in, std::byte*
 * results, const std::byte* data, int64 chunk_size, int64 output_count)`:
 * results[r] = op over data[r*chunk_size .. (r+1)*chunk_size). Sum of f32/f64
 * accumulates in double and stores In; Sum of i64/bool accumulates wrapping int64
 * and stores int64; Max/Min are NaN-propagating and store In
 * (reference src/cuda/kernels.inl:426-445). Max/Min of an empty chunk is an error. */
int kd_reduce(int op, int out_dtype, int in_dtype, void* results, const void* data,
              int64_t chunk_size, int64_t output_count);

/* Column reductions: results[j] = op over i < outer of data[i * inner + j] (j < inner), i.e. a
 * contiguous tensor reduced over its leading dims, with kd_reduce's ops, accumulators and
 * output dtypes. It replaces, for that case, kael's device reduction plan (reference
 * src/ops/reduce.cpp:118-153 plan_reduction + :309-314 device_reduce), which first copies the
 * tensor with the reduced dims moved last and then calls kd_reduce with chunk = outer and
 * rows = inner: the result is the one that copy and kd_reduce give (max / min and integer sums
 * bit for bit; floating sums accumulate in double in a different order). Max/Min of an empty
 * column is an error. */
int kd_reduce_columns(int op, int out_dtype, int in_dtype, void* results, const void* data,
                      int64_t outer, int64_t inner);

/* kd_reduce without any allocation: no reference counterpart. For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments, kernels and results as kd_reduce (bit for bit); the segment
 * partials of its split path (few long rows) go to a static 64 KiB device buffer that each GPU
 * holds until the process ends, instead of the backend's growable workspace. A call whose
 * partials would not fit fails with KD_E_INVALID (on 256 CUs they take at most 12 KiB). Every
 * call on one GPU shares that buffer. Calls from several host threads are serialised around it
 * (each call's two launches are enqueued together under a lock), and a call on another stream
 * than the previous call's first drains that stream, so calls never overlap on the buffer; work
 * that another library or a graph replay puts on the buffer's stream meanwhile is not covered. */
int kd_reduce_noalloc(int op, int out_dtype, int in_dtype, void* results, const void* data,
                      int64_t chunk_size, int64_t output_count);

/* Replaces the host round trip of reference src/ops/reduce.cpp:399-421 `argmax` / `argmin`
 * (`on_host` + `arg_extreme`, :256-268, `best_position`, :236-254): results[r] = the index
 * in [0, chunk_size) of the first largest (largest != 0) or first smallest element of
 * data[r*chunk_size .. (r+1)*chunk_size), where the first NaN, if any, wins. An empty chunk
 * is an error (plan_nonempty_reduction). */
int kd_arg_reduce(int largest, int in_dtype, int64_t* results, const void* data, int64_t chunk_size,
                  int64_t output_count);

/* Replaces the host round trip of reference src/ops/sequence.cpp:95-117 `cumsum` along a
 * contiguous last dim: out[r][i] = in[r][0] + ... + in[r][i] for `rows` rows of `size`
 * elements. f32/f64 store In (sums accumulated in double here, sequentially in In by the
 * reference: equal within rounding); i64/bool store wrapping int64 (bit-exact). */
int kd_cumsum(int in_dtype, void* out, const void* in, int64_t size, int64_t rows);

/* kael's random draws on the device. `state` (host memory, 313 words) is a std::mt19937_64 in the
 * layout libstdc++ streams it with operator<<: the 312 state words, then the index (0..312) of the
 * next word to temper. Each call draws exactly `count` values, one per element in order, as
 * std::uniform_real_distribution<double>(0, 1) draws them from that engine (libstdc++'s
 * generate_canonical: one 64-bit word per value), writes the result, and returns with `state`
 * advanced past those draws; the call blocks until both are done. */

/* Writes the state of std::mt19937_64(seed) (kael::manual_seed, reference src/random.cpp:62-65);
 * host only. */
void kd_mt19937_64_seed(uint64_t* state, uint64_t seed);

/* reference src/random.cpp:106-110 `bernoulli(shape, probability, dtype)` =
 * (rand(shape, F64) < probability).to(dtype), without the host tensor and its copy: out[i] = 1
 * where draw i < probability, else 0, in dtype (f32, f64, i64 or bool). */
int kd_bernoulli(int dtype, void* out, int64_t count, double probability, uint64_t* state);

/* reference src/nn/functional.cpp:32-39 `dropout(input, p, training)` with keep = 1 - p: out[i] =
 * (in[i] * m[i]) / T(keep), m as kd_bernoulli(dtype, ..., keep) draws it and each op rounded to
 * the element type, in one launch; `mask` (may be NULL) receives m, which the backward pass
 * needs. f32 or f64, contiguous `count` elements; keep in (0, 1]; out may equal in. */
int kd_dropout(int dtype, void* out, void* mask, const void* in, int64_t count, double keep, uint64_t* state);

/* reference device_kernels.h:111-112 `matmul(DType, const std::byte* a, const std::byte* b,
 * std::byte* out, const MatmulSizes&)`: out[b] = a[b] . b[b] for contiguous row-major
 * batches, overwriting out. f32 on the FP32 matrix cores; f64 and i64 (wrapping) on the
 * vector ALUs; bool rejected. */
int kd_matmul(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes);

/* Extension of kd_matmul with element strides per operand, so that transposed or
 * batch-broadcast operands are read in place instead of being materialised by
 * convert (reference src/ops/linalg.cpp:56-76, src/nn/layers.cpp:43,
 * src/autograd/functions_linalg.cpp:37,44). Strides are in elements, for
 * (batch, row, column) of each operand; a batch stride of 0 broadcasts. */
typedef struct kd_matmul_strides {
    int64_t a[3];
    int64_t b[3];
    int64_t out[3];
} kd_matmul_strides;
int kd_matmul_strided(int dtype, const void* a, const void* b, void* out,
                      const kd_matmul_sizes* sizes, const kd_matmul_strides* strides);

/* kd_matmul_strided followed by kael's Linear bias add (reference src/nn/layers.cpp:42-44:
 * product + bias, the bias broadcast over the rows): out[b][m][n] = product + bias[n], the sum
 * rounded once as kael's separate add rounds it (wrapping for i64), in the product's epilogue
 * instead of a second launch that reads and writes the product again. bias: `columns` contiguous
 * elements of dtype. */
int kd_matmul_strided_bias(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                           const kd_matmul_strides* strides, const void* bias);

/* kd_matmul_strided over a two-level batch: batch index i = o * heads + h (sizes->batches a
 * multiple of heads) addresses each operand at o * strides->X[0] + h * heads->X elements. This is
 * how the per-head views of attention (reference src/nn/transformer.cpp:115-136: the [batch,
 * head, token, dim] transposes of the fused qkv projection, of keys.mT() and of the output
 * gradient) are read in place: their batch dims collapse to no single stride, so kael's
 * matmul copies them (src/ops/linalg.cpp:56-76) before the product. heads = 1 is
 * kd_matmul_strided. */
typedef struct kd_matmul_heads {
    int64_t heads;
    int64_t a, b, out;
} kd_matmul_heads;
int kd_matmul_strided_heads(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                            const kd_matmul_strides* strides, const kd_matmul_heads* heads);

/* reference device_kernels.h:113-114 `gather(DType, std::byte* out, const std::byte* data,
 * const int64* indices, const IndexLayout&)`; indices must already be range-checked
 * by the caller (reference src/internal/index_checks.h:37-43). */
int kd_gather(int dtype, void* out, const void* data, const int64_t* indices,
              const kd_index_layout* layout);

/* reference device_kernels.h:115-116 `scatter_add(DType, std::byte* data, const int64*
 * indices, const std::byte* source, const IndexLayout&)`: atomic data[pos] += source[e];
 * i64 wraps; dtypes f32, f64, i64 (the reference sends bool to the host). */
int kd_scatter_add(int dtype, void* data, const int64_t* indices, const void* source,
                   const kd_index_layout* layout);

/* The smallest and largest of `count` > 0 indices indices[i * stride], written to the host pair
 * bounds[0] (min), bounds[1] (max) before the call returns (one stream sync). Replaces the range
 * check kael runs before a device gather / scatter_add (reference src/internal/index_checks.h:
 * 37-43, max(indices).item() then min(indices).item(): two reductions and two blocking reads of
 * a contiguous copy of the broadcast indices) and on cross-entropy targets (src/ops/nn.cpp:97-98,
 * src/nn/loss.cpp:27-28); the caller checks the pair in the same order, max first. */
int kd_index_bounds(const int64_t* indices, int64_t count, int64_t stride, int64_t* bounds);

/* kael's causal self-attention without a KV cache or dropout (reference
 * src/nn/transformer.cpp:114-136: the fused projection viewed [B, T, 3, H, D], q / k / v selected
 * and transposed per head, softmax(masked_fill(q . k^T / sqrt(D), triu mask, -inf)) . v, the heads
 * merged with transpose(1, 2).contiguous()) in one launch instead of the two products, the scale,
 * the mask, the row softmax and the merge copy. qkv [B, T, 3, H, D] and out [B, T, H * D] are
 * contiguous and 16-byte aligned; lse [B, H, T] receives each row's log-sum-exp (scaled, masked
 * scores) for the backward. f32 and D = 64 only (KD_E_UNSUPPORTED otherwise). */
int kd_causal_attention(int dtype, void* out, void* lse, const void* qkv, int64_t batch, int64_t length,
                        int64_t heads, int64_t head_dim);

/* Its backward (kael's autograd for the same chain: the two products' MatmulBackward,
 * SoftmaxBackward, MaskedFillBackward, the division's backward and the select / transpose
 * backward into one tensor): dqkv [B, T, 3, H, D], every element written, from dout
 * [B, T, H * D] and the forward's qkv, out and lse, in one launch. */
int kd_causal_attention_backward(int dtype, void* dqkv, const void* dout, const void* qkv, const void* out,
                                 const void* lse, int64_t batch, int64_t length, int64_t heads, int64_t head_dim);

/* kael's causal self-attention with a KV cache (reference src/nn/transformer.cpp:103-138: the
 * cached keys and values concatenated with the new ones at :119-126, the future mask's rows
 * past .. past + T at :131, then the chain above), forward only, as one launch: `length` new
 * queries at positions keys - length .. keys - 1 against the keys and values of positions
 * 0 .. keys - 1, query t seeing keys 0 .. keys - length + t. q is [batch, heads, length, 64] and
 * k, v are [batch, heads, keys, 64], each read in place through the strides (elements) of its
 * batch, head and position dims in q_strides / k_strides / v_strides (features contiguous):
 * kael's per-head views of the fused projection and its cache tensors. out [batch, length,
 * heads * 64] receives the heads merged (transpose(1, 2).contiguous()). f32 and D = 64 only
 * (KD_E_UNSUPPORTED otherwise). */
int kd_cached_attention(int dtype, void* out, const void* q, const int64_t* q_strides, const void* k,
                        const int64_t* k_strides, const void* v, const int64_t* v_strides, int64_t batch,
                        int64_t heads, int64_t length, int64_t keys, int64_t head_dim);

/* ---- fused row kernels (extensions replacing composed device paths) ---- */

/* Row softmax over `rows` contiguous rows of `cols`: max, exp(x-max), sum in double,
 * divide by the float-rounded sum. `log_softmax` != 0 gives x-max-log(sum).
 * Follows reference src/ops/nn.cpp:60-84; replaces the 5-kernel composition of
 * nn.cpp:158-159 / 176-177. dtype f32 or f64. */
int kd_softmax_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols,
                    int log_softmax);

/* Row standardisation (LayerNorm core): mean and population variance in double,
 * out = (x - mean) / sqrt(var + eps). With `weight`/`bias` non-NULL (length cols)
 * the affine `* weight + bias` is fused in (each rounded as the reference's separate
 * mul and add kernels round it). Follows reference src/ops/nn.cpp:114-129 and
 * src/nn/layers.cpp:60-68; replaces the ~10 launches of nn.cpp:253-258. */
int kd_standardize_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols,
                        double eps, const void* weight, const void* bias);

/* Per-row cross-entropy loss: log(sum exp(x - max)) - (x[target] - max), sum in
 * double. Follows reference src/ops/nn.cpp:105-112 (replaces the device branch
 * nn.cpp:185-187). targets are int64 in [0, cols), range-checked by the caller. */
int kd_cross_entropy_rows(int dtype, void* losses, const void* logits, const int64_t* targets,
                          int64_t rows, int64_t cols);

/* Cross-entropy gradient: out = softmax(x) * w[row] - w[row] * onehot(target).
 * Follows reference src/ops/nn.cpp:214-240 (CPU only in the reference). */
int kd_cross_entropy_grad(int dtype, void* out, const void* logits, const int64_t* targets,
                          const void* row_weights, int64_t rows, int64_t cols);

/* Backward of kd_softmax_rows over `rows` contiguous rows of `cols`: from the forward output y and
 * the incoming gradient g, out = y * (g - sum(g * y)) (softmax) or out = g - exp(y) * sum(g)
 * (log_softmax != 0), each element op rounded to the element type and each row sum accumulated in
 * double and rounded, as kael's composed device ops round them. Replaces SoftmaxBackward and
 * LogSoftmaxBackward of reference src/autograd/functions_reduce.cpp:150-164 (3-4 launches each
 * plus temporaries). dtype f32 or f64; out may not alias y or g. */
int kd_softmax_rows_backward(int dtype, void* out, const void* y, const void* grad, int64_t rows,
                             int64_t cols, int log_softmax);

/* Backward of kd_standardize_rows (without the affine step) over `rows` contiguous rows of `cols`:
 * from the input x, the forward output y and the incoming gradient g,
 * out = ((g - mean(g)) - y * mean(g * y)) / sqrt(var(x) + eps), with mean = sum / n and the
 * population variance sum((x - mean(x))^2) / n, every element op rounded to the element type and
 * every sum accumulated in double and rounded, as kael's composed device ops round them. Replaces
 * StandardizeBackward of reference src/autograd/functions_reduce.cpp:176-192 (~12 launches).
 * dtype f32 or f64; out may not alias x, y or g. */
int kd_standardize_rows_backward(int dtype, void* out, const void* x, const void* y, const void* grad,
                                 int64_t rows, int64_t cols, double eps);

/* kael's LayerNorm::forward, standardize(x) * weight + bias (reference src/nn/layers.cpp:60-68),
 * in one launch: `out` as kd_standardize_rows with the affine step, and `standardized` the rows
 * before it (what kael's standardize returns, which the backward reads). dtype f32 or f64; weight
 * and bias of length cols. */
int kd_layer_norm_rows(int dtype, void* out, void* standardized, const void* in, int64_t rows, int64_t cols,
                       double eps, const void* weight, const void* bias);

/* The backward of kd_layer_norm_rows as kael composes it from AddBackward, MulBackward and
 * StandardizeBackward (reference src/autograd/functions_math.cpp:54-72,
 * functions_reduce.cpp:176-192) for the gradient g of `out`, with y the standardized rows:
 * grad_in = kd_standardize_rows_backward(x, y, g * weight) (each product rounded),
 * grad_weight[c] = sum over rows of g * y (products rounded, summed in double),
 * grad_bias[c] = sum over rows of g (in double). Two launches for rows of <= 1024 elements
 * (cols % 4 == 0, 16-byte aligned) instead of ~9. grad_weight / grad_bias may be NULL (not
 * computed). dtype f32 or f64; outputs may not alias inputs. */
int kd_layer_norm_rows_backward(int dtype, void* grad_in, void* grad_weight, void* grad_bias, const void* x,
                                const void* standardized, const void* grad, const void* weight, int64_t rows,
                                int64_t cols, double eps);

/* ---- optimizer steps (extensions replacing composed device paths) ------ */

/* One Adam / AdamW step of a contiguous parameter tensor in place, with its first and second
 * moments: the element chain of reference src/optim/optimizer.cpp:93-120 (AdamBase::update),
 * each op rounded as kael's separate device op rounds it, the scalars converted to the element
 * type as kael's scalar fills convert them, bias corrections 1 - beta^step with the host's pow.
 * weight_decay > 0 with decoupled == 0 adds p * weight_decay to the gradient (Adam); with
 * decoupled != 0 it scales p by 1 - lr * weight_decay first (AdamW). `step` >= 1 is the
 * parameter's step count after the increment. Replaces 14 element launches and 7 fills per
 * tensor. dtype f32 or f64. */
int kd_adam_step(int dtype, void* param, const void* grad, void* first, void* second, int64_t count,
                 double learning_rate, double beta1, double beta2, double epsilon, double weight_decay,
                 int decoupled, int64_t step);

/* One parameter tensor of kd_adam_step_many: contiguous param, grad and moments of `count`
 * elements; `step` >= 1 is the tensor's own step count after the increment. */
typedef struct kd_adam_tensor {
    void* param;
    const void* grad;
    void* first;
    void* second;
    int64_t count;
    int64_t step;
} kd_adam_tensor;

/* kd_adam_step over `n` tensors, the same bits as n kd_adam_step calls in table order, in one
 * launch per 32 tensors: the loop of reference src/optim/optimizer.cpp:93-120 (AdamBase::update)
 * over every parameter with a gradient, 52 launches per step for the char-GPT config. The table
 * is read on the host during the call. Tensors whose memory overlaps memory another of them
 * writes (param, first or second) are rejected with KD_E_INVALID before anything runs. */
int kd_adam_step_many(int dtype, const kd_adam_tensor* tensors, int64_t n, double learning_rate, double beta1,
                      double beta2, double epsilon, double weight_decay, int decoupled);

/* One SGD step without momentum: p -= (g (+ p * weight_decay if > 0)) * learning_rate, as
 * reference src/optim/optimizer.cpp:60-80 computes it. dtype f32 or f64. */
int kd_sgd_step(int dtype, void* param, const void* grad, int64_t count, double learning_rate,
                double weight_decay);

/* ---- host-side layout planning ----------------------------------------- */

/* Builds the kd_element_layout that kael's TensorIterator would hand to the device for
 * these operands (reference src/iterator.cpp:152-172 prepare_loop, :47-63 coalesce_dims,
 * :112-132 device_layout; src/shape.cpp:123-145 broadcast_strides): operand 0 is the output
 * with `ranks[0]` dims; inputs broadcast against it (trailing alignment; size-1 dims get
 * stride 0); strides are converted to bytes; size-1 dims are dropped and mergeable dims
 * coalesced from the innermost outward; an empty result becomes one dim of size 1.
 * shapes/strides are [operands][KD_MAX_DIMS] arrays of ELEMENT counts. Host only. */
int kd_layout_build(kd_element_layout* out, int operands, const int* ranks, const int64_t* shapes,
                    const int64_t* strides, const int* element_sizes, void* const* bases);

/* ---- GPT-2 decode engine (config C5) ---------------------------------------- */

/* The workload of reference examples/gpt2_generate.cpp: kael's GPT (src/nn/transformer.cpp:
 * 103-237) run by nn::generate with temperature 0 and a KV cache (:256-295), batch 1, f32.
 * No single reference function corresponds: kael composes it from ~700 device calls per
 * token. This engine keeps kael's parameter layout and arithmetic (LayerNorm = standardize
 * then affine, Linear = x.W^T then + bias, tanh GELU, scores / sqrt(head_dim), row softmax
 * with a double sum, greedy first-maximum argmax) and runs each token as one HIP graph. */
typedef struct kd_gpt_config {
    int64_t vocab_size;    /* GptConfig::vocab_size (include/kael/nn/transformer.h:19-30) */
    int64_t max_positions; /* GptConfig::max_positions */
    int64_t layers;
    int64_t heads;
    int64_t dimension;
    int32_t tanh_gelu;     /* GptConfig::tanh_gelu */
    int32_t flags;         /* KD_GPT_EAGER: launch each step's kernels directly instead of
                              replaying the captured graph (for kernel-level profiling);
                              KD_GPT_STEPWISE_PREFILL: run the prompt one cached step per
                              position instead of the batched prefill (for comparison);
                              other bits are KD_E_INVALID */
} kd_gpt_config;
#define KD_GPT_EAGER 1
#define KD_GPT_STEPWISE_PREFILL 2

int kd_gpt_create(void** handle, const kd_gpt_config* config);
/* KD_OK when kd_gpt_create would accept `config` on this device (sizes, head_dim a multiple of 4 up
 * to 64, 4 * dimension <= 4096, at most 64 heads and 8192 positions); otherwise the status and
 * message kd_gpt_create would give. Allocates nothing. */
int kd_gpt_supported(const kd_gpt_config* config);
/* The parameters of kael's GPT as `manual_seed(seed); GPT model(config)` initialises them (reference
 * src/nn/transformer.cpp:167-207 with src/nn/layers.cpp:17-73 and src/random.cpp:62-88), on the
 * host, concatenated in GPT::named_parameters() order (the names kd_gpt_load_parameter takes):
 * *count receives the total; with params non-NULL, `capacity` floats must hold it. Draws through
 * the standard library's std::mt19937_64 and distributions as kael does, so the values are kael's
 * on the same standard library. Needs no device. */
int kd_gpt_kael_init(const kd_gpt_config* config, uint64_t seed, float* params, int64_t capacity, int64_t* count);
void kd_gpt_destroy(void* handle);
/* Uploads one parameter by its kael name (GPT::named_parameters(), e.g. "blocks.3.attn.qkv.weight")
 * from host f32 data holding all `count` elements in kael's row-major layout. */
int kd_gpt_load_parameter(void* handle, const char* name, const float* data, int64_t count);
/* The same from device memory (`data` is a device pointer to `count` contiguous f32 elements, e.g.
 * the storage of kael's parameter tensor on this device); the copy is complete on return. No
 * reference counterpart: it serves the optional kael branch that runs nn::generate on this engine. */
int kd_gpt_load_parameter_device(void* handle, const char* name, const float* data, int64_t count);
/* reference src/nn/transformer.cpp:297-308 `load_gpt2_weights(GPT&, path)` over
 * src/io/safetensors.cpp:258-318 `read_safetensors`: loads a Hugging Face GPT-2 checkpoint
 * (model.safetensors) into the engine. The file is memory-mapped and checked as the reference checks
 * it (header size, entry dtype / shape / offsets, entries tiling the data, bool bytes); names are
 * translated to kael's (transformer. prefix dropped, h.N. -> blocks.N., c_attn -> qkv, ...), the
 * Conv1D weights of qkv / proj / fc1 / fc2 transposed from [in, out], entries kael's GPT does not
 * have ignored; a missing parameter or a wrong shape is KD_E_INVALID before anything is copied
 * (Module::load_state_dict). Values convert to f32 as kael's copy_ converts F64 / I64 / BOOL; F16
 * and BF16, which the reference rejects, are widened; other dtypes are KD_E_UNSUPPORTED. */
int kd_gpt_load_safetensors(void* handle, const char* path);
/* One tensor of a safetensors file as f32 on the host (no device needed), the file checked as
 * kd_gpt_load_safetensors checks it: *dims = its rank, shape[0..rank) its sizes (shape may be NULL);
 * with out == NULL only the rank and shape are returned, else `capacity` (elements) must hold it.
 * The reference's counterpart is src/io/safetensors.cpp:320-322 `load_safetensors` (a map of every
 * tensor); this returns one tensor per call so that a plain C caller needs no map type. */
int kd_safetensors_tensor(const char* path, const char* name, float* out, int64_t capacity, int64_t* shape,
                          int32_t* dims);
/* Runs the prompt through the model from position 0 with an empty KV cache; the last position's
 * picked token (greedy or sampled, kd_gpt_set_sampling) becomes the first generated token. Clears any previous sequence. A prompt longer
 * than max_positions runs its last max_positions tokens, as nn::generate does (reference
 * src/nn/transformer.cpp:270-284). By default all positions pass each layer together (GEMMs on
 * the matrix cores, causal attention); KD_GPT_STEPWISE_PREFILL runs them as cached single-token
 * steps. */
int kd_gpt_prefill(void* handle, const int64_t* prompt, int64_t length);
/* Generates `count` more tokens, greedily or sampled (reference nn::generate with use_cache):
 * one cached step each while the KV cache has room; once it holds max_positions positions, each
 * token clears it and reruns the sequence's last max_positions tokens from position 0, as
 * nn::generate does. `tokens` (host, may be NULL) receives the `count` new ids. */
int kd_gpt_decode(void* handle, int64_t count, int64_t* tokens);
/* Teacher-forced cached forward over `count` tokens starting at position 0; writes the logits
 * of every position (count x vocab, host). Used for step-by-step parity. */
int kd_gpt_forward_logits(void* handle, const int64_t* tokens, int64_t count, float* logits);
/* The full sequence so far (prompt + generated), `capacity` entries at most; returns its length
 * through `length`. */
int kd_gpt_sequence(void* handle, int64_t* ids, int64_t capacity, int64_t* length);
/* The logits of the most recent position (vocab_size floats, host): the prompt's last position
 * after kd_gpt_prefill, the last step's after kd_gpt_decode. No reference counterpart (kael's
 * generate returns tokens only); for parity checks of the prefill paths. */
int kd_gpt_logits(void* handle, float* logits);
/* The pick of every following prefill and decode step: temperature 0 is the greedy pick (the
 * default); temperature > 0 is kael's sample_next (reference src/nn/transformer.cpp:39-50:
 * logits / temperature, with 0 < top_k < vocab_size the top_k largest kept, otherwise (top_k 0,
 * kael's default, or top_k >= vocab_size) every entry, softmax, multinomial of one sample,
 * src/random.cpp:106-160) on the device, drawing the next uniform given by kd_gpt_set_uniforms
 * for each sampled token. Without a top-k the softmax and multinomial sums run over the whole
 * vocabulary in index order, as kael's do, in one wave (about 0.5 ms per token for GPT-2's).
 * A vocabulary above KD_GPT_SAMPLE_MAX_VOCAB, whose keys no longer fit the picking workgroup's
 * registers, is KD_E_UNSUPPORTED when sampled (kael's own loop samples). */
#define KD_GPT_SAMPLE_MAX_VOCAB 65536
int kd_gpt_set_sampling(void* handle, double temperature, int64_t top_k);
/* The uniform draws in [0, 1) for the next `count` sampled picks, in order (at most
 * max_positions + 1): what uniform_real_distribution<double>(0, 1) on kael's generator returns
 * for each multinomial sample (one draw per sampled token). A sampled pick with no draw left
 * fails the call that ran it. No reference counterpart: kael draws inside multinomial. */
int kd_gpt_set_uniforms(void* handle, const double* uniforms, int64_t count);
/* How many of the uniforms given by kd_gpt_set_uniforms the sampled picks have used. */
int kd_gpt_draws_used(void* handle, int64_t* used);

/* ---- measurement helpers (no reference counterpart; used by the bench) -- */

/* HIP events recorded on the backend stream. */
int kd_event_create(void** event);
int kd_event_destroy(void* event);
int kd_event_record(void* event);
int kd_event_elapsed_ms(float* ms, void* start, void* stop);
/* Device properties: compute units, max engine clock (kHz), and the gfx arch name. */
int kd_device_info(int* compute_units, int* clock_khz, char* arch, int arch_len);

#ifdef __cplusplus
}
#endif

#endif /* KD_API_H */
