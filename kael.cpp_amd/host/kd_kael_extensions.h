// kd_kael_extensions.h - kael::device functions that the MI355X backend adds to kael's device
// interface (reference include/kael/device_kernels.h:96-116) for the fused paths: row softmax /
// log-softmax, row standardization, cross-entropy losses and gradient, GELU backward as one
// element op, matmul over strided (transposed or batch-broadcast) operands, the Adam / SGD
// parameter updates as one kernel per tensor (Adam also over a list of tensors), the reductions kael otherwise computes on the
// host (prod, all, any, argmax / argmin, cumsum), and dropout with its mask drawn on the device.
//
// Defined in backend_hip.cpp. Unmodified kael never calls them; the device branches that do are
// optional kael patches (a one-line include of this header at the end of kael/device_kernels.h,
// and a device branch at each site; oracle/kael_fused.py holds them as anchored insertions).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "kael/device_kernels.h"

namespace kael::device {

// Softmax (log = false) or log-softmax (log = true) of `rows` contiguous rows of `cols`
// elements (reference src/ops/nn.cpp:60-84 row semantics).
void softmax_rows(DType dtype, std::byte* out, const std::byte* in, std::int64_t rows, std::int64_t cols,
                  bool log);

// (x - mean) / sqrt(var + eps) over `rows` contiguous rows of `cols` elements, mean and
// population variance in double (reference src/ops/nn.cpp:114-129).
void standardize_rows(DType dtype, std::byte* out, const std::byte* in, std::int64_t rows, std::int64_t cols,
                      double eps);

// losses[r] = log(sum exp(x - max)) - (x[target[r]] - max) (reference src/ops/nn.cpp:105-112);
// targets are device int64 in [0, cols).
void cross_entropy_rows(DType dtype, std::byte* losses, const std::byte* logits, const std::int64_t* targets,
                        std::int64_t rows, std::int64_t cols);

// out = softmax(x) * w[r] with w[r] subtracted at the target (reference src/ops/nn.cpp:214-240).
void cross_entropy_grad(DType dtype, std::byte* out, const std::byte* logits, const std::int64_t* targets,
                        const std::byte* row_weights, std::int64_t rows, std::int64_t cols);

// Backward of softmax_rows from its output y and the incoming gradient: y * (g - sum(g * y)), or
// g - exp(y) * sum(g) when `log` (reference src/autograd/functions_reduce.cpp:150-164).
void softmax_rows_backward(DType dtype, std::byte* out, const std::byte* y, const std::byte* grad, std::int64_t rows,
                           std::int64_t cols, bool log);

// Backward of standardize_rows from its input x, output y and the incoming gradient:
// ((g - mean(g)) - y * mean(g * y)) / sqrt(var(x) + eps) (reference
// src/autograd/functions_reduce.cpp:176-192).
void standardize_rows_backward(DType dtype, std::byte* out, const std::byte* x, const std::byte* y,
                               const std::byte* grad, std::int64_t rows, std::int64_t cols, double eps);

// LayerNorm::forward in one pass (reference src/nn/layers.cpp:60-68): out = standardized * w + b
// and the standardized rows themselves, over `rows` contiguous rows of `cols`.
void layer_norm_rows(DType dtype, std::byte* out, std::byte* standardized, const std::byte* in, std::int64_t rows,
                     std::int64_t cols, double eps, const std::byte* weight, const std::byte* bias);

// Its backward as kael composes it (AddBackward, MulBackward, StandardizeBackward): grad_in from
// g * w; grad_weight = column sums of g * standardized, grad_bias = column sums of g (either may be
// null).
void layer_norm_rows_backward(DType dtype, std::byte* grad_in, std::byte* grad_weight, std::byte* grad_bias,
                              const std::byte* x, const std::byte* standardized, const std::byte* grad,
                              const std::byte* weight, std::int64_t rows, std::int64_t cols, double eps);

// The element op computing grad * d/dx gelu(x) over operands (out, x, grad), tanh form when
// `approximate` (reference src/autograd/functions_math.cpp:35-46 slopes).
ElementOp gelu_backward_op(bool approximate);

// out[b] = a[b] . b[b] with per-operand element strides {batch, row, column}; a batch stride of 0
// broadcasts the operand (reference src/ops/linalg.cpp:56-76 without the operand copies).
void matmul_strided(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes,
                    const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides);

// matmul_strided with kael's Linear bias add in the product's epilogue: out = product + bias[n]
// (reference src/nn/layers.cpp:42-44), the sum rounded once.
void matmul_strided_bias(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes,
                         const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides,
                         const std::byte* bias);

// matmul_strided over a two-level batch: batch i = o * heads + h reads operand X at
// o * X_strides[0] + h * head_strides[X] (X = a, b, out), for the per-head attention views whose
// batch dims collapse to no single stride (reference src/nn/transformer.cpp:115-136).
void matmul_strided_heads(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes,
                          const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides,
                          std::int64_t heads, const std::int64_t* head_strides);

// One Adam / AdamW step of a contiguous parameter with its moments, in place (reference
// src/optim/optimizer.cpp:93-120): `step` is the parameter's step count after the increment,
// `decoupled` selects AdamW's weight decay. Same rounding as kael's composed ops.
void adam_step(DType dtype, std::byte* param, const std::byte* grad, std::byte* first, std::byte* second,
               std::int64_t count, double learning_rate, double beta1, double beta2, double epsilon,
               double weight_decay, bool decoupled, std::int64_t step);

// One parameter of adam_step_many: contiguous tensors of `count` elements and the parameter's
// step count after the increment.
struct AdamTensor {
    std::byte* param;
    const std::byte* grad;
    std::byte* first;
    std::byte* second;
    std::int64_t count;
    std::int64_t step;
};

// adam_step over every tensor of the list, the same results as one adam_step per tensor in list
// order (reference src/optim/optimizer.cpp:93-120 loop), in one launch per 32 tensors. The tensors
// must not share memory that any of them writes.
void adam_step_many(DType dtype, const std::vector<AdamTensor>& tensors, double learning_rate, double beta1,
                    double beta2, double epsilon, double weight_decay, bool decoupled);

// One SGD step without momentum, in place (reference src/optim/optimizer.cpp:60-80).
void sgd_step(DType dtype, std::byte* param, const std::byte* grad, std::int64_t count, double learning_rate,
              double weight_decay);

// The reductions that device::reduce does not cover (reference device_kernels.h:54 has Sum, Max
// and Min only; kael runs these through a host copy, src/ops/reduce.cpp:362-369,399-451).
enum class ExtraReduceOp { Prod, All, Any };

// results[r] = op over data[r * chunk_size .. (r + 1) * chunk_size), as device::reduce: Prod of
// f32 / f64 accumulates in double and stores In, of i64 / bool wrapping int64 stored as I64
// (reference src/ops/reduce.cpp:202-219,362-369); All / Any store Bool, NaN counting as nonzero,
// an empty chunk giving true / false (:423-451).
void reduce_extra(ExtraReduceOp op, DType in, std::byte* results, const std::byte* data, std::int64_t chunk_size,
                  std::int64_t output_count);

// results[r] = the position in [0, chunk_size) of the first largest (largest = true) or first
// smallest element of chunk r, the first NaN winning (reference src/ops/reduce.cpp:236-268);
// chunk_size > 0.
void arg_reduce(bool largest, DType in, std::int64_t* results, const std::byte* data, std::int64_t chunk_size,
                std::int64_t output_count);

// results[j] = op over i < outer of data[i * inner + j] for j < inner: device::reduce (Sum, Max,
// Min; same accumulators and output dtype `out`) of a contiguous tensor over its leading dims, read
// in place instead of through plan_reduction's transposed copy (reference src/ops/reduce.cpp:118-153).
void reduce_columns(ReduceOp op, DType out, DType in, std::byte* results, const std::byte* data, std::int64_t outer,
                    std::int64_t inner);

// bounds[0] = min, bounds[1] = max of the `count` > 0 device indices indices[i * stride], on the
// host when the call returns: kael's range check of device indices (reference
// src/internal/index_checks.h:37-43) and of cross-entropy targets (src/ops/nn.cpp:97-98) in one
// call and one sync instead of two reductions read back one at a time.
void index_bounds(const std::int64_t* indices, std::int64_t count, std::int64_t stride, std::int64_t bounds[2]);

// kael's causal self-attention without a KV cache or dropout (reference src/nn/transformer.cpp:
// 114-136) over the fused projection's output qkv [B, T, 3, H, D] (contiguous): out [B, T, H * D]
// with the heads merged, lse [B, H, T] the rows' log-sum-exp for the backward. f32, D = 64.
void causal_attention(DType dtype, std::byte* out, std::byte* lse, const std::byte* qkv, std::int64_t batch,
                      std::int64_t length, std::int64_t heads, std::int64_t head_dim);

// Its backward: dqkv [B, T, 3, H, D] (every element written) from dout [B, T, H * D] (contiguous)
// and the forward's qkv, out and lse.
void causal_attention_backward(DType dtype, std::byte* dqkv, const std::byte* dout, const std::byte* qkv,
                               const std::byte* out, const std::byte* lse, std::int64_t batch, std::int64_t length,
                               std::int64_t heads, std::int64_t head_dim);

// The attention of `length` new queries against a KV cache of `keys` positions (reference
// src/nn/transformer.cpp:103-138 with a cache), forward only: q [B, H, length, D], k and v
// [B, H, keys, D] read through the element strides of their batch, head and position dims
// (features contiguous); out [B, length, H * D] with the heads merged. f32, D = 64.
void cached_attention(DType dtype, std::byte* out, const std::byte* q, const std::int64_t* q_strides,
                      const std::byte* k, const std::int64_t* k_strides, const std::byte* v,
                      const std::int64_t* v_strides, std::int64_t batch, std::int64_t heads, std::int64_t length,
                      std::int64_t keys, std::int64_t head_dim);

// Running sums along `rows` contiguous rows of `size` elements (reference src/ops/sequence.cpp:95-117):
// f32 / f64 store In, i64 / bool wrapping int64.
void cumsum_rows(DType in, std::byte* out, const std::byte* data, std::int64_t size, std::int64_t rows);

// Dropout of `count` contiguous f32 / f64 elements with the mask drawn on the device (reference
// src/nn/functional.cpp:32-39, bernoulli src/random.cpp:106-110): out = in * m / T(keep) and mask = m,
// m[i] = 1 where the i-th uniform draw of the std::mt19937_64 whose libstdc++ stream form is
// `state` (312 words, then the position) is below keep; `state` comes back advanced by `count` draws.
void dropout(DType dtype, std::byte* out, std::byte* mask, const std::byte* in, std::int64_t count, double keep,
             std::uint64_t* state);

// The GPT decode engine (kd_gpt_*), for the optional branch of nn::generate (reference
// src/nn/transformer.cpp:256-295) that runs greedy generation with a KV cache on the device.
struct GptEngineShape {
    std::int64_t vocab_size;
    std::int64_t max_positions;
    std::int64_t layers;
    std::int64_t heads;
    std::int64_t dimension;
    bool tanh_gelu;
};

// Whether the engine runs a model of this shape on this device (false: kael's own path runs).
bool gpt_engine_supported(const GptEngineShape& shape);
void* gpt_engine_create(const GptEngineShape& shape);
void gpt_engine_destroy(void* engine) noexcept;
// Copies parameter `name` (a GPT::named_parameters() name) from `count` contiguous f32 device elements.
void gpt_engine_load(void* engine, const char* name, const std::byte* device_data, std::int64_t count);
// Runs the prompt (host ids; its last max_positions when longer) and returns the first greedy token.
std::int64_t gpt_engine_prefill(void* engine, const std::int64_t* prompt, std::int64_t length);
// The next `count` tokens into `tokens` (host), greedy or sampled.
void gpt_engine_decode(void* engine, std::int64_t count, std::int64_t* tokens);
// The pick of the following steps: temperature 0 greedy; temperature > 0 with 0 < top_k < vocab
// kael's sample_next (src/nn/transformer.cpp:39-50) on the device, for vocabularies of at most
// kGptSampleMaxVocab entries.
inline constexpr std::int64_t kGptSampleMaxVocab = 65536;
void gpt_engine_set_sampling(void* engine, double temperature, std::int64_t top_k);
// The uniform draws of the next `count` sampled picks, in order (at most max_positions + 1).
void gpt_engine_set_uniforms(void* engine, const double* uniforms, std::int64_t count);

} // namespace kael::device
