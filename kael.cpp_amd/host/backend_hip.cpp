// backend_hip.cpp - the drop-in kael device backend for MI355X.
//
// Defines every function of `namespace kael::device` (reference include/kael/device_kernels.h:96-116)
// on top of the C ABI in include/kd_api.h. It takes the place of the backend translation unit
// that kael's build picks (reference CMakeLists.txt:26-36: src/cuda/backend.cu, backend_fake.cpp
// or backend_none.cpp): compile this file with kael's include directory and link libkd.so.
// Failures become kael::Error carrying the backend's message (as KAEL_CUDA_CHECK does in
// reference src/cuda/backend.cu:17-32); release() never throws (backend.cu:88-90). The fused
// entry points of kd_kael_extensions.h are defined at the end.
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "kael/device_kernels.h"
#include "kael/error.h"

#include "kd_api.h"
#include "kd_kael_extensions.h"

namespace kael::device {

namespace {

// The C mirrors must be byte-for-byte the reference structs: they are passed by pointer.
static_assert(sizeof(kd_element_layout) == sizeof(ElementLayout));
static_assert(offsetof(kd_element_layout, count) == offsetof(ElementLayout, count));
static_assert(offsetof(kd_element_layout, shape) == offsetof(ElementLayout, shape));
static_assert(offsetof(kd_element_layout, strides) == offsetof(ElementLayout, strides));
static_assert(offsetof(kd_element_layout, base) == offsetof(ElementLayout, base));
static_assert(sizeof(kd_index_layout) == sizeof(IndexLayout));
static_assert(offsetof(kd_index_layout, shape) == offsetof(IndexLayout, shape));
static_assert(offsetof(kd_index_layout, source_strides) == offsetof(IndexLayout, source_strides));
static_assert(sizeof(kd_matmul_sizes) == sizeof(MatmulSizes));
static_assert(static_cast<int>(DType::F32) == KD_F32 && static_cast<int>(DType::Bool) == KD_BOOL);
static_assert(static_cast<int>(ElementOp::MaskedFill) == KD_OP_MASKED_FILL);
static_assert(static_cast<int>(ReduceOp::Min) == KD_REDUCE_MIN);

void check(int status, const char* what) {
    if (status != KD_OK) {
        throw Error(std::string("MI355X backend: ") + what + " failed: " + kd_last_error());
    }
}

const kd_element_layout* c_layout(const ElementLayout& layout) {
    return reinterpret_cast<const kd_element_layout*>(&layout);
}

} // namespace

bool available() { return kd_available() != 0; }

void synchronize() { check(kd_synchronize(), "synchronize"); }

std::byte* allocate(std::int64_t bytes) {
    void* block = nullptr;
    check(kd_malloc(&block, bytes), "allocate");
    return static_cast<std::byte*>(block);
}

void release(std::byte* block) noexcept { kd_free(block); }

void copy_to_device(std::byte* target, const std::byte* source, std::int64_t bytes) {
    check(kd_copy_h2d(target, source, bytes), "copy_to_device");
}

void copy_to_host(std::byte* target, const std::byte* source, std::int64_t bytes) {
    check(kd_copy_d2h(target, source, bytes), "copy_to_host");
}

void copy_within_device(std::byte* target, const std::byte* source, std::int64_t bytes) {
    check(kd_copy_d2d(target, source, bytes), "copy_within_device");
}

void fill(DType dtype, std::byte* target, std::int64_t count, const void* value) {
    check(kd_fill(static_cast<int>(dtype), target, count, value), "fill");
}

void convert(DType out, DType in, const ElementLayout& layout) {
    check(kd_convert(static_cast<int>(out), static_cast<int>(in), c_layout(layout)), "convert");
}

void elementwise(ElementOp op, DType out, DType in, const ElementLayout& layout, ElementParameters parameters) {
    kd_element_parameters p;
    p.reals[0] = parameters.reals[0];
    p.reals[1] = parameters.reals[1];
    p.integers[0] = parameters.integers[0];
    p.integers[1] = parameters.integers[1];
    check(kd_elementwise(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in), c_layout(layout), p),
          "elementwise");
}

void reduce(ReduceOp op, DType out, DType in, std::byte* results, const std::byte* data, std::int64_t chunk_size,
            std::int64_t output_count) {
    check(kd_reduce(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in), results, data, chunk_size,
                    output_count),
          "reduce");
}

void matmul(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes) {
    const kd_matmul_sizes s{sizes.batches, sizes.rows, sizes.inner, sizes.columns};
    check(kd_matmul(static_cast<int>(dtype), a, b, out, &s), "matmul");
}

void gather(DType dtype, std::byte* out, const std::byte* data, const std::int64_t* indices,
            const IndexLayout& layout) {
    check(kd_gather(static_cast<int>(dtype), out, data, indices, reinterpret_cast<const kd_index_layout*>(&layout)),
          "gather");
}

void scatter_add(DType dtype, std::byte* data, const std::int64_t* indices, const std::byte* source,
                 const IndexLayout& layout) {
    check(kd_scatter_add(static_cast<int>(dtype), data, indices, source,
                         reinterpret_cast<const kd_index_layout*>(&layout)),
          "scatter_add");
}

// ---- extensions (kd_kael_extensions.h) ----------------------------------------------------

void softmax_rows(DType dtype, std::byte* out, const std::byte* in, std::int64_t rows, std::int64_t cols, bool log) {
    check(kd_softmax_rows(static_cast<int>(dtype), out, in, rows, cols, log ? 1 : 0), "softmax_rows");
}

void standardize_rows(DType dtype, std::byte* out, const std::byte* in, std::int64_t rows, std::int64_t cols,
                      double eps) {
    check(kd_standardize_rows(static_cast<int>(dtype), out, in, rows, cols, eps, nullptr, nullptr), "standardize_rows");
}

void cross_entropy_rows(DType dtype, std::byte* losses, const std::byte* logits, const std::int64_t* targets,
                        std::int64_t rows, std::int64_t cols) {
    check(kd_cross_entropy_rows(static_cast<int>(dtype), losses, logits, targets, rows, cols), "cross_entropy_rows");
}

void cross_entropy_grad(DType dtype, std::byte* out, const std::byte* logits, const std::int64_t* targets,
                        const std::byte* row_weights, std::int64_t rows, std::int64_t cols) {
    check(kd_cross_entropy_grad(static_cast<int>(dtype), out, logits, targets, row_weights, rows, cols),
          "cross_entropy_grad");
}

void softmax_rows_backward(DType dtype, std::byte* out, const std::byte* y, const std::byte* grad, std::int64_t rows,
                           std::int64_t cols, bool log) {
    check(kd_softmax_rows_backward(static_cast<int>(dtype), out, y, grad, rows, cols, log ? 1 : 0),
          "softmax_rows_backward");
}

void standardize_rows_backward(DType dtype, std::byte* out, const std::byte* x, const std::byte* y,
                               const std::byte* grad, std::int64_t rows, std::int64_t cols, double eps) {
    check(kd_standardize_rows_backward(static_cast<int>(dtype), out, x, y, grad, rows, cols, eps),
          "standardize_rows_backward");
}

void layer_norm_rows(DType dtype, std::byte* out, std::byte* standardized, const std::byte* in, std::int64_t rows,
                     std::int64_t cols, double eps, const std::byte* weight, const std::byte* bias) {
    check(kd_layer_norm_rows(static_cast<int>(dtype), out, standardized, in, rows, cols, eps, weight, bias),
          "layer_norm_rows");
}

void layer_norm_rows_backward(DType dtype, std::byte* grad_in, std::byte* grad_weight, std::byte* grad_bias,
                              const std::byte* x, const std::byte* standardized, const std::byte* grad,
                              const std::byte* weight, std::int64_t rows, std::int64_t cols, double eps) {
    check(kd_layer_norm_rows_backward(static_cast<int>(dtype), grad_in, grad_weight, grad_bias, x, standardized, grad,
                                      weight, rows, cols, eps),
          "layer_norm_rows_backward");
}

ElementOp gelu_backward_op(bool approximate) {
    return static_cast<ElementOp>(approximate ? KD_OP_GELU_TANH_BACKWARD : KD_OP_GELU_EXACT_BACKWARD);
}

void matmul_strided(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes,
                    const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides) {
    const kd_matmul_sizes s{sizes.batches, sizes.rows, sizes.inner, sizes.columns};
    kd_matmul_strides st;
    for (int i = 0; i < 3; ++i) {
        st.a[i] = a_strides[i];
        st.b[i] = b_strides[i];
        st.out[i] = out_strides[i];
    }
    check(kd_matmul_strided(static_cast<int>(dtype), a, b, out, &s, &st), "matmul_strided");
}

void matmul_strided_bias(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes,
                         const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides,
                         const std::byte* bias) {
    const kd_matmul_sizes s{sizes.batches, sizes.rows, sizes.inner, sizes.columns};
    kd_matmul_strides st;
    for (int i = 0; i < 3; ++i) {
        st.a[i] = a_strides[i];
        st.b[i] = b_strides[i];
        st.out[i] = out_strides[i];
    }
    check(kd_matmul_strided_bias(static_cast<int>(dtype), a, b, out, &s, &st, bias), "matmul_strided_bias");
}

void matmul_strided_heads(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& sizes,
                          const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides,
                          std::int64_t heads, const std::int64_t* head_strides) {
    const kd_matmul_sizes s{sizes.batches, sizes.rows, sizes.inner, sizes.columns};
    kd_matmul_strides st;
    for (int i = 0; i < 3; ++i) {
        st.a[i] = a_strides[i];
        st.b[i] = b_strides[i];
        st.out[i] = out_strides[i];
    }
    const kd_matmul_heads h{heads, head_strides[0], head_strides[1], head_strides[2]};
    check(kd_matmul_strided_heads(static_cast<int>(dtype), a, b, out, &s, &st, &h), "matmul_strided_heads");
}

void adam_step(DType dtype, std::byte* param, const std::byte* grad, std::byte* first, std::byte* second,
               std::int64_t count, double learning_rate, double beta1, double beta2, double epsilon,
               double weight_decay, bool decoupled, std::int64_t step) {
    check(kd_adam_step(static_cast<int>(dtype), param, grad, first, second, count, learning_rate, beta1, beta2,
                       epsilon, weight_decay, decoupled ? 1 : 0, step),
          "adam_step");
}

void adam_step_many(DType dtype, const std::vector<AdamTensor>& tensors, double learning_rate, double beta1,
                    double beta2, double epsilon, double weight_decay, bool decoupled) {
    thread_local std::vector<kd_adam_tensor> table;
    table.clear();
    for (const AdamTensor& t : tensors) table.push_back({t.param, t.grad, t.first, t.second, t.count, t.step});
    check(kd_adam_step_many(static_cast<int>(dtype), table.data(), static_cast<std::int64_t>(table.size()),
                            learning_rate, beta1, beta2, epsilon, weight_decay, decoupled ? 1 : 0),
          "adam_step_many");
}

void sgd_step(DType dtype, std::byte* param, const std::byte* grad, std::int64_t count, double learning_rate,
              double weight_decay) {
    check(kd_sgd_step(static_cast<int>(dtype), param, grad, count, learning_rate, weight_decay), "sgd_step");
}

void reduce_extra(ExtraReduceOp op, DType in, std::byte* results, const std::byte* data, std::int64_t chunk_size,
                  std::int64_t output_count) {
    const int code = op == ExtraReduceOp::Prod ? KD_REDUCE_PROD : op == ExtraReduceOp::All ? KD_REDUCE_ALL : KD_REDUCE_ANY;
    const int out = op != ExtraReduceOp::Prod ? KD_BOOL : (in == DType::F32 || in == DType::F64) ? static_cast<int>(in) : KD_I64;
    check(kd_reduce(code, out, static_cast<int>(in), results, data, chunk_size, output_count), "reduce_extra");
}

void arg_reduce(bool largest, DType in, std::int64_t* results, const std::byte* data, std::int64_t chunk_size,
                std::int64_t output_count) {
    check(kd_arg_reduce(largest ? 1 : 0, static_cast<int>(in), results, data, chunk_size, output_count), "arg_reduce");
}

void cumsum_rows(DType in, std::byte* out, const std::byte* data, std::int64_t size, std::int64_t rows) {
    check(kd_cumsum(static_cast<int>(in), out, data, size, rows), "cumsum_rows");
}

void dropout(DType dtype, std::byte* out, std::byte* mask, const std::byte* in, std::int64_t count, double keep,
             std::uint64_t* state) {
    check(kd_dropout(static_cast<int>(dtype), out, mask, in, count, keep, state), "dropout");
}

void reduce_columns(ReduceOp op, DType out, DType in, std::byte* results, const std::byte* data, std::int64_t outer,
                    std::int64_t inner) {
    check(kd_reduce_columns(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in), results, data, outer,
                            inner),
          "reduce_columns");
}

void causal_attention(DType dtype, std::byte* out, std::byte* lse, const std::byte* qkv, std::int64_t batch,
                      std::int64_t length, std::int64_t heads, std::int64_t head_dim) {
    check(kd_causal_attention(static_cast<int>(dtype), out, lse, qkv, batch, length, heads, head_dim),
          "causal_attention");
}

void causal_attention_backward(DType dtype, std::byte* dqkv, const std::byte* dout, const std::byte* qkv,
                               const std::byte* out, const std::byte* lse, std::int64_t batch, std::int64_t length,
                               std::int64_t heads, std::int64_t head_dim) {
    check(kd_causal_attention_backward(static_cast<int>(dtype), dqkv, dout, qkv, out, lse, batch, length, heads,
                                       head_dim),
          "causal_attention_backward");
}

void cached_attention(DType dtype, std::byte* out, const std::byte* q, const std::int64_t* q_strides,
                      const std::byte* k, const std::int64_t* k_strides, const std::byte* v,
                      const std::int64_t* v_strides, std::int64_t batch, std::int64_t heads, std::int64_t length,
                      std::int64_t keys, std::int64_t head_dim) {
    check(kd_cached_attention(static_cast<int>(dtype), out, q, q_strides, k, k_strides, v, v_strides, batch, heads,
                              length, keys, head_dim),
          "cached_attention");
}

void index_bounds(const std::int64_t* indices, std::int64_t count, std::int64_t stride, std::int64_t bounds[2]) {
    check(kd_index_bounds(indices, count, stride, bounds), "index_bounds");
}

namespace {

kd_gpt_config engine_config(const GptEngineShape& s) {
    kd_gpt_config c{};
    c.vocab_size = s.vocab_size;
    c.max_positions = s.max_positions;
    c.layers = s.layers;
    c.heads = s.heads;
    c.dimension = s.dimension;
    c.tanh_gelu = s.tanh_gelu ? 1 : 0;
    c.flags = 0;
    return c;
}

} // namespace

bool gpt_engine_supported(const GptEngineShape& shape) {
    const kd_gpt_config c = engine_config(shape);
    return kd_gpt_supported(&c) == KD_OK;
}

void* gpt_engine_create(const GptEngineShape& shape) {
    const kd_gpt_config c = engine_config(shape);
    void* engine = nullptr;
    check(kd_gpt_create(&engine, &c), "gpt_engine_create");
    return engine;
}

void gpt_engine_destroy(void* engine) noexcept { kd_gpt_destroy(engine); }

void gpt_engine_load(void* engine, const char* name, const std::byte* device_data, std::int64_t count) {
    check(kd_gpt_load_parameter_device(engine, name, reinterpret_cast<const float*>(device_data), count),
          "gpt_engine_load");
}

std::int64_t gpt_engine_prefill(void* engine, const std::int64_t* prompt, std::int64_t length) {
    check(kd_gpt_prefill(engine, prompt, length), "gpt_engine_prefill");
    std::int64_t total = 0;
    check(kd_gpt_sequence(engine, nullptr, 0, &total), "gpt_engine_prefill");
    std::vector<std::int64_t> ids(static_cast<std::size_t>(total));
    check(kd_gpt_sequence(engine, ids.data(), total, &total), "gpt_engine_prefill");
    return ids.back();
}

void gpt_engine_decode(void* engine, std::int64_t count, std::int64_t* tokens) {
    check(kd_gpt_decode(engine, count, tokens), "gpt_engine_decode");
}

static_assert(kGptSampleMaxVocab == KD_GPT_SAMPLE_MAX_VOCAB);

void gpt_engine_set_sampling(void* engine, double temperature, std::int64_t top_k) {
    check(kd_gpt_set_sampling(engine, temperature, top_k), "gpt_engine_set_sampling");
}

void gpt_engine_set_uniforms(void* engine, const double* uniforms, std::int64_t count) {
    check(kd_gpt_set_uniforms(engine, uniforms, count), "gpt_engine_set_uniforms");
}

} // namespace kael::device
