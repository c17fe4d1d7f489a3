/*
 * kd_oracle.h - TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C CPU restatement of the reference device semantics, with the same entry points
 * and argument meaning as include/kd_api.h (prefix `oracle_` instead of `kd_`). Pointers
 * are host memory. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker. Each function cites the reference lines it
 * restates.
 */
#ifndef KD_ORACLE_H
#define KD_ORACLE_H

#include "kd_api.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* oracle_last_error(void);

int oracle_fill(int dtype, void* target, int64_t count, const void* value);
int oracle_convert(int out_dtype, int in_dtype, const kd_element_layout* layout);
int oracle_elementwise(int op, int out_dtype, int in_dtype, const kd_element_layout* layout,
                       kd_element_parameters parameters);
int oracle_reduce(int op, int out_dtype, int in_dtype, void* results, const void* data,
                  int64_t chunk_size, int64_t output_count);
int oracle_reduce_columns(int op, int out_dtype, int in_dtype, void* results, const void* data,
                          int64_t outer, int64_t inner);
int oracle_index_bounds(const int64_t* indices, int64_t count, int64_t stride, int64_t* bounds);
int oracle_causal_attention(int dtype, void* out, void* lse, const void* qkv, int64_t batch, int64_t length,
                            int64_t heads, int64_t head_dim);
int oracle_causal_attention_backward(int dtype, void* dqkv, const void* dout, const void* qkv, const void* out,
                                     const void* lse, int64_t batch, int64_t length, int64_t heads, int64_t head_dim);
int oracle_sample_topk(const float* logits, int64_t vocab, double temperature, int64_t top_k, double uniform,
                       int64_t* token);
int oracle_cached_attention(int dtype, void* out, const void* q, const int64_t* q_strides, const void* k,
                            const int64_t* k_strides, const void* v, const int64_t* v_strides, int64_t batch,
                            int64_t heads, int64_t length, int64_t keys, int64_t head_dim);
int oracle_arg_reduce(int largest, int in_dtype, int64_t* results, const void* data, int64_t chunk_size,
                      int64_t output_count);
int oracle_cumsum(int in_dtype, void* out, const void* in, int64_t size, int64_t rows);
void oracle_mt19937_64_seed(uint64_t* state, uint64_t seed);
int oracle_mt19937_64_draws(uint64_t* state, int64_t count, uint64_t* out);
int oracle_bernoulli(int dtype, void* out, int64_t count, double probability, uint64_t* state);
int oracle_dropout(int dtype, void* out, void* mask, const void* in, int64_t count, double keep, uint64_t* state);
/* exact == 0: the reference device order (MatmulTiles, sequential k in T);
 * exact != 0: f32 inputs accumulated in double (error-analysis reference). */
int oracle_matmul(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                  int exact);
int oracle_matmul_strided(int dtype, const void* a, const void* b, void* out,
                          const kd_matmul_sizes* sizes, const kd_matmul_strides* strides);
int oracle_matmul_strided_bias(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                               const kd_matmul_strides* strides, const void* bias);
int oracle_matmul_strided_heads(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                                const kd_matmul_strides* strides, const kd_matmul_heads* heads);
int oracle_gather(int dtype, void* out, const void* data, const int64_t* indices,
                  const kd_index_layout* layout);
int oracle_scatter_add(int dtype, void* data, const int64_t* indices, const void* source,
                       const kd_index_layout* layout);
int oracle_softmax_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols,
                        int log_softmax);
int oracle_standardize_rows(int dtype, void* out, const void* in, int64_t rows, int64_t cols,
                            double eps, const void* weight, const void* bias);
int oracle_cross_entropy_rows(int dtype, void* losses, const void* logits, const int64_t* targets,
                              int64_t rows, int64_t cols);
int oracle_cross_entropy_grad(int dtype, void* out, const void* logits, const int64_t* targets,
                              const void* row_weights, int64_t rows, int64_t cols);
int oracle_softmax_rows_backward(int dtype, void* out, const void* y, const void* grad, int64_t rows,
                                 int64_t cols, int log_softmax);
int oracle_standardize_rows_backward(int dtype, void* out, const void* x, const void* y, const void* grad,
                                     int64_t rows, int64_t cols, double eps);
int oracle_layer_norm_rows(int dtype, void* out, void* standardized, const void* in, int64_t rows, int64_t cols,
                           double eps, const void* weight, const void* bias);
int oracle_layer_norm_rows_backward(int dtype, void* grad_in, void* grad_weight, void* grad_bias, const void* x,
                                    const void* standardized, const void* grad, const void* weight, int64_t rows,
                                    int64_t cols, double eps);
int oracle_adam_step(int dtype, void* param, const void* grad, void* first, void* second, int64_t count,
                     double learning_rate, double beta1, double beta2, double epsilon, double weight_decay,
                     int decoupled, int64_t step);
int oracle_adam_step_many(int dtype, const kd_adam_tensor* tensors, int64_t n, double learning_rate, double beta1,
                          double beta2, double epsilon, double weight_decay, int decoupled);
int oracle_sgd_step(int dtype, void* param, const void* grad, int64_t count, double learning_rate,
                    double weight_decay);
int oracle_layout_build(kd_element_layout* out, int operands, const int* ranks,
                        const int64_t* shapes, const int64_t* strides, const int* element_sizes,
                        void* const* bases);

#ifdef __cplusplus
}
#endif

#endif
