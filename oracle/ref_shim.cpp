// ref_shim.cpp - TEST INFRASTRUCTURE ONLY (the checker, never the product).
//
// extern "C" entry points over the reference kael C++ core, compiled unmodified from
// /root/reference/src by oracle/Makefile into oracle/_ref/libkael_ref.so. Two families:
//
//  ref_dev_*  the reference's own device tasks (src/cuda/kernels.inl) executed on the host by
//             the reference's emulation backend src/cuda/backend_fake.cpp. They take the same
//             kd_* layouts as the HIP backend and pin the C restatement in oracle/kd_oracle.c
//             at the exact device boundary (include/kael/device_kernels.h:96-116).
//  ref_*      kael's CPU path through the public tensor API (ops, nn, autograd, optim): the
//             op-level oracle and the timed CPU baseline.
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <optional>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "kael/debug.h"
#include "kael/device_kernels.h"
#include "kael/kael.h"
#include "kael/nn/layernorm.h"
#include "kael/nn/linear.h"
#include "kael/nn/loss.h"
#include "kael/nn/activation.h"
#include "kael/nn/functional.h"
#include "kael/nn/sequential.h"
#include "kael/nn/transformer.h"
#include "kael/optim/adam.h"
#include "kael/optim/sgd.h"

#include "kd_api.h"

namespace kael::detail {
// Declared in the reference's autograd sources (defined in src/ops/nn.cpp:214-240).
Tensor cross_entropy_gradient(const Tensor& logits, const Tensor& targets, const Tensor& scale);
} // namespace kael::detail

namespace {

thread_local std::string g_error;

// Marks a point of the oracle backend's call trace; defined only in the builds that link
// oracle_backend.cpp (weak: null elsewhere).
extern "C" void oracle_trace_mark(const char* name) __attribute__((weak));
void trace_mark(const char* name) {
    if (oracle_trace_mark != nullptr) oracle_trace_mark(name);
}

template <typename F> int guarded(F&& f) {
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

static_assert(sizeof(kd_element_layout) == sizeof(kael::device::ElementLayout));
static_assert(sizeof(kd_index_layout) == sizeof(kael::device::IndexLayout));
static_assert(sizeof(kd_matmul_sizes) == sizeof(kael::device::MatmulSizes));

kael::DType to_dtype(int code) { return static_cast<kael::DType>(code); }

kael::device::ElementLayout to_layout(const kd_element_layout* l) {
    kael::device::ElementLayout out{};
    std::memcpy(&out, l, sizeof(out));
    return out;
}

kael::device::IndexLayout to_index_layout(const kd_index_layout* l) {
    kael::device::IndexLayout out{};
    std::memcpy(&out, l, sizeof(out));
    return out;
}

// A CPU tensor holding a copy of `count` elements of `dtype` at `data`.
kael::Tensor host_tensor(const void* data, const kael::Shape& shape, kael::DType dtype) {
    kael::Tensor t = kael::empty(shape, dtype);
    std::memcpy(t.data_ptr_raw(), data,
                static_cast<std::size_t>(t.numel() * kael::element_size(dtype)));
    return t;
}

void copy_out(const kael::Tensor& t, void* out) {
    const kael::Tensor c = t.contiguous();
    std::memcpy(out, c.data_ptr_raw(),
                static_cast<std::size_t>(c.numel() * kael::element_size(c.dtype())));
}

} // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

void ref_set_threads(int64_t n) { kael::set_num_threads(n); }
int64_t ref_get_threads(void) { return kael::get_num_threads(); }

// ---- boundary-level: the reference device tasks, run on the host -------------------------

int ref_dev_fill(int dtype, void* target, int64_t count, const void* value) {
    return guarded([&] {
        kael::device::fill(to_dtype(dtype), static_cast<std::byte*>(target), count, value);
    });
}

int ref_dev_convert(int out, int in, const kd_element_layout* layout) {
    return guarded([&] { kael::device::convert(to_dtype(out), to_dtype(in), to_layout(layout)); });
}

int ref_dev_elementwise(int op, int out, int in, const kd_element_layout* layout,
                        kd_element_parameters p) {
    return guarded([&] {
        kael::device::ElementParameters params{};
        params.reals = {p.reals[0], p.reals[1]};
        params.integers = {p.integers[0], p.integers[1]};
        kael::device::elementwise(static_cast<kael::device::ElementOp>(op), to_dtype(out),
                                  to_dtype(in), to_layout(layout), params);
    });
}

int ref_dev_reduce(int op, int out, int in, void* results, const void* data, int64_t chunk,
                   int64_t rows) {
    return guarded([&] {
        kael::device::reduce(static_cast<kael::device::ReduceOp>(op), to_dtype(out), to_dtype(in),
                             static_cast<std::byte*>(results),
                             static_cast<const std::byte*>(data), chunk, rows);
    });
}

int ref_dev_matmul(int dtype, const void* a, const void* b, void* out,
                   const kd_matmul_sizes* sizes) {
    return guarded([&] {
        kael::device::matmul(to_dtype(dtype), static_cast<const std::byte*>(a),
                             static_cast<const std::byte*>(b), static_cast<std::byte*>(out),
                             {sizes->batches, sizes->rows, sizes->inner, sizes->columns});
    });
}

int ref_dev_gather(int dtype, void* out, const void* data, const int64_t* indices,
                   const kd_index_layout* layout) {
    return guarded([&] {
        kael::device::gather(to_dtype(dtype), static_cast<std::byte*>(out),
                             static_cast<const std::byte*>(data), indices,
                             to_index_layout(layout));
    });
}

int ref_dev_scatter_add(int dtype, void* data, const int64_t* indices, const void* source,
                        const kd_index_layout* layout) {
    return guarded([&] {
        kael::device::scatter_add(to_dtype(dtype), static_cast<std::byte*>(data), indices,
                                  static_cast<const std::byte*>(source), to_index_layout(layout));
    });
}

// ---- host-side layout planning (TensorIterator) ---------------------------------------------

// Runs kael::coalesce_dims on (shape, byte strides per operand) and writes the merged
// result. Returns the number of merged dims (or -1).
int ref_coalesce(int dims, int operands, const int64_t* shape, const int64_t* strides,
                 int64_t* out_shape, int64_t* out_strides) {
    int result = -1;
    const int rc = guarded([&] {
        kael::LoopDims loop;
        loop.shape.assign(shape, shape + dims);
        for (int op = 0; op < operands; ++op) {
            loop.operand_strides.emplace_back(strides + op * dims, strides + (op + 1) * dims);
        }
        const kael::LoopDims merged = kael::coalesce_dims(loop);
        const int n = static_cast<int>(merged.shape.size());
        for (int d = 0; d < n; ++d) {
            out_shape[d] = merged.shape[static_cast<std::size_t>(d)];
            for (int op = 0; op < operands; ++op) {
                out_strides[op * 8 + d] =
                    merged.operand_strides[static_cast<std::size_t>(op)][static_cast<std::size_t>(d)];
            }
        }
        result = n;
    });
    return rc == 0 ? result : -1;
}

// ---- op-level: kael's CPU path ----------------------------------------------------------------

int ref_matmul(int dtype, const void* a, const void* b, void* out, int64_t batches, int64_t m,
               int64_t k, int64_t n) {
    return guarded([&] {
        const kael::DType dt = to_dtype(dtype);
        const kael::Tensor ta = host_tensor(a, {batches, m, k}, dt);
        const kael::Tensor tb = host_tensor(b, {batches, k, n}, dt);
        copy_out(kael::matmul(ta, tb), out);
    });
}

int ref_softmax(int dtype, void* out, const void* in, int64_t rows, int64_t cols, int log) {
    return guarded([&] {
        const kael::Tensor x = host_tensor(in, {rows, cols}, to_dtype(dtype));
        copy_out(log ? kael::log_softmax(x, -1) : kael::softmax(x, -1), out);
    });
}

// kael's CPU reductions of a [rows, cols] tensor along dim 1: what = 0 prod, 1 all, 2 any,
// 3 argmax, 4 argmin, 5 cumsum (src/ops/reduce.cpp, src/ops/sequence.cpp).
int ref_host_reduce(int what, int dtype, void* out, const void* in, int64_t rows, int64_t cols) {
    return guarded([&] {
        const kael::Tensor x = host_tensor(in, {rows, cols}, to_dtype(dtype));
        switch (what) {
        case 0: copy_out(kael::prod(x, {1}), out); break;
        case 1: copy_out(kael::all(x, {1}), out); break;
        case 2: copy_out(kael::any(x, {1}), out); break;
        case 3: copy_out(kael::argmax(x, 1), out); break;
        case 4: copy_out(kael::argmin(x, 1), out); break;
        case 5: copy_out(kael::cumsum(x, 1), out); break;
        default: throw std::runtime_error("ref_host_reduce: unknown reduction");
        }
    });
}

int ref_layer_norm(int dtype, void* out, const void* in, int64_t rows, int64_t cols, double eps,
                   const void* weight, const void* bias) {
    return guarded([&] {
        const kael::DType dt = to_dtype(dtype);
        const kael::Tensor x = host_tensor(in, {rows, cols}, dt);
        kael::Tensor y = kael::standardize(x, 1, eps);
        if (weight != nullptr) {
            y = y * host_tensor(weight, {cols}, dt) + host_tensor(bias, {cols}, dt);
        }
        copy_out(y, out);
    });
}

int ref_cross_entropy(int dtype, void* losses, const void* logits, const int64_t* targets,
                      int64_t rows, int64_t cols) {
    return guarded([&] {
        const kael::Tensor x = host_tensor(logits, {rows, cols}, to_dtype(dtype));
        const kael::Tensor t = host_tensor(targets, {rows}, kael::DType::I64);
        copy_out(kael::cross_entropy_losses(x, t), losses);
    });
}

int ref_cross_entropy_grad(int dtype, void* out, const void* logits, const int64_t* targets,
                           const void* weights, int64_t rows, int64_t cols) {
    return guarded([&] {
        const kael::DType dt = to_dtype(dtype);
        const kael::Tensor x = host_tensor(logits, {rows, cols}, dt);
        const kael::Tensor t = host_tensor(targets, {rows}, kael::DType::I64);
        const kael::Tensor w = host_tensor(weights, {rows}, dt);
        copy_out(kael::detail::cross_entropy_gradient(x, t, w), out);
    });
}

// g * gelu'(x) through kael's autograd (GeluBackward, src/autograd/functions_math.cpp:221-231).
int ref_gelu_backward(int dtype, void* out, const void* x, const void* g, int64_t n,
                      int approximate) {
    return guarded([&] {
        const kael::DType dt = to_dtype(dtype);
        kael::Tensor tx = host_tensor(x, {n}, dt);
        tx.requires_grad_();
        const kael::Tensor y = kael::gelu(tx, approximate != 0);
        y.backward(host_tensor(g, {n}, dt));
        copy_out(*tx.grad(), out);
    });
}

// ---- workloads (inputs from kael's own RNG, as the benchmark configs specify) ------------------

// rand(shape)*2-1 after manual_seed(seed): the matmul / elementwise config recipe.
int ref_uniform_pm1(uint64_t seed, int64_t count, float* out) {
    return guarded([&] {
        kael::manual_seed(seed);
        copy_out(kael::rand({count}) * 2 - 1, out);
    });
}

// Times `iters` calls of kael::matmul on f32 [m,k]x[k,n] CPU tensors (after one warm-up call)
// and returns the median seconds per call.
int ref_time_matmul(int64_t m, int64_t k, int64_t n, int iters, double* median_seconds) {
    return guarded([&] {
        kael::manual_seed(0);
        const kael::Tensor a = kael::rand({m, k}) * 2 - 1;
        const kael::Tensor b = kael::rand({k, n}) * 2 - 1;
        (void)kael::matmul(a, b);
        std::vector<double> times;
        for (int i = 0; i < iters; ++i) {
            const auto t0 = std::chrono::steady_clock::now();
            const kael::Tensor c = kael::matmul(a, b);
            const auto t1 = std::chrono::steady_clock::now();
            times.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(times.begin(), times.end());
        *median_seconds = times[times.size() / 2];
    });
}

// Times one of the elementwise/reduction ops of the C2 config on CPU tensors; `which`:
// 0 a+b, 1 a*b, 2 a.T()+b, 3 sum(a,{1}), 4 max(a). Median seconds per call.
// The reference's own device benchmark bodies (benchmarks/bench_cuda.cpp:23-52) on kael's CPU path:
// which 0 = rand({n}) + rand({n}), 1 = sum(rand({n})), 2 = matmul(rand({n,n}), rand({n,n})),
// 3 = nn::functional::dropout(rand({n}), 0.1, true) (a fresh mask every call); median seconds.
int ref_time_device_bench(int which, int64_t n, int iters, double* median_seconds) {
    return guarded([&] {
        kael::manual_seed(0);
        const kael::Tensor a = which == 2 ? kael::rand({n, n}) : kael::rand({n});
        const kael::Tensor b = which == 2 ? kael::rand({n, n}) : kael::rand({n});
        const auto run = [&] {
            switch (which) {
            case 0: return a + b;
            case 1: return kael::sum(a);
            case 2: return kael::matmul(a, b);
            default: return kael::nn::functional::dropout(a, 0.1, true);
            }
        };
        (void)run();
        std::vector<double> times;
        for (int i = 0; i < iters; ++i) {
            const auto t0 = std::chrono::steady_clock::now();
            const kael::Tensor c = run();
            const auto t1 = std::chrono::steady_clock::now();
            times.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(times.begin(), times.end());
        *median_seconds = times[times.size() / 2];
    });
}

int ref_time_c2(int which, int64_t rows, int64_t cols, int iters, double* median_seconds) {
    return guarded([&] {
        kael::manual_seed(1);
        const kael::Tensor a = kael::rand({rows, cols}) * 2 - 1;
        const kael::Tensor b = kael::rand({rows, 1}) * 2 - 1;
        const auto run = [&] {
            switch (which) {
            case 0: return a + b;
            case 1: return a * b;
            case 2: return a.T() + b;
            case 3: return kael::sum(a, {1});
            default: return kael::max(a);
            }
        };
        (void)run();
        std::vector<double> times;
        for (int i = 0; i < iters; ++i) {
            const auto t0 = std::chrono::steady_clock::now();
            const kael::Tensor c = run();
            const auto t1 = std::chrono::steady_clock::now();
            times.push_back(std::chrono::duration<double>(t1 - t0).count());
        }
        std::sort(times.begin(), times.end());
        *median_seconds = times[times.size() / 2];
    });
}

// ---- GPT (C5 decode) ----------------------------------------------------------------------------

struct RefGpt {
    std::unique_ptr<kael::nn::GPT> model;
    std::vector<kael::nn::NamedTensor> named;
};

void* ref_gpt_create(int64_t vocab, int64_t positions, int64_t layers, int64_t heads,
                     int64_t dimension, uint64_t seed, int tanh_gelu) {
    RefGpt* handle = nullptr;
    guarded([&] {
        kael::nn::GptConfig config;
        config.vocab_size = vocab;
        config.max_positions = positions;
        config.layers = layers;
        config.heads = heads;
        config.dimension = dimension;
        config.tanh_gelu = tanh_gelu != 0;
        kael::manual_seed(seed);
        auto h = std::make_unique<RefGpt>();
        h->model = std::make_unique<kael::nn::GPT>(config);
        h->model->eval();
        h->named = h->model->named_parameters();
        handle = h.release();
    });
    return handle;
}

void ref_gpt_destroy(void* handle) { delete static_cast<RefGpt*>(handle); }

int64_t ref_gpt_param_count(void* handle) {
    return static_cast<int64_t>(static_cast<RefGpt*>(handle)->named.size());
}

// Name (NUL-terminated into name[len]), rank and shape of parameter i; copies the values into
// `data` when it is non-NULL.
int ref_gpt_param(void* handle, int64_t i, char* name, int len, int64_t* shape, int* rank,
                  float* data) {
    return guarded([&] {
        const auto& entry = static_cast<RefGpt*>(handle)->named.at(static_cast<std::size_t>(i));
        std::snprintf(name, static_cast<std::size_t>(len), "%s", entry.first.c_str());
        const kael::Tensor& t = entry.second;
        *rank = static_cast<int>(t.dim());
        for (int d = 0; d < *rank; ++d) {
            shape[d] = t.size(d);
        }
        if (data != nullptr) {
            copy_out(t.detach(), data);
        }
    });
}

// Overwrites parameter i (the model on the CPU) with `data`, all of its elements in row-major
// order: a model with weights from elsewhere (the benchmark's own random init).
int ref_gpt_set_param(void* handle, int64_t i, const float* data) {
    return guarded([&] {
        kael::Tensor t = static_cast<RefGpt*>(handle)->named.at(static_cast<std::size_t>(i)).second;
        if (t.device() != kael::Device::CPU || !t.is_contiguous() || t.dtype() != kael::DType::F32)
            throw std::runtime_error("ref_gpt_set_param: the parameter is not a contiguous f32 CPU tensor");
        std::memcpy(t.data_ptr_raw(), data, static_cast<std::size_t>(t.numel()) * sizeof(float));
    });
}

// Full forward (no cache) of `tokens` [batch, length]; logits [batch, length, vocab].
int ref_gpt_forward(void* handle, const int64_t* tokens, int64_t batch, int64_t length,
                    float* logits) {
    return guarded([&] {
        const kael::autograd::NoGradGuard guard;
        const kael::Tensor ids = host_tensor(tokens, {batch, length}, kael::DType::I64);
        copy_out(static_cast<RefGpt*>(handle)->model->forward(ids), logits);
    });
}

// Teacher-forced cached decode: prefill tokens[0..prompt) with a KV cache, then feed
// tokens[prompt..total) one at a time. Writes the last-position logits of the prefill and of
// every step: (total - prompt + 1) rows of vocab floats.
int ref_gpt_cached_logits(void* handle, const int64_t* tokens, int64_t prompt, int64_t total,
                          float* logits) {
    return guarded([&] {
        const kael::autograd::NoGradGuard guard;
        auto& model = *static_cast<RefGpt*>(handle)->model;
        const int64_t vocab = model.config().vocab_size;
        kael::nn::KvCache cache;
        const kael::Tensor ids = host_tensor(tokens, {1, total}, kael::DType::I64);
        kael::Tensor out = model.forward(ids.narrow(1, 0, prompt), &cache);
        copy_out(out.select(1, prompt - 1), logits);
        for (int64_t t = prompt; t < total; ++t) {
            out = model.forward(ids.narrow(1, t, 1), &cache);
            copy_out(out.select(1, 0), logits + (t - prompt + 1) * vocab);
        }
    });
}

// kael::nn::generate (greedy, KV cache) of `new_tokens` after `prompt`; writes the generated
// ids and the wall seconds of the call.
int ref_gpt_generate(void* handle, const int64_t* prompt, int64_t length, int64_t new_tokens,
                     int64_t* out_tokens, double* seconds) {
    return guarded([&] {
        auto& model = *static_cast<RefGpt*>(handle)->model;
        const kael::Tensor ids = host_tensor(prompt, {1, length}, kael::DType::I64);
        const auto t0 = std::chrono::steady_clock::now();
        const kael::Tensor seq = kael::nn::generate(
            model, ids, {.max_new_tokens = new_tokens, .temperature = 0.0});
        const auto t1 = std::chrono::steady_clock::now();
        *seconds = std::chrono::duration<double>(t1 - t0).count();
        copy_out(seq, out_tokens);
    });
}

} // extern "C"

// ---- golden cases through kael's public API ---------------------------------------------------
//
// Runs one case of the reference's golden suite (tests/golden/manifest.txt; op table of
// tests/test_golden.cpp:134-232) with the inputs placed on `device` (0 = CPU, 1 = the device
// backend this library was linked with) after applying the case's view to each input. The
// result is returned contiguous on the host: dtype code, rank, shape and bytes.

namespace {

std::vector<std::string> split_text(const std::string& text, char separator) {
    std::vector<std::string> parts;
    std::string part;
    for (char ch : text) {
        if (ch == separator) {
            parts.push_back(part);
            part.clear();
        } else {
            part.push_back(ch);
        }
    }
    parts.push_back(part);
    return parts;
}

std::vector<int64_t> ints_of(const std::vector<std::string>& texts) {
    std::vector<int64_t> out;
    for (const auto& t : texts) {
        if (!t.empty()) out.push_back(std::stoll(t));
    }
    return out;
}

struct CaseArgs {
    std::vector<std::pair<std::string, std::string>> items;
    explicit CaseArgs(const std::string& encoded) {
        if (encoded.empty()) return;
        for (const auto& item : split_text(encoded, ',')) {
            const auto colon = item.find(':');
            items.emplace_back(item.substr(0, colon), colon == std::string::npos ? "" : item.substr(colon + 1));
        }
    }
    const std::string* find(const std::string& key) const {
        for (const auto& [k, v] : items) {
            if (k == key) return &v;
        }
        return nullptr;
    }
    bool has(const std::string& key) const { return find(key) != nullptr; }
    int64_t integer(const std::string& key) const { return std::stoll(*find(key)); }
    double real(const std::string& key) const { return std::stod(*find(key)); }
    bool flag(const std::string& key) const { return has(key) && *find(key) == "1"; }
    kael::Dims dims(const std::string& key) const {
        if (!has(key)) return {};
        const auto v = ints_of(split_text(*find(key), '/'));
        return kael::Dims(v.begin(), v.end());
    }
};

kael::Tensor view_of(const kael::Tensor& t, const std::string& view) {
    const auto parts = split_text(view, ':');
    const auto args = ints_of(std::vector<std::string>(parts.begin() + 1, parts.end()));
    if (parts[0] == "none") return t;
    if (parts[0] == "transpose") return t.transpose(args[0], args[1]);
    if (parts[0] == "permute") return t.permute(kael::Dims(args.begin(), args.end()));
    if (parts[0] == "slice") return t.slice(args[0], args[1], args[2], args[3]);
    if (parts[0] == "expand") return t.expand(kael::Shape(args.begin(), args.end()));
    throw kael::Error("unknown golden view " + view);
}

kael::Tensor run_golden_op(const std::string& op, std::vector<kael::Tensor>& in, const CaseArgs& a) {
    using kael::Tensor;
    if (op == "add") return kael::add(in[0], in[1]);
    if (op == "sub") return kael::sub(in[0], in[1]);
    if (op == "mul") return kael::mul(in[0], in[1]);
    if (op == "div") return kael::div(in[0], in[1]);
    if (op == "floor_divide") return kael::floor_divide(in[0], in[1]);
    if (op == "pow") return kael::pow(in[0], in[1]);
    if (op == "maximum") return kael::maximum(in[0], in[1]);
    if (op == "minimum") return kael::minimum(in[0], in[1]);
    if (op == "eq") return kael::eq(in[0], in[1]);
    if (op == "ne") return kael::ne(in[0], in[1]);
    if (op == "lt") return kael::lt(in[0], in[1]);
    if (op == "le") return kael::le(in[0], in[1]);
    if (op == "gt") return kael::gt(in[0], in[1]);
    if (op == "ge") return kael::ge(in[0], in[1]);
    if (op == "logical_and") return kael::logical_and(in[0], in[1]);
    if (op == "logical_or") return kael::logical_or(in[0], in[1]);
    if (op == "logical_xor") return kael::logical_xor(in[0], in[1]);
    if (op == "neg") return kael::neg(in[0]);
    if (op == "abs") return kael::abs(in[0]);
    if (op == "sign") return kael::sign(in[0]);
    if (op == "exp") return kael::exp(in[0]);
    if (op == "log") return kael::log(in[0]);
    if (op == "log1p") return kael::log1p(in[0]);
    if (op == "expm1") return kael::expm1(in[0]);
    if (op == "sqrt") return kael::sqrt(in[0]);
    if (op == "rsqrt") return kael::rsqrt(in[0]);
    if (op == "sin") return kael::sin(in[0]);
    if (op == "cos") return kael::cos(in[0]);
    if (op == "tanh") return kael::tanh(in[0]);
    if (op == "sigmoid") return kael::sigmoid(in[0]);
    if (op == "relu") return kael::relu(in[0]);
    if (op == "gelu") return kael::gelu(in[0]);
    if (op == "gelu_tanh") return kael::gelu(in[0], true);
    if (op == "add_") { Tensor self = in[0]; return self.add_(in[1]); }
    if (op == "sub_") { Tensor self = in[0]; return self.sub_(in[1]); }
    if (op == "mul_") { Tensor self = in[0]; return self.mul_(in[1]); }
    if (op == "div_") { Tensor self = in[0]; return self.div_(in[1]); }
    if (op == "pow_") { Tensor self = in[0]; return self.pow_(in[1]); }
    if (op == "copy_") { Tensor self = in[0]; return self.copy_(in[1]); }
    if (op == "clamp_") { Tensor self = in[0]; return self.clamp_(a.real("min"), a.real("max")); }
    if (op == "sum") return kael::sum(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "prod") return kael::prod(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "mean") return kael::mean(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "max") return kael::max(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "min") return kael::min(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "all") return kael::all(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "any") return kael::any(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "norm") return kael::norm(in[0], a.dims("dims"), a.flag("keepdim"));
    if (op == "var") return kael::var(in[0], a.dims("dims"), a.flag("keepdim"), 1);
    if (op == "std") return kael::std(in[0], a.dims("dims"), a.flag("keepdim"), 1);
    if (op == "var_correction0") return kael::var(in[0], a.dims("dims"), a.flag("keepdim"), 0);
    if (op == "argmax")
        return a.has("dim") ? kael::argmax(in[0], a.integer("dim"), a.flag("keepdim")) : kael::argmax(in[0]);
    if (op == "argmin")
        return a.has("dim") ? kael::argmin(in[0], a.integer("dim"), a.flag("keepdim")) : kael::argmin(in[0]);
    if (op == "cumsum") return kael::cumsum(in[0], a.integer("dim"));
    if (op == "matmul") return kael::matmul(in[0], in[1]);
    if (op == "dot") return kael::dot(in[0], in[1]);
    if (op == "outer") return kael::outer(in[0], in[1]);
    if (op == "cat") return kael::cat(in, a.integer("dim"));
    if (op == "stack") return kael::stack(in, a.integer("dim"));
    if (op == "where") return kael::where(in[0], in[1], in[2]);
    if (op == "masked_fill") return kael::masked_fill(in[0], in[1], a.real("value"));
    if (op == "index_select") return kael::index_select(in[0], a.integer("dim"), in[1]);
    if (op == "gather") return kael::gather(in[0], a.integer("dim"), in[1]);
    if (op == "scatter_add_") { Tensor self = in[0]; return self.scatter_add_(a.integer("dim"), in[1], in[2]); }
    if (op == "logsumexp") return kael::logsumexp(in[0], a.integer("dim"), a.flag("keepdim"));
    if (op == "softmax") return kael::softmax(in[0], a.integer("dim"));
    if (op == "log_softmax") return kael::log_softmax(in[0], a.integer("dim"));
    if (op == "clamp") return kael::clamp(in[0], a.real("min"), a.real("max"));
    throw kael::Error("no golden op " + op);
}

} // namespace

extern "C" {

// inputs: `n` base arrays (contiguous host data of dtypes[i], ranks[i], shapes[i*8..]) and a
// view string per input; `args` is the manifest's args field. Output bytes go to `out`
// (capacity `out_bytes`); returns the output byte count, or -1 on error (ref_last_error()).
int64_t ref_golden(const char* op, const char* args, int n, const void* const* datas, const int* dtypes,
                   const int* ranks, const int64_t* shapes, const char* const* views, int device, void* out,
                   int64_t out_bytes, int* out_dtype, int* out_rank, int64_t* out_shape) {
    int64_t written = -1;
    guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        std::vector<kael::Tensor> inputs;
        for (int i = 0; i < n; ++i) {
            kael::Shape shape(shapes + i * 8, shapes + i * 8 + ranks[i]);
            kael::Tensor base = host_tensor(datas[i], shape, to_dtype(dtypes[i]));
            inputs.push_back(view_of(base.to(dev), views[i]));
        }
        const kael::Tensor result = run_golden_op(op, inputs, CaseArgs(args)).cpu().contiguous();
        const int64_t bytes = result.numel() * kael::element_size(result.dtype());
        if (bytes > out_bytes) throw kael::Error("golden output buffer too small");
        std::memcpy(out, result.data_ptr_raw(), static_cast<std::size_t>(bytes));
        *out_dtype = static_cast<int>(result.dtype());
        *out_rank = static_cast<int>(result.dim());
        for (int d = 0; d < result.dim(); ++d) out_shape[d] = result.size(d);
        written = bytes;
    });
    return written;
}

int ref_device_available(void) { return kael::cuda_is_available() ? 1 : 0; }

} // extern "C"

// ---- training workloads (configs C3 and C4) through kael's autograd and optimizers ---------------

namespace {

std::vector<float> flat_parameters(const std::vector<kael::Tensor>& params) {
    std::vector<float> out;
    for (const kael::Tensor& p : params) {
        const kael::Tensor c = p.detach().cpu().contiguous();
        const float* d = c.data_ptr<float>();
        out.insert(out.end(), d, d + c.numel());
    }
    return out;
}

} // namespace

extern "C" {

// C3: Linear(784,128)-ReLU-Linear(128,10), manual_seed(2) for the Kaiming-uniform init and the
// inputs x = rand({64,784}), y = randint(0,10,{64}); cross-entropy, backward, SGD lr 0.01.
// device 0 = CPU, 1 = the linked device backend. Writes the loss of every step, the flattened
// final parameters (when params_out is non-NULL; 101770 floats) and the wall seconds of the loop.
int ref_train_mlp(int device, int64_t steps, float* losses, float* params_out, double* seconds) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(2);
        kael::nn::Sequential model{std::make_shared<kael::nn::Linear>(784, 128), std::make_shared<kael::nn::ReLU>(),
                                   std::make_shared<kael::nn::Linear>(128, 10)};
        const kael::Tensor x = kael::rand({64, 784}).to(dev);
        const kael::Tensor y = kael::randint(0, 10, {64}).to(dev);
        model.to(dev);
        kael::optim::SGD optimizer(model.parameters(), kael::optim::SgdOptions{.learning_rate = 0.01});
        const auto t0 = std::chrono::steady_clock::now();
        for (int64_t step = 0; step < steps; ++step) {
            trace_mark("step");
            optimizer.zero_grad();
            const kael::Tensor loss = kael::nn::cross_entropy(model(x), y);
            loss.backward();
            optimizer.step();
            losses[step] = loss.item<float>();
        }
        const auto t1 = std::chrono::steady_clock::now();
        *seconds = std::chrono::duration<double>(t1 - t0).count();
        if (params_out != nullptr) {
            const std::vector<float> flat = flat_parameters(model.parameters());
            std::memcpy(params_out, flat.data(), flat.size() * sizeof(float));
        }
    });
}

// `steps` steps of kael's own optimizer on one parameter of n elements (kind 0 SGD, 1 Adam,
// 2 AdamW; dtype 0 f32, 1 f64), starting from `init`; the gradient of step s is
// grads[s*n .. (s+1)*n), produced by backward of sum(p * g), which is exactly g. device 0 = CPU,
// 1 = the linked device backend. Writes the final parameter.
int ref_optim_steps(int kind, int device, int dtype, int64_t n, int64_t steps, const void* init, const void* grads,
                    void* out, double learning_rate, double beta1, double beta2, double epsilon,
                    double weight_decay) {
    return guarded([&] {
        const kael::DType dt = dtype == 0 ? kael::DType::F32 : kael::DType::F64;
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        const std::size_t es = static_cast<std::size_t>(kael::element_size(dt));
        kael::Tensor p = host_tensor(init, {n}, dt).to(dev);
        p.requires_grad_(true);
        std::unique_ptr<kael::optim::Optimizer> optimizer;
        if (kind == 0) {
            kael::optim::SgdOptions o;
            o.learning_rate = learning_rate;
            o.weight_decay = weight_decay;
            optimizer = std::make_unique<kael::optim::SGD>(std::vector<kael::Tensor>{p}, o);
        } else if (kind == 1) {
            kael::optim::AdamOptions o;
            o.learning_rate = learning_rate;
            o.beta1 = beta1;
            o.beta2 = beta2;
            o.epsilon = epsilon;
            o.weight_decay = weight_decay;
            optimizer = std::make_unique<kael::optim::Adam>(std::vector<kael::Tensor>{p}, o);
        } else {
            kael::optim::AdamWOptions o;
            o.learning_rate = learning_rate;
            o.beta1 = beta1;
            o.beta2 = beta2;
            o.epsilon = epsilon;
            o.weight_decay = weight_decay;
            optimizer = std::make_unique<kael::optim::AdamW>(std::vector<kael::Tensor>{p}, o);
        }
        for (int64_t s = 0; s < steps; ++s) {
            optimizer->zero_grad();
            const kael::Tensor g =
                host_tensor(static_cast<const std::byte*>(grads) + static_cast<std::size_t>(s * n) * es, {n}, dt).to(dev);
            kael::sum(p * g).backward();
            optimizer->step();
        }
        copy_out(p.detach().cpu(), out);
    });
}

// A char-GPT (tanh GELU) of the given size, manual_seed(3) for the N(0,0.02) init and
// ids = randint(0,vocab,{batch,context}), targets = randint(0,vocab,{batch*context}); forward,
// cross-entropy, backward, Adam (defaults). Writes each step's loss and the seconds.
// ref_train_chargpt is config C4: {vocab 96, context 128, 4 layers, 4 heads, dim 256}, batch 32.
int ref_train_gpt_params(int device, int64_t steps, int64_t vocab, int64_t context, int64_t layers, int64_t heads,
                         int64_t dimension, int64_t batch, float* losses, float* params_out, double* seconds);

int ref_train_gpt(int device, int64_t steps, int64_t vocab, int64_t context, int64_t layers, int64_t heads,
                  int64_t dimension, int64_t batch, float* losses, double* seconds) {
    return ref_train_gpt_params(device, steps, vocab, context, layers, heads, dimension, batch, losses, nullptr,
                                seconds);
}

// ref_train_gpt that also writes the flattened final parameters (GPT::parameters() order) when
// params_out is non-NULL.
int ref_train_gpt_params(int device, int64_t steps, int64_t vocab, int64_t context, int64_t layers, int64_t heads,
                         int64_t dimension, int64_t batch, float* losses, float* params_out, double* seconds) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(3);
        kael::nn::GptConfig config;
        config.vocab_size = vocab;
        config.max_positions = context;
        config.layers = layers;
        config.heads = heads;
        config.dimension = dimension;
        kael::nn::GPT model(config);
        const kael::Tensor ids = kael::randint(0, vocab, {batch, context}).to(dev);
        const kael::Tensor targets = kael::randint(0, vocab, {batch * context}).to(dev);
        model.to(dev);
        kael::optim::Adam optimizer(model.parameters());
        const auto t0 = std::chrono::steady_clock::now();
        for (int64_t step = 0; step < steps; ++step) {
            trace_mark("step");
            optimizer.zero_grad();
            const kael::Tensor logits = model(ids).reshape({batch * context, vocab});
            const kael::Tensor loss = kael::nn::cross_entropy(logits, targets);
            loss.backward();
            optimizer.step();
            losses[step] = loss.item<float>();
        }
        const auto t1 = std::chrono::steady_clock::now();
        *seconds = std::chrono::duration<double>(t1 - t0).count();
        if (params_out != nullptr) {
            const std::vector<float> flat = flat_parameters(model.parameters());
            std::memcpy(params_out, flat.data(), flat.size() * sizeof(float));
        }
    });
}

// std::mt19937_64(seed) after `skip` draws: the next `count` raw draws into `out`, then the
// engine's libstdc++ stream form (operator<<: 312 state words, then the position) into
// state_out[313].
int ref_mt_draws(uint64_t seed, int64_t skip, int64_t count, uint64_t* out, uint64_t* state_out) {
    return guarded([&] {
        std::mt19937_64 engine(seed);
        engine.discard(static_cast<unsigned long long>(skip));
        for (int64_t i = 0; i < count; ++i) out[i] = engine();
        std::stringstream words;
        words << engine;
        for (int i = 0; i < 313; ++i) words >> state_out[i];
        if (!words) throw kael::Error("ref_mt_draws: the engine's stream form is not 313 words");
    });
}

// kael::bernoulli({count}, p, dtype) on the CPU after manual_seed(seed) and `skip` draws of
// kael::rand; writes the mask and the next kael::rand F64 value (the generator's continuation).
int ref_bernoulli(uint64_t seed, int64_t skip, int dtype, int64_t count, double p, void* out, double* next) {
    return guarded([&] {
        kael::manual_seed(seed);
        if (skip > 0) (void)kael::rand({skip}, kael::DType::F64);
        copy_out(kael::bernoulli({count}, p, to_dtype(dtype)), out);
        *next = kael::rand({1}, kael::DType::F64).item<double>();
    });
}

// kael::nn::functional::dropout(x, p, true) over `count` elements of `in` (dtype code f32 / f64) on
// `device` (0 CPU, 1 the linked backend) after manual_seed(seed) and `skip` draws of kael::rand;
// writes the output and the next kael::rand F64 value. With `g` and `grad_out` non-NULL, also the
// gradient of sum(dropout(x) * g) with respect to x.
int ref_dropout(int device, uint64_t seed, int64_t skip, int dtype, const void* in, int64_t count, double p,
                void* out, double* next, const void* g, void* grad_out) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        const kael::DType dt = to_dtype(dtype);
        kael::manual_seed(seed);
        if (skip > 0) (void)kael::rand({skip}, kael::DType::F64);
        kael::Tensor x = host_tensor(in, {count}, dt).to(dev);
        if (grad_out != nullptr) x.requires_grad_(true);
        const kael::Tensor y = kael::nn::functional::dropout(x, p, true);
        copy_out(y.detach().cpu(), out);
        *next = kael::rand({1}, kael::DType::F64).item<double>();
        if (grad_out != nullptr) {
            kael::sum(y * host_tensor(g, {count}, dt).to(dev)).backward();
            copy_out(x.grad()->cpu(), grad_out);
        }
    });
}

// One forward and backward of the char-GPT that ref_train_gpt_params builds (same seed, ids and
// targets), no optimizer step: writes the loss and every parameter's gradient, flattened in
// GPT::parameters() order (ref_gpt_param_total floats), and, when params_out is non-NULL, the
// initial parameters in the same order.
int ref_gpt_grads(int device, int64_t vocab, int64_t context, int64_t layers, int64_t heads, int64_t dimension,
                  int64_t batch, float* loss_out, float* grads_out, float* params_out) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(3);
        kael::nn::GptConfig config;
        config.vocab_size = vocab;
        config.max_positions = context;
        config.layers = layers;
        config.heads = heads;
        config.dimension = dimension;
        kael::nn::GPT model(config);
        const kael::Tensor ids = kael::randint(0, vocab, {batch, context}).to(dev);
        const kael::Tensor targets = kael::randint(0, vocab, {batch * context}).to(dev);
        model.to(dev);
        if (params_out != nullptr) {
            const std::vector<float> flat = flat_parameters(model.parameters());
            std::memcpy(params_out, flat.data(), flat.size() * sizeof(float));
        }
        const kael::Tensor logits = model(ids).reshape({batch * context, vocab});
        const kael::Tensor loss = kael::nn::cross_entropy(logits, targets);
        loss.backward();
        *loss_out = loss.item<float>();
        std::vector<kael::Tensor> grads;
        for (const kael::Tensor& p : model.parameters()) {
            const std::optional<kael::Tensor> g = p.grad();
            if (!g) throw kael::Error("ref_gpt_grads: a parameter received no gradient");
            grads.push_back(*g);
        }
        const std::vector<float> flat = flat_parameters(grads);
        std::memcpy(grads_out, flat.data(), flat.size() * sizeof(float));
    });
}

// Number of parameters of the GPT that ref_train_gpt_params builds (the size of params_out).
int64_t ref_gpt_param_total(int64_t vocab, int64_t context, int64_t layers, int64_t heads, int64_t dimension) {
    int64_t total = -1;
    guarded([&] {
        kael::nn::GptConfig config;
        config.vocab_size = vocab;
        config.max_positions = context;
        config.layers = layers;
        config.heads = heads;
        config.dimension = dimension;
        kael::nn::GPT model(config);
        total = 0;
        for (const kael::Tensor& p : model.parameters()) total += p.numel();
    });
    return total;
}

// The gradient of a row op through kael's autograd on `device` (0 CPU, 1 the linked device
// backend): x [rows, cols] (dtype 0 f32, 1 f64) requires grad, y = softmax(x, -1) (kind 0),
// log_softmax(x, -1) (kind 1) or standardize(x, 1, eps) (kind 2), and sum(y * g).backward() hands
// exactly g to y's backward; writes x.grad, and y when y_out is non-NULL.
int ref_row_grad(int kind, int device, int dtype, const void* x, const void* g, int64_t rows, int64_t cols, double eps,
                 void* grad_out, void* y_out) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        const kael::DType dt = dtype == 0 ? kael::DType::F32 : kael::DType::F64;
        kael::Tensor xt = host_tensor(x, {rows, cols}, dt).to(dev);
        xt.requires_grad_(true);
        const kael::Tensor gt = host_tensor(g, {rows, cols}, dt).to(dev);
        const kael::Tensor y = kind == 0   ? kael::softmax(xt, -1)
                               : kind == 1 ? kael::log_softmax(xt, -1)
                                           : kael::standardize(xt, 1, eps);
        kael::sum(y * gt).backward();
        copy_out(xt.grad()->cpu(), grad_out);
        if (y_out != nullptr) copy_out(y.detach().cpu(), y_out);
    });
}

// Gradients of kael's tied LM-head product through its autograd on `device`
// (reference src/nn/transformer.cpp:235-236: matmul(weight, h.mT()).mT()): manual_seed(seed);
// w = (rand({n, k}) * 2 - 1) * 0.05, h = rand({batch, m, k}) * 2 - 1, gout = rand({batch, m, n}) * 2 - 1;
// sum(matmul(w, h.mT()).mT() * gout).backward(). Writes w.grad [n, k] and h.grad [batch, m, k].
int ref_head_grads(int device, int64_t batch, int64_t m, int64_t k, int64_t n, uint64_t seed, float* w_grad,
                   float* h_grad) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(seed);
        kael::Tensor w = ((kael::rand({n, k}) * 2 - 1) * 0.05).to(dev);
        kael::Tensor h = (kael::rand({batch, m, k}) * 2 - 1).to(dev);
        const kael::Tensor gout = (kael::rand({batch, m, n}) * 2 - 1).to(dev);
        w.requires_grad_(true);
        h.requires_grad_(true);
        kael::sum(kael::matmul(w, h.mT()).mT() * gout).backward();
        copy_out(w.grad()->cpu(), w_grad);
        copy_out(h.grad()->cpu(), h_grad);
    });
}

// Gradients through kael's select (reference src/autograd/functions_view.cpp:77-88) on `device` (0
// CPU, 1 the linked device backend) for the graph shapes a backward pass can give its select
// gradients: x [2, 3, 3, 4] (seeded uniform) requires grad and `which` picks the loss:
//   0  the attention split: parts = x * 1, q / k / v = parts.select(2, i) (q read transposed);
//   1  two of three indices selected from the leaf (the third slice stays zero);
//   2  the same index twice (once as dim -2) and a second index;
//   3  selects mixed with a gradient of the whole tensor (x * x);
//   4  selects along two different dims;
//   5  the split of case 0 on an intermediate that retains its gradient (also written to p_grad);
//   6  case 0 with anomaly detection on;
//   7  a select of a select, and a select along the last dim;
//   8  the split of case 0, backward twice with the graph retained (x.grad accumulates).
// Writes x.grad (72 values) and, for case 5, the intermediate's gradient (else zeros).
int ref_select_grads(int device, int which, uint64_t seed, float* x_grad, float* p_grad) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(seed);
        kael::Tensor x = (kael::rand({2, 3, 3, 4}) * 2 - 1).to(dev);
        const kael::Tensor wq = (kael::rand({3, 2, 4}) * 2 - 1).to(dev);
        const kael::Tensor wk = (kael::rand({2, 3, 4}) * 2 - 1).to(dev);
        const kael::Tensor wv = (kael::rand({2, 3, 4}) * 2 - 1).to(dev);
        const kael::Tensor wa = (kael::rand({3, 3, 4}) * 2 - 1).to(dev);
        x.requires_grad_(true);
        std::optional<kael::Tensor> retained;
        auto split = [&](const kael::Tensor& parts) {
            return kael::sum(parts.select(2, 0).transpose(0, 1) * wq) + kael::sum(parts.select(2, 1) * wk) +
                   kael::sum(parts.select(2, 2) * wv);
        };
        auto make_loss = [&]() -> kael::Tensor {
            switch (which) {
            case 0: case 6: case 8: return split(x * 1.0);
            case 1: return kael::sum(x.select(2, 0) * wk) + kael::sum(x.select(2, -1) * wv);
            case 2:
                return kael::sum(x.select(-2, 1) * wk) + kael::sum(x.select(2, 1) * wv) +
                       kael::sum(x.select(2, 0) * wq.transpose(0, 1));
            case 3: return kael::sum(x.select(2, 0) * wk) + kael::sum(x * x) + kael::sum(x.select(2, 1) * wv);
            case 4: return kael::sum(x.select(0, 1) * wa) + kael::sum(x.select(2, 2) * wv);
            case 5: {
                kael::Tensor p = x * 2.0;
                p.retain_grad();
                retained = p;
                return split(p);
            }
            case 7: return kael::sum(x.select(0, 1).select(1, 2) * wa.select(1, 0)) + kael::sum(x.select(3, 1));
            default: throw std::invalid_argument("unknown select case");
            }
        };
        const kael::Tensor loss = make_loss();
        if (which == 6) kael::set_anomaly_detection(true);
        try {
            if (which == 8) loss.backward(true);
            loss.backward();
        } catch (...) {
            if (which == 6) kael::set_anomaly_detection(false);
            throw;
        }
        if (which == 6) kael::set_anomaly_detection(false);
        copy_out(x.grad()->cpu(), x_grad);
        if (retained) {
            copy_out(retained->grad()->cpu(), p_grad);
        } else {
            std::fill(p_grad, p_grad + 72, 0.0f);
        }
    });
}

// kael's attention chain as CausalSelfAttention::forward composes it (reference
// src/nn/transformer.cpp:114-136, no cache, no dropout), op by op through kael's tensor API on
// `device` (0 CPU, 1 the linked device backend): qkv [B, T, 3 H D] (host f32) requires grad, the
// view / selects / transposes, q . k^T / sqrt(D), masked_fill with triu(ones, 1), softmax, . v,
// transpose(1, 2).contiguous(); then sum(out * dout).backward(). Writes out [B, T, H D] and
// qkv.grad.
int ref_attention_chain(int device, const float* qkv, const float* dout, int64_t batch, int64_t length,
                        int64_t heads, int64_t head_dim, float* out, float* dqkv) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        const int64_t dim = heads * head_dim;
        kael::Tensor x = host_tensor(qkv, {batch, length, 3 * dim}, kael::DType::F32).to(dev);
        x.requires_grad_(true);
        const kael::Tensor g = host_tensor(dout, {batch, length, dim}, kael::DType::F32).to(dev);
        const kael::Tensor parts = x.view({batch, length, 3, heads, head_dim});
        const kael::Tensor q = parts.select(2, 0).transpose(1, 2);
        const kael::Tensor k = parts.select(2, 1).transpose(1, 2);
        const kael::Tensor v = parts.select(2, 2).transpose(1, 2);
        const kael::Tensor mask = kael::triu(kael::ones({length, length}, kael::DType::Bool), 1).to(dev);
        const kael::Tensor scores = kael::matmul(q, k.mT()) / std::sqrt(static_cast<double>(head_dim));
        const kael::Tensor masked = kael::masked_fill(scores, mask, -std::numeric_limits<double>::infinity());
        const kael::Tensor mixed = kael::matmul(kael::softmax(masked, -1), v).transpose(1, 2).contiguous();
        const kael::Tensor y = mixed.view({batch, length, dim});
        kael::sum(y * g).backward();
        copy_out(y.detach().cpu(), out);
        copy_out(x.grad()->cpu(), dqkv);
    });
}

// kael's CausalSelfAttention module (its qkv and proj Linears and the attention; reference
// src/nn/transformer.cpp:92-138) on `device`: seeded parameters (kael's init) and input x
// [B, T, C] uniform in [-1, 1), sum(module(x) * g).backward() with g uniform. Writes the output
// (B T C), x.grad (B T C) and the parameter gradients in named_parameters() order into grads
// (3 C C + 3 C + C C + C values).
int ref_attention_module(int device, int64_t batch, int64_t length, int64_t dim, int64_t heads, uint64_t seed,
                         float* out, float* x_grad, float* grads) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(seed);
        kael::nn::CausalSelfAttention attention(dim, heads, length);
        kael::Tensor x = (kael::rand({batch, length, dim}) * 2 - 1).to(dev);
        const kael::Tensor g = (kael::rand({batch, length, dim}) * 2 - 1).to(dev);
        attention.to(dev);
        x.requires_grad_(true);
        const kael::Tensor y = attention.forward(x);
        kael::sum(y * g).backward();
        copy_out(y.detach().cpu(), out);
        copy_out(x.grad()->cpu(), x_grad);
        int64_t at = 0;
        for (auto& [name, p] : attention.named_parameters()) {
            copy_out(p.grad()->cpu(), grads + at);
            at += p.numel();
        }
    });
}

// kael's sample_next for one row of logits (reference src/nn/transformer.cpp:39-50, the
// function is internal to that file, so its four ops are called here as it calls them) with
// temperature > 0 and top_k, on the CPU path: manual_seed(seed), `skip` uniform draws
// (kael::rand of that many f64 values), then logits / temperature, topk and masked_fill when
// 0 < top_k < vocab (as sample_next tests it), softmax and multinomial of one sample. Writes the
// picked id.
int ref_sample_next(uint64_t seed, int64_t skip, const float* logits, int64_t vocab, double temperature, int64_t top_k,
                    int64_t* token) {
    return guarded([&] {
        kael::manual_seed(seed);
        if (skip > 0) (void)kael::rand({skip}, kael::DType::F64);
        const kael::Tensor last = host_tensor(logits, {1, vocab}, kael::DType::F32);
        kael::Tensor scaled = last / temperature;
        if (top_k > 0 && top_k < vocab) {  // sample_next's condition: top_k 0 (its default) masks nothing
            const kael::Tensor smallest_kept = kael::topk(scaled, top_k).values.select(-1, top_k - 1);
            scaled = kael::masked_fill(scaled, scaled < smallest_kept.unsqueeze(-1),
                                       -std::numeric_limits<double>::infinity());
        }
        const kael::Tensor next = kael::multinomial(kael::softmax(scaled, -1), 1, true);
        *token = next.item<std::int64_t>();
    });
}

// kael's CausalSelfAttention module with a KV cache (reference src/nn/transformer.cpp:103-138)
// on `device` (0 CPU, 1 the linked device backend), as generation runs it (no gradient):
// manual_seed(seed), the module for `total` positions, x [B, total, C] uniform in [-1, 1), then
// forward(x[:, :prompt], &cache) and forward(x[:, t:t+step], &cache) for t = prompt, prompt + step,
// ... (the last chunk may be shorter). Writes the outputs, concatenated along the positions, to
// out_cached (B total C) and the cacheless forward of the whole x to out_full.
int ref_cached_attention_module(int device, int64_t batch, int64_t prompt, int64_t total, int64_t step, int64_t dim,
                                int64_t heads, uint64_t seed, float* out_cached, float* out_full) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(seed);
        kael::nn::CausalSelfAttention attention(dim, heads, total);
        const kael::Tensor x = (kael::rand({batch, total, dim}) * 2 - 1).to(dev);
        attention.to(dev);
        const kael::autograd::NoGradGuard guard;
        kael::nn::LayerCache cache;
        std::vector<kael::Tensor> parts{attention.forward(x.slice(1, 0, prompt), &cache)};
        for (int64_t t = prompt; t < total; t += step)
            parts.push_back(attention.forward(x.slice(1, t, std::min(total, t + step)), &cache));
        copy_out(kael::cat(parts, 1).cpu(), out_cached);
        copy_out(attention.forward(x).cpu(), out_full);
    });
}

// kael's LayerNorm module (reference src/nn/layers.cpp:55-68) through its autograd on `device` (0
// CPU, 1 the linked device backend): weight and bias set from w / b, x [rows, cols] (dtype 0 f32,
// 1 f64) requires grad, sum(LayerNorm(x) * g).backward(). Writes the output, kael's standardize(x)
// on the same device (the rows the backward reads), x.grad, weight.grad and bias.grad.
int ref_layer_norm_grads(int device, int dtype, const void* x, const void* w, const void* b, const void* g, int64_t rows,
                         int64_t cols, double eps, void* out, void* standardized, void* grad_x, void* grad_w,
                         void* grad_b) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        const kael::DType dt = dtype == 0 ? kael::DType::F32 : kael::DType::F64;
        kael::nn::LayerNorm norm({cols}, eps, dt);
        {
            const kael::autograd::NoGradGuard guard;
            for (auto& [name, p] : norm.named_parameters()) p.copy_(host_tensor(name == "weight" ? w : b, {cols}, dt));
        }
        norm.to(dev);
        kael::Tensor xt = host_tensor(x, {rows, cols}, dt).to(dev);
        xt.requires_grad_(true);
        const kael::Tensor gt = host_tensor(g, {rows, cols}, dt).to(dev);
        const kael::Tensor y = norm.forward(xt);
        kael::sum(y * gt).backward();
        copy_out(y.detach().cpu(), out);
        copy_out(kael::autograd::without_grad([&] { return kael::standardize(xt.detach(), 1, eps); }).cpu(), standardized);
        copy_out(xt.grad()->cpu(), grad_x);
        for (const auto& [name, p] : norm.named_parameters()) copy_out(p.grad()->cpu(), name == "weight" ? grad_w : grad_b);
    });
}

// Gradients of a Linear-shaped product through kael's autograd on `device`: manual_seed(seed);
// x = rand({batch, m, k}) * 2 - 1, w = (rand({n, k}) * 2 - 1) * 0.05, gout = rand({batch, m, n}) * 2 - 1;
// y = matmul(x, w.T()) (kael's Linear, src/nn/layers.cpp:42-43); sum(y * gout).backward(). Writes
// w.grad [n, k] and x.grad [batch, m, k].
int ref_linear_grads(int device, int64_t batch, int64_t m, int64_t k, int64_t n, uint64_t seed, float* w_grad,
                     float* x_grad) {
    return guarded([&] {
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        kael::manual_seed(seed);
        kael::Tensor x = (kael::rand({batch, m, k}) * 2 - 1).to(dev);
        kael::Tensor w = ((kael::rand({n, k}) * 2 - 1) * 0.05).to(dev);
        const kael::Tensor gout = (kael::rand({batch, m, n}) * 2 - 1).to(dev);
        x.requires_grad_(true);
        w.requires_grad_(true);
        kael::sum(kael::matmul(x, w.T()) * gout).backward();
        copy_out(w.grad()->cpu(), w_grad);
        copy_out(x.grad()->cpu(), x_grad);
    });
}

// nn::generate (greedy, KV cache) on `device` with an on_token callback, as
// examples/gpt2_generate.cpp:80-92 passes one: it records every token it is handed (reading each
// [1, 1] tensor with item(), as the example's printer does) and stops the generation once it has
// seen `stop_after` tokens. Writes the returned sequence (prompt + generated; its length through
// `total`) and the tokens the callback saw (their count through `seen`).
int ref_gpt_generate_streamed(void* handle, int device, const int64_t* prompt, int64_t length, int64_t new_tokens,
                              int64_t stop_after, int64_t* out_tokens, int64_t* total, int64_t* seen_tokens,
                              int64_t* seen) {
    return guarded([&] {
        auto& model = *static_cast<RefGpt*>(handle)->model;
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        model.to(dev);
        const kael::Tensor ids = host_tensor(prompt, {1, length}, kael::DType::I64).to(dev);
        int64_t count = 0;
        const auto printer = [&](const kael::Tensor& token) {
            if (token.dim() != 2 || token.size(0) != 1 || token.size(1) != 1 || token.device() != dev)
                throw std::runtime_error("on_token got a tensor of another shape or device");
            seen_tokens[count++] = token.item<std::int64_t>();
            return count < stop_after;
        };
        const kael::Tensor seq = kael::nn::generate(
            model, ids, {.max_new_tokens = new_tokens, .temperature = 0.0, .on_token = printer});
        *total = seq.size(1);
        *seen = count;
        copy_out(seq.cpu(), out_tokens);
        model.to(kael::Device::CPU);
    });
}

int ref_train_chargpt(int device, int64_t steps, float* losses, double* seconds) {
    return ref_train_gpt(device, steps, 96, 128, 4, 4, 256, 32, losses, seconds);
}

// kael's GPT-2 small generate on `device`, timed (the drop-in path end to end).
int ref_gpt_generate_on(void* handle, int device, const int64_t* prompt, int64_t length, int64_t new_tokens,
                        int64_t* out_tokens, double* seconds) {
    return guarded([&] {
        auto& model = *static_cast<RefGpt*>(handle)->model;
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        model.to(dev);
        const kael::Tensor ids = host_tensor(prompt, {1, length}, kael::DType::I64).to(dev);
        const auto t0 = std::chrono::steady_clock::now();
        const kael::Tensor seq = kael::nn::generate(model, ids, {.max_new_tokens = new_tokens, .temperature = 0.0});
        const auto t1 = std::chrono::steady_clock::now();
        *seconds = std::chrono::duration<double>(t1 - t0).count();
        copy_out(seq.cpu(), out_tokens);
        model.to(kael::Device::CPU);
    });
}

// kael's nn::generate with sampling (temperature > 0, optional top-k; reference
// src/nn/transformer.cpp:39-50, 256-295) on `device`, after kael::manual_seed(seed), of the
// prompt repeated over `batch` rows: the loop of generate with its KV cache and sample_next
// (through kael's optional branches, a batch-1 prompt with 0 < top_k < vocab runs on the decode
// engine instead). Writes the sequence (batch x (length + new_tokens) ids), the wall time and
// the generator's next uniform draw after the call (kael::rand of one f64).
int ref_gpt_generate_sampled(void* handle, int device, const int64_t* prompt, int64_t length, int64_t batch,
                             int64_t new_tokens, double temperature, int64_t top_k, uint64_t seed, int64_t* out_tokens,
                             double* seconds, double* next_draw) {
    return guarded([&] {
        auto& model = *static_cast<RefGpt*>(handle)->model;
        const kael::Device dev = device == 0 ? kael::Device::CPU : kael::Device::CUDA;
        model.to(dev);
        std::vector<int64_t> rows;
        for (int64_t b = 0; b < batch; ++b) rows.insert(rows.end(), prompt, prompt + length);
        const kael::Tensor ids = host_tensor(rows.data(), {batch, length}, kael::DType::I64).to(dev);
        kael::manual_seed(seed);
        const auto t0 = std::chrono::steady_clock::now();
        const kael::Tensor seq = kael::nn::generate(
            model, ids, {.max_new_tokens = new_tokens, .temperature = temperature, .top_k = top_k});
        const auto t1 = std::chrono::steady_clock::now();
        *seconds = std::chrono::duration<double>(t1 - t0).count();
        copy_out(seq.cpu(), out_tokens);
        *next_draw = kael::rand({1}, kael::DType::F64).item<double>();
        model.to(kael::Device::CPU);
    });
}

} // extern "C"
