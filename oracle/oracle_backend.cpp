// oracle_backend.cpp - TEST INFRASTRUCTURE ONLY.
//
// Defines `namespace kael::device` (reference include/kael/device_kernels.h:96-116) on top of the
// C restatement in kd_oracle.c, with host memory standing in for device memory. Linked with the
// unmodified kael core it lets kael's own host code (TensorIterator, reductions planning,
// autograd, nn) drive the oracle, so the reference's golden suite pins the restatement.
#include <atomic>
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "kael/device_kernels.h"
#include "kael/error.h"

#include "kd_kael_extensions.h"
#include "kd_oracle.h"

namespace kael::device {

namespace {

void check(int status, const char* what) {
    if (status != KD_OK) throw Error(std::string("oracle backend: ") + what + " failed: " + oracle_last_error());
}

// Call trace. With KD_ORACLE_TRACE=<path> every device call is appended to <path> as one JSON
// object per line, device pointers written as [allocation id, byte offset] (host pointers as
// null), so that a training step's exact sequence of backend calls can be replayed against the C
// ABI elsewhere (bench.py replays the traces that tests/golden/make_step_traces.py writes).
// Host-to-device copies carry their bytes (hex) when at most KD_ORACLE_TRACE_PAYLOAD bytes (default
// 64 KiB: token ids and targets, whose values index other tensors); larger copies (parameters)
// carry only their size.
std::int64_t trace_payload() {
    static const std::int64_t limit = [] {
        const char* v = std::getenv("KD_ORACLE_TRACE_PAYLOAD");
        return v != nullptr ? std::strtoll(v, nullptr, 10) : std::int64_t{64 * 1024};
    }();
    return limit;
}

struct Trace {
    std::mutex mu;
    std::FILE* file = nullptr;
    bool opened = false;
    std::map<std::uintptr_t, std::pair<std::int64_t, std::int64_t>> blocks;  // start -> (id, bytes)
    std::int64_t next_id = 0;

    std::FILE* out() {
        if (!opened) {
            opened = true;
            if (const char* path = std::getenv("KD_ORACLE_TRACE")) file = std::fopen(path, "w");
        }
        return file;
    }
};
Trace& trace() {
    static Trace t;
    return t;
}

// [id, offset] of a pointer into a live allocation, or null.
std::string tp(const void* p) {
    auto& t = trace();
    const auto a = reinterpret_cast<std::uintptr_t>(p);
    auto it = t.blocks.upper_bound(a);
    if (p == nullptr || it == t.blocks.begin()) return "null";
    --it;
    if (a >= it->first + static_cast<std::uintptr_t>(it->second.second > 0 ? it->second.second : 1)) return "null";
    return "[" + std::to_string(it->second.first) + "," + std::to_string(a - it->first) + "]";
}

std::string ints(const std::int64_t* v, int n) {
    std::string s = "[";
    for (int i = 0; i < n; ++i) s += (i ? "," : "") + std::to_string(v[i]);
    return s + "]";
}

std::string real(double v) {  // infinities and NaN as Python's json module reads them
    if (v != v) return "NaN";
    if (v > 1.7976931348623157e308) return "Infinity";
    if (v < -1.7976931348623157e308) return "-Infinity";
    char b[40];
    std::snprintf(b, sizeof b, "%.17g", v);
    return b;
}

std::string hex(const void* p, std::int64_t n) {
    static const char* digits = "0123456789abcdef";
    std::string s;
    s.reserve(static_cast<std::size_t>(2 * n));
    const auto* b = static_cast<const unsigned char*>(p);
    for (std::int64_t i = 0; i < n; ++i) {
        s += digits[b[i] >> 4];
        s += digits[b[i] & 15];
    }
    return s;
}

std::string layout_json(const kd_element_layout& l) {
    std::string s = "{\"dims\":" + std::to_string(l.dims) + ",\"operands\":" + std::to_string(l.operands) +
                    ",\"count\":" + std::to_string(l.count) + ",\"shape\":" + ints(l.shape, l.dims) + ",\"strides\":[";
    for (int o = 0; o < l.operands; ++o) s += (o ? "," : "") + ints(l.strides[o], l.dims);
    s += "],\"base\":[";
    for (int o = 0; o < l.operands; ++o) s += (o ? "," : "") + tp(l.base[o]);
    return s + "]}";
}

std::string index_json(const kd_index_layout& l) {
    return "{\"dims\":" + std::to_string(l.dims) + ",\"axis\":" + std::to_string(l.axis) + ",\"count\":" +
           std::to_string(l.count) + ",\"shape\":" + ints(l.shape, l.dims) + ",\"data_strides\":" +
           ints(l.data_strides, l.dims) + ",\"index_strides\":" + ints(l.index_strides, l.dims) +
           ",\"source_strides\":" + ints(l.source_strides, l.dims) + "}";
}

// Writes one record (`body` holds the fields after "op"), under the trace lock.
void emit(const char* op, const std::string& body) {
    std::FILE* f = trace().out();
    if (f == nullptr) return;
    std::fprintf(f, "{\"op\":\"%s\"%s%s}\n", op, body.empty() ? "" : ",", body.c_str());
}

#define KD_TRACE(op, body)                                      \
    do {                                                        \
        std::lock_guard<std::mutex> trace_lock(trace().mu);     \
        if (trace().out() != nullptr) emit(op, body);           \
    } while (0)

std::string kv(const char* key, const std::string& value) { return std::string("\"") + key + "\":" + value; }
std::string kv(const char* key, std::int64_t value) { return kv(key, std::to_string(value)); }

} // namespace

bool available() { return true; }
void synchronize() {}

std::byte* allocate(std::int64_t bytes) {
    void* p = std::malloc(static_cast<std::size_t>(bytes > 0 ? bytes : 1));
    if (p == nullptr) throw Error("oracle backend: out of memory");
    std::lock_guard<std::mutex> lock(trace().mu);
    if (trace().out() != nullptr) {
        const std::int64_t id = trace().next_id++;
        trace().blocks[reinterpret_cast<std::uintptr_t>(p)] = {id, bytes};
        emit("alloc", kv("id", id) + "," + kv("bytes", bytes));
    }
    return static_cast<std::byte*>(p);
}

void release(std::byte* block) noexcept {
    {
        std::lock_guard<std::mutex> lock(trace().mu);
        auto& blocks = trace().blocks;
        const auto it = blocks.find(reinterpret_cast<std::uintptr_t>(block));
        if (it != blocks.end()) {
            emit("free", kv("id", it->second.first));
            blocks.erase(it);
        }
    }
    std::free(block);
}

void copy_to_device(std::byte* t, const std::byte* s, std::int64_t n) {
    KD_TRACE("h2d", kv("t", tp(t)) + "," + kv("bytes", n) + (n <= trace_payload() ? ",\"data\":\"" + hex(s, n) + "\"" : ""));
    std::memcpy(t, s, static_cast<std::size_t>(n));
}
void copy_to_host(std::byte* t, const std::byte* s, std::int64_t n) {
    KD_TRACE("d2h", kv("s", tp(s)) + "," + kv("bytes", n));
    std::memcpy(t, s, static_cast<std::size_t>(n));
}
void copy_within_device(std::byte* t, const std::byte* s, std::int64_t n) {
    KD_TRACE("d2d", kv("t", tp(t)) + "," + kv("s", tp(s)) + "," + kv("bytes", n));
    std::memmove(t, s, static_cast<std::size_t>(n));
}

void fill(DType dtype, std::byte* target, std::int64_t count, const void* value) {
    KD_TRACE("fill", kv("dtype", static_cast<int>(dtype)) + "," + kv("t", tp(target)) + "," + kv("count", count) + "," +
                         kv("value", "\"" + hex(value, element_size(dtype)) + "\""));
    check(oracle_fill(static_cast<int>(dtype), target, count, value), "fill");
}

void convert(DType out, DType in, const ElementLayout& layout) {
    const auto& l = reinterpret_cast<const kd_element_layout&>(layout);
    KD_TRACE("convert", kv("out", static_cast<int>(out)) + "," + kv("in", static_cast<int>(in)) + "," + kv("layout", layout_json(l)));
    check(oracle_convert(static_cast<int>(out), static_cast<int>(in), &l), "convert");
}

void elementwise(ElementOp op, DType out, DType in, const ElementLayout& layout, ElementParameters p) {
    kd_element_parameters kp;
    kp.reals[0] = p.reals[0];
    kp.reals[1] = p.reals[1];
    kp.integers[0] = p.integers[0];
    kp.integers[1] = p.integers[1];
    KD_TRACE("elementwise", kv("eop", static_cast<int>(op)) + "," + kv("out", static_cast<int>(out)) + "," +
                                kv("in", static_cast<int>(in)) + "," +
                                kv("layout", layout_json(reinterpret_cast<const kd_element_layout&>(layout))) + "," +
                                kv("reals", "[" + real(kp.reals[0]) + "," + real(kp.reals[1]) + "]") + "," +
                                kv("ints", ints(kp.integers, 2)));
    check(oracle_elementwise(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in),
                             reinterpret_cast<const kd_element_layout*>(&layout), kp),
          "elementwise");
}

void reduce(ReduceOp op, DType out, DType in, std::byte* results, const std::byte* data, std::int64_t chunk,
            std::int64_t rows) {
    KD_TRACE("reduce", kv("rop", static_cast<int>(op)) + "," + kv("out", static_cast<int>(out)) + "," +
                           kv("in", static_cast<int>(in)) + "," + kv("results", tp(results)) + "," + kv("data", tp(data)) +
                           "," + kv("chunk", chunk) + "," + kv("rows", rows));
    check(oracle_reduce(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in), results, data, chunk, rows),
          "reduce");
}

void matmul(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& s) {
    const kd_matmul_sizes sizes{s.batches, s.rows, s.inner, s.columns};
    KD_TRACE("matmul", kv("dtype", static_cast<int>(dtype)) + "," + kv("a", tp(a)) + "," + kv("b", tp(b)) + "," +
                           kv("c", tp(out)) + "," + kv("sizes", ints(&sizes.batches, 4)));
    check(oracle_matmul(static_cast<int>(dtype), a, b, out, &sizes, 0), "matmul");
}

void gather(DType dtype, std::byte* out, const std::byte* data, const std::int64_t* indices, const IndexLayout& l) {
    KD_TRACE("gather", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," + kv("data", tp(data)) + "," +
                           kv("indices", tp(indices)) + "," +
                           kv("layout", index_json(reinterpret_cast<const kd_index_layout&>(l))));
    check(oracle_gather(static_cast<int>(dtype), out, data, indices, reinterpret_cast<const kd_index_layout*>(&l)),
          "gather");
}

void scatter_add(DType dtype, std::byte* data, const std::int64_t* indices, const std::byte* source,
                 const IndexLayout& l) {
    KD_TRACE("scatter_add", kv("dtype", static_cast<int>(dtype)) + "," + kv("data", tp(data)) + "," +
                                kv("indices", tp(indices)) + "," + kv("source", tp(source)) + "," +
                                kv("layout", index_json(reinterpret_cast<const kd_index_layout&>(l))));
    check(oracle_scatter_add(static_cast<int>(dtype), data, indices, source, reinterpret_cast<const kd_index_layout*>(&l)),
          "scatter_add");
}

// The fused entry points of kael.cpp_amd/host/kd_kael_extensions.h, over the same restatement.
// Each call is counted so that tests can check that the patched kael branches ran.

namespace {
// 0 softmax_rows, 1 standardize_rows, 2 cross_entropy_rows, 3 cross_entropy_grad,
// 4 gelu_backward_op, 5 matmul_strided, 6 adam_step, 7 sgd_step, 8 reduce_extra,
// 9 arg_reduce, 10 cumsum_rows, 11 softmax_rows_backward, 12 standardize_rows_backward,
// 13 reduce_columns, 14 adam_step_many, 15 matmul_strided_heads, 16 layer_norm_rows,
// 17 layer_norm_rows_backward, 18 matmul_strided_bias, 19 index_bounds, 20 causal_attention,
// 21 causal_attention_backward, 22 dropout, 23 cached_attention.
constexpr int kExtensions = 24;
std::atomic<long long> g_extension_calls[kExtensions];
} // namespace

void softmax_rows(DType dtype, std::byte* out, const std::byte* in, std::int64_t rows, std::int64_t cols, bool log) {
    ++g_extension_calls[0];
    KD_TRACE("softmax_rows", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," + kv("x", tp(in)) + "," +
                                 kv("rows", rows) + "," + kv("cols", cols) + "," + kv("log", log ? 1 : 0));
    check(oracle_softmax_rows(static_cast<int>(dtype), out, in, rows, cols, log ? 1 : 0), "softmax_rows");
}

void standardize_rows(DType dtype, std::byte* out, const std::byte* in, std::int64_t rows, std::int64_t cols,
                      double eps) {
    ++g_extension_calls[1];
    KD_TRACE("standardize_rows", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," + kv("x", tp(in)) +
                                     "," + kv("rows", rows) + "," + kv("cols", cols) + "," + kv("eps", real(eps)));
    check(oracle_standardize_rows(static_cast<int>(dtype), out, in, rows, cols, eps, nullptr, nullptr),
          "standardize_rows");
}

void cross_entropy_rows(DType dtype, std::byte* losses, const std::byte* logits, const std::int64_t* targets,
                        std::int64_t rows, std::int64_t cols) {
    ++g_extension_calls[2];
    KD_TRACE("cross_entropy_rows", kv("dtype", static_cast<int>(dtype)) + "," + kv("losses", tp(losses)) + "," +
                                       kv("logits", tp(logits)) + "," + kv("targets", tp(targets)) + "," + kv("rows", rows) +
                                       "," + kv("cols", cols));
    check(oracle_cross_entropy_rows(static_cast<int>(dtype), losses, logits, targets, rows, cols), "cross_entropy_rows");
}

void cross_entropy_grad(DType dtype, std::byte* out, const std::byte* logits, const std::int64_t* targets,
                        const std::byte* row_weights, std::int64_t rows, std::int64_t cols) {
    ++g_extension_calls[3];
    KD_TRACE("cross_entropy_grad", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," +
                                       kv("logits", tp(logits)) + "," + kv("targets", tp(targets)) + "," +
                                       kv("weights", tp(row_weights)) + "," + kv("rows", rows) + "," + kv("cols", cols));
    check(oracle_cross_entropy_grad(static_cast<int>(dtype), out, logits, targets, row_weights, rows, cols),
          "cross_entropy_grad");
}

void softmax_rows_backward(DType dtype, std::byte* out, const std::byte* y, const std::byte* grad, std::int64_t rows,
                           std::int64_t cols, bool log) {
    ++g_extension_calls[11];
    KD_TRACE("softmax_rows_backward", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," + kv("y", tp(y)) +
                                          "," + kv("grad", tp(grad)) + "," + kv("rows", rows) + "," + kv("cols", cols) + "," +
                                          kv("log", log ? 1 : 0));
    check(oracle_softmax_rows_backward(static_cast<int>(dtype), out, y, grad, rows, cols, log ? 1 : 0),
          "softmax_rows_backward");
}

void standardize_rows_backward(DType dtype, std::byte* out, const std::byte* x, const std::byte* y,
                               const std::byte* grad, std::int64_t rows, std::int64_t cols, double eps) {
    ++g_extension_calls[12];
    KD_TRACE("standardize_rows_backward", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," +
                                              kv("x", tp(x)) + "," + kv("y", tp(y)) + "," + kv("grad", tp(grad)) + "," +
                                              kv("rows", rows) + "," + kv("cols", cols) + "," + kv("eps", real(eps)));
    check(oracle_standardize_rows_backward(static_cast<int>(dtype), out, x, y, grad, rows, cols, eps),
          "standardize_rows_backward");
}

void layer_norm_rows(DType dtype, std::byte* out, std::byte* standardized, const std::byte* in, std::int64_t rows,
                     std::int64_t cols, double eps, const std::byte* weight, const std::byte* bias) {
    ++g_extension_calls[16];
    KD_TRACE("layer_norm_rows", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," +
                                    kv("y", tp(standardized)) + "," + kv("x", tp(in)) + "," + kv("rows", rows) + "," +
                                    kv("cols", cols) + "," + kv("eps", real(eps)) + "," + kv("w", tp(weight)) + "," +
                                    kv("b", tp(bias)));
    check(oracle_layer_norm_rows(static_cast<int>(dtype), out, standardized, in, rows, cols, eps, weight, bias),
          "layer_norm_rows");
}

void layer_norm_rows_backward(DType dtype, std::byte* grad_in, std::byte* grad_weight, std::byte* grad_bias,
                              const std::byte* x, const std::byte* standardized, const std::byte* grad,
                              const std::byte* weight, std::int64_t rows, std::int64_t cols, double eps) {
    ++g_extension_calls[17];
    KD_TRACE("layer_norm_rows_backward", kv("dtype", static_cast<int>(dtype)) + "," + kv("gx", tp(grad_in)) + "," +
                                             kv("gw", tp(grad_weight)) + "," + kv("gb", tp(grad_bias)) + "," +
                                             kv("x", tp(x)) + "," + kv("y", tp(standardized)) + "," +
                                             kv("grad", tp(grad)) + "," + kv("w", tp(weight)) + "," + kv("rows", rows) +
                                             "," + kv("cols", cols) + "," + kv("eps", real(eps)));
    check(oracle_layer_norm_rows_backward(static_cast<int>(dtype), grad_in, grad_weight, grad_bias, x, standardized,
                                          grad, weight, rows, cols, eps),
          "layer_norm_rows_backward");
}

ElementOp gelu_backward_op(bool approximate) {
    ++g_extension_calls[4];
    return static_cast<ElementOp>(approximate ? KD_OP_GELU_TANH_BACKWARD : KD_OP_GELU_EXACT_BACKWARD);
}

void matmul_strided(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& s,
                    const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides) {
    ++g_extension_calls[5];
    const kd_matmul_sizes sizes{s.batches, s.rows, s.inner, s.columns};
    kd_matmul_strides st;
    for (int i = 0; i < 3; ++i) {
        st.a[i] = a_strides[i];
        st.b[i] = b_strides[i];
        st.out[i] = out_strides[i];
    }
    KD_TRACE("matmul_strided", kv("dtype", static_cast<int>(dtype)) + "," + kv("a", tp(a)) + "," + kv("b", tp(b)) + "," +
                                   kv("c", tp(out)) + "," + kv("sizes", ints(&sizes.batches, 4)) + "," + kv("sa", ints(st.a, 3)) +
                                   "," + kv("sb", ints(st.b, 3)) + "," + kv("sc", ints(st.out, 3)));
    check(oracle_matmul_strided(static_cast<int>(dtype), a, b, out, &sizes, &st), "matmul_strided");
}

void matmul_strided_bias(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& s,
                         const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides,
                         const std::byte* bias) {
    ++g_extension_calls[18];
    const kd_matmul_sizes sizes{s.batches, s.rows, s.inner, s.columns};
    kd_matmul_strides st;
    for (int i = 0; i < 3; ++i) {
        st.a[i] = a_strides[i];
        st.b[i] = b_strides[i];
        st.out[i] = out_strides[i];
    }
    KD_TRACE("matmul_strided_bias", kv("dtype", static_cast<int>(dtype)) + "," + kv("a", tp(a)) + "," + kv("b", tp(b)) +
                                        "," + kv("c", tp(out)) + "," + kv("sizes", ints(&sizes.batches, 4)) + "," +
                                        kv("sa", ints(st.a, 3)) + "," + kv("sb", ints(st.b, 3)) + "," +
                                        kv("sc", ints(st.out, 3)) + "," + kv("bias", tp(bias)));
    check(oracle_matmul_strided_bias(static_cast<int>(dtype), a, b, out, &sizes, &st, bias), "matmul_strided_bias");
}

void matmul_strided_heads(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& s,
                          const std::int64_t* a_strides, const std::int64_t* b_strides, const std::int64_t* out_strides,
                          std::int64_t heads, const std::int64_t* head_strides) {
    ++g_extension_calls[15];
    const kd_matmul_sizes sizes{s.batches, s.rows, s.inner, s.columns};
    kd_matmul_strides st;
    for (int i = 0; i < 3; ++i) {
        st.a[i] = a_strides[i];
        st.b[i] = b_strides[i];
        st.out[i] = out_strides[i];
    }
    const kd_matmul_heads h{heads, head_strides[0], head_strides[1], head_strides[2]};
    KD_TRACE("matmul_strided_heads", kv("dtype", static_cast<int>(dtype)) + "," + kv("a", tp(a)) + "," + kv("b", tp(b)) +
                                         "," + kv("c", tp(out)) + "," + kv("sizes", ints(&sizes.batches, 4)) + "," +
                                         kv("sa", ints(st.a, 3)) + "," + kv("sb", ints(st.b, 3)) + "," +
                                         kv("sc", ints(st.out, 3)) + "," + kv("heads", ints(&h.heads, 4)));
    check(oracle_matmul_strided_heads(static_cast<int>(dtype), a, b, out, &sizes, &st, &h), "matmul_strided_heads");
}

void adam_step(DType dtype, std::byte* param, const std::byte* grad, std::byte* first, std::byte* second,
               std::int64_t count, double learning_rate, double beta1, double beta2, double epsilon,
               double weight_decay, bool decoupled, std::int64_t step) {
    ++g_extension_calls[6];
    KD_TRACE("adam_step", kv("dtype", static_cast<int>(dtype)) + "," + kv("p", tp(param)) + "," + kv("g", tp(grad)) + "," +
                              kv("m", tp(first)) + "," + kv("v", tp(second)) + "," + kv("count", count) + "," +
                              kv("lr", real(learning_rate)) + "," + kv("b1", real(beta1)) + "," + kv("b2", real(beta2)) + "," +
                              kv("eps", real(epsilon)) + "," + kv("wd", real(weight_decay)) + "," +
                              kv("decoupled", decoupled ? 1 : 0) + "," + kv("step", step));
    check(oracle_adam_step(static_cast<int>(dtype), param, grad, first, second, count, learning_rate, beta1, beta2,
                           epsilon, weight_decay, decoupled ? 1 : 0, step),
          "adam_step");
}

void adam_step_many(DType dtype, const std::vector<AdamTensor>& tensors, double learning_rate, double beta1,
                    double beta2, double epsilon, double weight_decay, bool decoupled) {
    ++g_extension_calls[14];
    std::vector<kd_adam_tensor> table;
    for (const AdamTensor& t : tensors) table.push_back({t.param, t.grad, t.first, t.second, t.count, t.step});
    const auto list = [&] {  // evaluated under the trace lock
        std::string s;
        for (const AdamTensor& t : tensors)
            s += std::string(s.empty() ? "" : ",") + "{" + kv("p", tp(t.param)) + "," + kv("g", tp(t.grad)) + "," +
                 kv("m", tp(t.first)) + "," + kv("v", tp(t.second)) + "," + kv("count", t.count) + "," +
                 kv("step", t.step) + "}";
        return s;
    };
    KD_TRACE("adam_step_many", kv("dtype", static_cast<int>(dtype)) + ",\"tensors\":[" + list() + "]," +
                                   kv("lr", real(learning_rate)) + "," + kv("b1", real(beta1)) + "," + kv("b2", real(beta2)) +
                                   "," + kv("eps", real(epsilon)) + "," + kv("wd", real(weight_decay)) + "," +
                                   kv("decoupled", decoupled ? 1 : 0));
    check(oracle_adam_step_many(static_cast<int>(dtype), table.data(), static_cast<std::int64_t>(table.size()),
                                learning_rate, beta1, beta2, epsilon, weight_decay, decoupled ? 1 : 0),
          "adam_step_many");
}

void sgd_step(DType dtype, std::byte* param, const std::byte* grad, std::int64_t count, double learning_rate,
              double weight_decay) {
    ++g_extension_calls[7];
    KD_TRACE("sgd_step", kv("dtype", static_cast<int>(dtype)) + "," + kv("p", tp(param)) + "," + kv("g", tp(grad)) + "," +
                             kv("count", count) + "," + kv("lr", real(learning_rate)) + "," + kv("wd", real(weight_decay)));
    check(oracle_sgd_step(static_cast<int>(dtype), param, grad, count, learning_rate, weight_decay), "sgd_step");
}

void reduce_extra(ExtraReduceOp op, DType in, std::byte* results, const std::byte* data, std::int64_t chunk_size,
                  std::int64_t output_count) {
    ++g_extension_calls[8];
    const int code = op == ExtraReduceOp::Prod ? KD_REDUCE_PROD : op == ExtraReduceOp::All ? KD_REDUCE_ALL : KD_REDUCE_ANY;
    const int out = op != ExtraReduceOp::Prod ? KD_BOOL : (in == DType::F32 || in == DType::F64) ? static_cast<int>(in) : KD_I64;
    KD_TRACE("reduce", kv("rop", code) + "," + kv("out", out) + "," + kv("in", static_cast<int>(in)) + "," +
                           kv("results", tp(results)) + "," + kv("data", tp(data)) + "," + kv("chunk", chunk_size) + "," +
                           kv("rows", output_count));
    check(oracle_reduce(code, out, static_cast<int>(in), results, data, chunk_size, output_count), "reduce_extra");
}

void arg_reduce(bool largest, DType in, std::int64_t* results, const std::byte* data, std::int64_t chunk_size,
                std::int64_t output_count) {
    ++g_extension_calls[9];
    KD_TRACE("arg_reduce", kv("largest", largest ? 1 : 0) + "," + kv("in", static_cast<int>(in)) + "," +
                               kv("results", tp(results)) + "," + kv("data", tp(data)) + "," + kv("chunk", chunk_size) + "," +
                               kv("rows", output_count));
    check(oracle_arg_reduce(largest ? 1 : 0, static_cast<int>(in), results, data, chunk_size, output_count),
          "arg_reduce");
}

void reduce_columns(ReduceOp op, DType out, DType in, std::byte* results, const std::byte* data, std::int64_t outer,
                    std::int64_t inner) {
    ++g_extension_calls[13];
    KD_TRACE("reduce_columns", kv("rop", static_cast<int>(op)) + "," + kv("out", static_cast<int>(out)) + "," +
                                   kv("in", static_cast<int>(in)) + "," + kv("results", tp(results)) + "," +
                                   kv("data", tp(data)) + "," + kv("outer", outer) + "," + kv("inner", inner));
    check(oracle_reduce_columns(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in), results, data, outer,
                                inner),
          "reduce_columns");
}

void index_bounds(const std::int64_t* indices, std::int64_t count, std::int64_t stride, std::int64_t bounds[2]) {
    ++g_extension_calls[19];
    KD_TRACE("index_bounds", kv("indices", tp(indices)) + "," + kv("count", count) + "," + kv("stride", stride));
    check(oracle_index_bounds(indices, count, stride, bounds), "index_bounds");
}

void causal_attention(DType dtype, std::byte* out, std::byte* lse, const std::byte* qkv, std::int64_t batch,
                      std::int64_t length, std::int64_t heads, std::int64_t head_dim) {
    ++g_extension_calls[20];
    KD_TRACE("causal_attention", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," +
                                     kv("lse", tp(lse)) + "," + kv("qkv", tp(qkv)) + "," + kv("batch", batch) + "," +
                                     kv("length", length) + "," + kv("heads", heads) + "," + kv("head_dim", head_dim));
    check(oracle_causal_attention(static_cast<int>(dtype), out, lse, qkv, batch, length, heads, head_dim),
          "causal_attention");
}

void causal_attention_backward(DType dtype, std::byte* dqkv, const std::byte* dout, const std::byte* qkv,
                               const std::byte* out, const std::byte* lse, std::int64_t batch, std::int64_t length,
                               std::int64_t heads, std::int64_t head_dim) {
    ++g_extension_calls[21];
    KD_TRACE("causal_attention_backward",
             kv("dtype", static_cast<int>(dtype)) + "," + kv("dqkv", tp(dqkv)) + "," + kv("dout", tp(dout)) + "," +
                 kv("qkv", tp(qkv)) + "," + kv("out", tp(out)) + "," + kv("lse", tp(lse)) + "," + kv("batch", batch) +
                 "," + kv("length", length) + "," + kv("heads", heads) + "," + kv("head_dim", head_dim));
    check(oracle_causal_attention_backward(static_cast<int>(dtype), dqkv, dout, qkv, out, lse, batch, length, heads,
                                           head_dim),
          "causal_attention_backward");
}

void cached_attention(DType dtype, std::byte* out, const std::byte* q, const std::int64_t* q_strides,
                      const std::byte* k, const std::int64_t* k_strides, const std::byte* v,
                      const std::int64_t* v_strides, std::int64_t batch, std::int64_t heads, std::int64_t length,
                      std::int64_t keys, std::int64_t head_dim) {
    ++g_extension_calls[23];
    check(oracle_cached_attention(static_cast<int>(dtype), out, q, q_strides, k, k_strides, v, v_strides, batch,
                                  heads, length, keys, head_dim),
          "cached_attention");
}

void cumsum_rows(DType in, std::byte* out, const std::byte* data, std::int64_t size, std::int64_t rows) {
    ++g_extension_calls[10];
    KD_TRACE("cumsum", kv("in", static_cast<int>(in)) + "," + kv("out", tp(out)) + "," + kv("data", tp(data)) + "," +
                           kv("size", size) + "," + kv("rows", rows));
    check(oracle_cumsum(static_cast<int>(in), out, data, size, rows), "cumsum_rows");
}

void dropout(DType dtype, std::byte* out, std::byte* mask, const std::byte* in, std::int64_t count, double keep,
             std::uint64_t* state) {
    ++g_extension_calls[22];
    KD_TRACE("dropout", kv("dtype", static_cast<int>(dtype)) + "," + kv("out", tp(out)) + "," + kv("mask", tp(mask)) +
                            "," + kv("in", tp(in)) + "," + kv("count", count) + "," + kv("keep", real(keep)));
    check(oracle_dropout(static_cast<int>(dtype), out, mask, in, count, keep, state), "dropout");
}

// The C oracle has no GPT decode engine: nn::generate's optional branch sees an unsupported
// shape and keeps kael's own loop.
bool gpt_engine_supported(const GptEngineShape&) { return false; }
void* gpt_engine_create(const GptEngineShape&) { throw Error("oracle backend: no GPT decode engine"); }
void gpt_engine_destroy(void*) noexcept {}
void gpt_engine_load(void*, const char*, const std::byte*, std::int64_t) {
    throw Error("oracle backend: no GPT decode engine");
}
std::int64_t gpt_engine_prefill(void*, const std::int64_t*, std::int64_t) {
    throw Error("oracle backend: no GPT decode engine");
}
void gpt_engine_decode(void*, std::int64_t, std::int64_t*) { throw Error("oracle backend: no GPT decode engine"); }
void gpt_engine_set_sampling(void*, double, std::int64_t) { throw Error("oracle backend: no GPT decode engine"); }
void gpt_engine_set_uniforms(void*, const double*, std::int64_t) {
    throw Error("oracle backend: no GPT decode engine");
}

} // namespace kael::device

// Marks a point of the call trace (ref_shim.cpp's training loops mark each step's start).
extern "C" void oracle_trace_mark(const char* name) {
    using namespace kael::device;
    KD_TRACE("mark", kv("name", std::string("\"") + name + "\""));
}

// Test hook: how many times extension `which` (numbered as g_extension_calls) has run.
extern "C" long long ref_extension_calls(int which) {
    return which >= 0 && which < kael::device::kExtensions ? kael::device::g_extension_calls[which].load() : -1;
}
