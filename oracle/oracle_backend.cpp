// oracle_backend.cpp - TEST INFRASTRUCTURE ONLY.
//
// Defines `namespace kael::device` (reference include/kael/device_kernels.h:96-116) on top of the
// C restatement in kd_oracle.c, with host memory standing in for device memory. Linked with the
// unmodified kael core it lets kael's own host code (TensorIterator, reductions planning,
// autograd, nn) drive the oracle, so the reference's golden suite pins the restatement.
#include <cstdlib>
#include <cstring>
#include <string>

#include "kael/device_kernels.h"
#include "kael/error.h"

#include "kd_oracle.h"

namespace kael::device {

namespace {

void check(int status, const char* what) {
    if (status != KD_OK) throw Error(std::string("oracle backend: ") + what + " failed: " + oracle_last_error());
}

} // namespace

bool available() { return true; }
void synchronize() {}

std::byte* allocate(std::int64_t bytes) {
    void* p = std::malloc(static_cast<std::size_t>(bytes > 0 ? bytes : 1));
    if (p == nullptr) throw Error("oracle backend: out of memory");
    return static_cast<std::byte*>(p);
}

void release(std::byte* block) noexcept { std::free(block); }

void copy_to_device(std::byte* t, const std::byte* s, std::int64_t n) { std::memcpy(t, s, static_cast<std::size_t>(n)); }
void copy_to_host(std::byte* t, const std::byte* s, std::int64_t n) { std::memcpy(t, s, static_cast<std::size_t>(n)); }
void copy_within_device(std::byte* t, const std::byte* s, std::int64_t n) { std::memmove(t, s, static_cast<std::size_t>(n)); }

void fill(DType dtype, std::byte* target, std::int64_t count, const void* value) {
    check(oracle_fill(static_cast<int>(dtype), target, count, value), "fill");
}

void convert(DType out, DType in, const ElementLayout& layout) {
    check(oracle_convert(static_cast<int>(out), static_cast<int>(in), reinterpret_cast<const kd_element_layout*>(&layout)),
          "convert");
}

void elementwise(ElementOp op, DType out, DType in, const ElementLayout& layout, ElementParameters p) {
    kd_element_parameters kp;
    kp.reals[0] = p.reals[0];
    kp.reals[1] = p.reals[1];
    kp.integers[0] = p.integers[0];
    kp.integers[1] = p.integers[1];
    check(oracle_elementwise(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in),
                             reinterpret_cast<const kd_element_layout*>(&layout), kp),
          "elementwise");
}

void reduce(ReduceOp op, DType out, DType in, std::byte* results, const std::byte* data, std::int64_t chunk,
            std::int64_t rows) {
    check(oracle_reduce(static_cast<int>(op), static_cast<int>(out), static_cast<int>(in), results, data, chunk, rows),
          "reduce");
}

void matmul(DType dtype, const std::byte* a, const std::byte* b, std::byte* out, const MatmulSizes& s) {
    const kd_matmul_sizes sizes{s.batches, s.rows, s.inner, s.columns};
    check(oracle_matmul(static_cast<int>(dtype), a, b, out, &sizes, 0), "matmul");
}

void gather(DType dtype, std::byte* out, const std::byte* data, const std::int64_t* indices, const IndexLayout& l) {
    check(oracle_gather(static_cast<int>(dtype), out, data, indices, reinterpret_cast<const kd_index_layout*>(&l)),
          "gather");
}

void scatter_add(DType dtype, std::byte* data, const std::int64_t* indices, const std::byte* source,
                 const IndexLayout& l) {
    check(oracle_scatter_add(static_cast<int>(dtype), data, indices, source, reinterpret_cast<const kd_index_layout*>(&l)),
          "scatter_add");
}

} // namespace kael::device
