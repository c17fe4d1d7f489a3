// kd_layout.cpp - host-side planning of element layouts, the part of kael's TensorIterator
// that decides what the device sees (reference src/iterator.cpp:47-63, 112-132, 152-172 and
// src/shape.cpp:123-145). Used by this backend's own host code and tests; kael itself keeps
// building its layouts with its own TensorIterator.
#include <cstring>
#include <string>

#include "kd_api.h"

namespace kd {
int fail(int status, const std::string& message);
}

extern "C" int kd_layout_build(kd_element_layout* out, int operands, const int* ranks, const int64_t* shapes,
                               const int64_t* strides, const int* element_sizes, void* const* bases) {
    using kd::fail;
    if (out == nullptr || ranks == nullptr || shapes == nullptr || strides == nullptr || element_sizes == nullptr)
        return fail(KD_E_INVALID, "kd_layout_build: null argument");
    if (operands < 1 || operands > KD_MAX_OPERANDS) return fail(KD_E_INVALID, "kd_layout_build: operand count");
    const int ndim = ranks[0];
    if (ndim < 0 || ndim > KD_MAX_DIMS) return fail(KD_E_INVALID, "kd_layout_build: output rank");

    int64_t shape[KD_MAX_DIMS];
    int64_t st[KD_MAX_OPERANDS][KD_MAX_DIMS];
    int64_t count = 1;
    for (int d = 0; d < ndim; ++d) {
        shape[d] = shapes[d];
        if (shape[d] < 0) return fail(KD_E_INVALID, "kd_layout_build: negative dim");
        count *= shape[d];
        st[0][d] = strides[d] * element_sizes[0];
    }
    // Inputs align on trailing dims; a dim of size 1 (or a missing leading dim) broadcasts
    // with stride 0 unless it already matches.
    for (int op = 1; op < operands; ++op) {
        const int r = ranks[op];
        if (r < 0 || r > ndim) return fail(KD_E_INVALID, "kd_layout_build: input rank exceeds the output rank");
        for (int d = 0; d < ndim; ++d) {
            const int src = d - (ndim - r);
            if (src < 0) {
                st[op][d] = 0;
                continue;
            }
            const int64_t size = shapes[op * KD_MAX_DIMS + src];
            if (size == shape[d]) st[op][d] = strides[op * KD_MAX_DIMS + src] * element_sizes[op];
            else if (size == 1) st[op][d] = 0;
            else return fail(KD_E_INVALID, "kd_layout_build: shapes do not broadcast");
        }
    }
    // Drop size-1 dims, then merge each dim into its outer neighbour when every operand's
    // outer stride equals inner stride x inner size.
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
        bool mergeable = true;
        for (int op = 0; op < operands; ++op)
            if (mst[op][outer] != mst[op][inner] * ms[inner]) mergeable = false;
        if (!mergeable) continue;
        ms[outer] *= ms[inner];
        for (int k = inner; k < n - 1; ++k) ms[k] = ms[k + 1];
        for (int op = 0; op < operands; ++op) {
            mst[op][outer] = mst[op][inner];
            for (int k = inner; k < n - 1; ++k) mst[op][k] = mst[op][k + 1];
        }
        --n;
    }
    std::memset(out, 0, sizeof *out);
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
    for (int op = 0; op < operands; ++op) out->base[op] = bases != nullptr ? bases[op] : nullptr;
    return KD_OK;
}
