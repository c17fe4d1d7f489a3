// kd_index.hip - gather and scatter_add for gfx950.
//
// Contract of reference src/cuda/kernels.inl:179-221 and 447-465: element e of the index
// space decodes to (index position, source position, data position) with IndexLayout's
// element strides; the data position along `axis` comes from indices[]. gather copies
// data -> out[e] (out is contiguous in e), scatter_add atomically adds source into data (i64
// wraps because two's-complement addition is the same operation as unsigned addition).
// Indices are range-checked by the host before the call (src/internal/index_checks.h:37-43).
//
// Decoding uses multiply-high division per dim. When the innermost dim is not the indexed
// axis, is contiguous in data and source and the indices do not vary along it (an embedding
// lookup, index_select, index_add_), the index space is a set of rows: one wave per row decodes
// the row and loads its index once, then copies (gather, 16-byte vectors when the row starts
// allow) or atomically adds (scatter) the row's elements, all lanes' loads issued before their
// stores. Otherwise every element is decoded on its own.
//
// kd_index_bounds returns the smallest and largest of a strided run of indices in one call (the
// range check kael makes before a device gather or scatter, and on cross-entropy targets): one
// or more workgroups fold their share, a second launch combines the workgroups' pairs, and the
// last launch writes the pair into a pinned host slot that is read after one stream sync.
#include <algorithm>
#include <climits>
#include <mutex>
#include <vector>

#include "kd_internal.h"

namespace kd {

namespace {

constexpr int kThreads = 256;

struct IndexPlan {
    int dims;
    int axis;
    FastDiv div[KD_MAX_DIMS];  // innermost first
    int64_t data_stride[KD_MAX_DIMS];
    int64_t index_stride[KD_MAX_DIMS];
    int64_t source_stride[KD_MAX_DIMS];
    int axis_slot;             // position of `axis` in the innermost-first order
    int64_t axis_data_stride;
};

struct Position {
    int64_t data, index, source;
};

__device__ __forceinline__ Position locate(const IndexPlan& p, const int64_t* __restrict__ indices, uint32_t e) {
    Position pos{0, 0, 0};
    for (int k = 0; k < p.dims; ++k) {
        const uint32_t q = p.div[k].div(e);
        const int64_t c = static_cast<int64_t>(e - q * p.div[k].divisor);
        e = q;
        pos.index += c * p.index_stride[k];
        pos.source += c * p.source_stride[k];
        if (k != p.axis_slot) pos.data += c * p.data_stride[k];
    }
    pos.data += indices[pos.index] * p.axis_data_stride;
    return pos;
}

// Row mode: the data and source offsets of the first element of row r (the index space with the
// innermost dim dropped).
__device__ __forceinline__ Position locate_row(const IndexPlan& p, const int64_t* __restrict__ indices, uint32_t r) {
    Position pos{0, 0, 0};
    for (int k = 1; k < p.dims; ++k) {
        const uint32_t q = p.div[k].div(r);
        const int64_t c = static_cast<int64_t>(r - q * p.div[k].divisor);
        r = q;
        pos.index += c * p.index_stride[k];
        pos.source += c * p.source_stride[k];
        if (k != p.axis_slot) pos.data += c * p.data_stride[k];
    }
    pos.data += indices[pos.index] * p.axis_data_stride;
    return pos;
}

template <typename T, int N> struct alignas(sizeof(T) * N) Vec {
    T v[N];
};

constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 4;

// out[r][0 .. inner) = data row of r, in chunks of V elements (V > 1 only when every row start of
// data and out is 16-byte aligned and inner is a multiple of V).
template <typename T, int V>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(T* __restrict__ out, const T* __restrict__ data,
                                                               const int64_t* __restrict__ indices, IndexPlan p,
                                                               uint32_t rows, uint32_t inner) {
    using Chunk = Vec<T, V>;
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const uint32_t chunks = inner / V;
    for (uint32_t r = blockIdx.x * kWaves + wave; r < rows; r += gridDim.x * kWaves) {
        const Chunk* __restrict__ src = reinterpret_cast<const Chunk*>(data + locate_row(p, indices, r).data);
        Chunk* __restrict__ dst = reinterpret_cast<Chunk*>(out + static_cast<int64_t>(r) * inner);
        uint32_t c = lane;
        for (; c + (kUnroll - 1) * 64 < chunks; c += kUnroll * 64) {
            Chunk x[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) x[u] = src[c + u * 64];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) dst[c + u * 64] = x[u];
        }
        for (; c < chunks; c += 64) dst[c] = src[c];
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void gather_kernel(T* __restrict__ out, const T* __restrict__ data,
                                                          const int64_t* __restrict__ indices, IndexPlan p,
                                                          uint32_t count) {
    for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < count; e += gridDim.x * kThreads) {
        out[e] = data[locate(p, indices, e).data];
    }
}

__device__ __forceinline__ void atomic_add_value(float* t, float v) { atomicAdd(t, v); }
__device__ __forceinline__ void atomic_add_value(double* t, double v) { atomicAdd(t, v); }
__device__ __forceinline__ void atomic_add_value(int64_t* t, int64_t v) {
    atomicAdd(reinterpret_cast<unsigned long long*>(t), static_cast<unsigned long long>(v));
}

template <typename T>
__global__ __launch_bounds__(kThreads) void scatter_add_kernel(T* data, const int64_t* __restrict__ indices,
                                                               const T* __restrict__ source, IndexPlan p,
                                                               uint32_t count) {
    for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < count; e += gridDim.x * kThreads) {
        const Position pos = locate(p, indices, e);
        atomic_add_value(data + pos.data, source[pos.source]);
    }
}

// Row mode of scatter_add: data row of r += source row of r, element by element with atomics.
template <typename T>
__global__ __launch_bounds__(kThreads) void scatter_rows_kernel(T* data, const int64_t* __restrict__ indices,
                                                                const T* __restrict__ source, IndexPlan p,
                                                                uint32_t rows, uint32_t inner) {
    const uint32_t lane = threadIdx.x % 64;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    for (uint32_t r = blockIdx.x * kWaves + wave; r < rows; r += gridDim.x * kWaves) {
        const Position pos = locate_row(p, indices, r);
        T* dst = data + pos.data;
        const T* __restrict__ src = source + pos.source;
        uint32_t c = lane;
        for (; c + (kUnroll - 1) * 64 < inner; c += kUnroll * 64) {
            T x[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) x[u] = src[c + u * 64];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) atomic_add_value(dst + c + u * 64, x[u]);
        }
        for (; c < inner; c += 64) atomic_add_value(dst + c, src[c]);
    }
}

// 64-bit decode for index spaces of 2^31 elements or more.
template <typename T, bool Scatter>
__global__ __launch_bounds__(kThreads) void index64_kernel(T* out_or_data, const T* in, const int64_t* indices,
                                                           kd_index_layout l) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; e < l.count;
         e += static_cast<int64_t>(gridDim.x) * kThreads) {
        int64_t rem = e, d = 0, ix = 0, s = 0;
        for (int dim = l.dims - 1; dim >= 0; --dim) {
            const int64_t c = rem % l.shape[dim];
            rem /= l.shape[dim];
            ix += c * l.index_strides[dim];
            s += c * l.source_strides[dim];
            if (dim != l.axis) d += c * l.data_strides[dim];
        }
        d += indices[ix] * l.data_strides[l.axis];
        if constexpr (Scatter) atomic_add_value(out_or_data + d, in[s]);
        else out_or_data[e] = in[d];
    }
}

int plan(const kd_index_layout& l, IndexPlan& p) {
    if (l.dims < 1 || l.dims > KD_MAX_DIMS) return fail(KD_E_INVALID, "index layout dims out of range");
    if (l.axis < 0 || l.axis >= l.dims) return fail(KD_E_INVALID, "index layout axis out of range");
    p.dims = l.dims;
    p.axis = l.axis;
    int k = 0;
    for (int dim = l.dims - 1; dim >= 0; --dim, ++k) {
        if (l.shape[dim] <= 0) return fail(KD_E_INVALID, "index layout has an empty dim with count > 0");
        p.div[k] = FastDiv(static_cast<uint32_t>(l.shape[dim]));
        p.data_stride[k] = l.data_strides[dim];
        p.index_stride[k] = l.index_strides[dim];
        p.source_stride[k] = l.source_strides[dim];
        if (dim == l.axis) p.axis_slot = k;
    }
    p.axis_data_stride = l.data_strides[l.axis];
    return KD_OK;
}

// Row mode applies when the innermost dim is not the indexed axis, is contiguous in data (and,
// for scatter, in source), the indices are constant along it, and rows are long enough to keep
// a wave busy.
bool row_mode(const IndexPlan& p, bool scatter) {
    return p.dims >= 2 && p.axis_slot != 0 && p.index_stride[0] == 0 && p.data_stride[0] == 1 &&
           (!scatter || p.source_stride[0] == 1) && p.div[0].divisor >= 64;
}

int row_grid(uint32_t rows) {
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((int64_t{rows} + kWaves - 1) / kWaves,
                                                                    int64_t{compute_units()} * 32)));
}

int grid_for(int64_t count) {
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((count + kThreads - 1) / kThreads,
                                                                    int64_t{compute_units()} * 32)));
}

template <typename T> int gather_typed(void* out, const void* data, const int64_t* indices, const kd_index_layout& l) {
    if (l.count < (int64_t{1} << 31)) {
        IndexPlan p;
        if (int rc = plan(l, p)) return rc;
        if (row_mode(p, false)) {
            constexpr int V = 16 / sizeof(T);
            const uint32_t inner = p.div[0].divisor, rows = static_cast<uint32_t>(l.count / inner);
            bool vec = inner % V == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(data) % 16 == 0;
            for (int k = 1; k < p.dims; ++k) vec = vec && p.data_stride[k] % V == 0;
            if (vec)
                hipLaunchKernelGGL((gather_rows_kernel<T, V>), dim3(row_grid(rows)), dim3(kThreads), 0, stream(),
                                   static_cast<T*>(out), static_cast<const T*>(data), indices, p, rows, inner);
            else
                hipLaunchKernelGGL((gather_rows_kernel<T, 1>), dim3(row_grid(rows)), dim3(kThreads), 0, stream(),
                                   static_cast<T*>(out), static_cast<const T*>(data), indices, p, rows, inner);
            KD_LAUNCH_CHECK();
            return KD_OK;
        }
        hipLaunchKernelGGL((gather_kernel<T>), dim3(grid_for(l.count)), dim3(kThreads), 0, stream(), static_cast<T*>(out),
                           static_cast<const T*>(data), indices, p, static_cast<uint32_t>(l.count));
    } else {
        hipLaunchKernelGGL((index64_kernel<T, false>), dim3(grid_for(l.count)), dim3(kThreads), 0, stream(),
                           static_cast<T*>(out), static_cast<const T*>(data), indices, l);
    }
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <typename T> int scatter_typed(void* data, const int64_t* indices, const void* source, const kd_index_layout& l) {
    if (l.count < (int64_t{1} << 31)) {
        IndexPlan p;
        if (int rc = plan(l, p)) return rc;
        if (row_mode(p, true)) {
            const uint32_t inner = p.div[0].divisor, rows = static_cast<uint32_t>(l.count / inner);
            hipLaunchKernelGGL((scatter_rows_kernel<T>), dim3(row_grid(rows)), dim3(kThreads), 0, stream(),
                               static_cast<T*>(data), indices, static_cast<const T*>(source), p, rows, inner);
            KD_LAUNCH_CHECK();
            return KD_OK;
        }
        hipLaunchKernelGGL((scatter_add_kernel<T>), dim3(grid_for(l.count)), dim3(kThreads), 0, stream(),
                           static_cast<T*>(data), indices, static_cast<const T*>(source), p, static_cast<uint32_t>(l.count));
    } else {
        hipLaunchKernelGGL((index64_kernel<T, true>), dim3(grid_for(l.count)), dim3(kThreads), 0, stream(),
                           static_cast<T*>(data), static_cast<const T*>(source), indices, l);
    }
    KD_LAUNCH_CHECK();
    return KD_OK;
}

// ---- index bounds ------------------------------------------------------------------------

constexpr int kBoundsThreads = 1024;
constexpr int64_t kBoundsPerBlock = int64_t{kBoundsThreads} * 16;  // elements one workgroup folds
constexpr int kBoundsMaxBlocks = 512;

__device__ __forceinline__ void fold_bounds(int64_t& lo, int64_t& hi, int64_t v) {
    lo = v < lo ? v : lo;
    hi = v > hi ? v : hi;
}

// Folds another (min, max) pair; an empty pair is (INT64_MAX, INT64_MIN) and changes nothing.
__device__ __forceinline__ void fold_pair(int64_t& lo, int64_t& hi, int64_t other_lo, int64_t other_hi) {
    lo = other_lo < lo ? other_lo : lo;
    hi = other_hi > hi ? other_hi : hi;
}

// The workgroup's (min, max) over its values (lo / hi per thread) into out[0..1].
__device__ void write_bounds(int64_t lo, int64_t hi, int64_t* out) {
    __shared__ int64_t slo[kBoundsThreads / 64], shi[kBoundsThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off /= 2) {
        const int64_t other_lo = __shfl_xor(lo, off);
        const int64_t other_hi = __shfl_xor(hi, off);
        fold_pair(lo, hi, other_lo, other_hi);
    }
    const int wave = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) {
        slo[wave] = lo;
        shi[wave] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kBoundsThreads / 64; ++w) fold_pair(lo, hi, slo[w], shi[w]);
        out[0] = lo;
        out[1] = hi;
    }
}

// Workgroup b folds elements [b * per, min(count, (b + 1) * per)) of indices[i * stride].
__global__ __launch_bounds__(kBoundsThreads) void bounds_kernel(const int64_t* __restrict__ indices, int64_t count,
                                                                int64_t stride, int64_t per, int64_t* out) {
    int64_t lo = INT64_MAX, hi = INT64_MIN;
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * per;
    const int64_t end = begin + per < count ? begin + per : count;
    for (int64_t i = begin + threadIdx.x; i < end; i += kBoundsThreads) fold_bounds(lo, hi, indices[i * stride]);
    write_bounds(lo, hi, out + 2 * blockIdx.x);
}

// One workgroup: the (min, max) of `pairs` workgroup pairs.
__global__ __launch_bounds__(kBoundsThreads) void bounds_combine_kernel(const int64_t* __restrict__ partial, int64_t pairs,
                                                                        int64_t* out) {
    int64_t lo = INT64_MAX, hi = INT64_MIN;
    for (int64_t i = threadIdx.x; i < pairs; i += kBoundsThreads) fold_pair(lo, hi, partial[2 * i], partial[2 * i + 1]);
    write_bounds(lo, hi, out);
}

// Pinned host slots for the bounds pairs: each call holds one from its launch until it has read
// the pair, so calls from several host threads never share a slot. Allocated in pages on first
// need and kept for the life of the process.
class BoundsSlots {
public:
    int take(int64_t** slot) {
        std::lock_guard<std::mutex> lock(mutex_);
        if (free_.empty()) {
            void* page = nullptr;
            KD_HIP(hipHostMalloc(&page, kPage * 2 * sizeof(int64_t), hipHostMallocCoherent));
            for (int i = kPage - 1; i >= 0; --i) free_.push_back(static_cast<int64_t*>(page) + 2 * i);
        }
        *slot = free_.back();
        free_.pop_back();
        return KD_OK;
    }
    void give(int64_t* slot) {
        std::lock_guard<std::mutex> lock(mutex_);
        free_.push_back(slot);
    }

private:
    static constexpr int kPage = 256;
    std::mutex mutex_;
    std::vector<int64_t*> free_;
};

BoundsSlots& bounds_slots() {
    static BoundsSlots* slots = new BoundsSlots();  // never destroyed: outlives every caller
    return *slots;
}

int index_bounds(const int64_t* indices, int64_t count, int64_t stride, int64_t* bounds) {
    const int64_t blocks = std::min<int64_t>((count + kBoundsPerBlock - 1) / kBoundsPerBlock, kBoundsMaxBlocks);
    const int64_t per = (count + blocks - 1) / blocks;
    int64_t* slot = nullptr;
    if (int rc = bounds_slots().take(&slot)) return rc;
    struct Release {
        int64_t* slot;
        ~Release() { bounds_slots().give(slot); }
    } release{slot};
    if (blocks == 1) {
        hipLaunchKernelGGL(bounds_kernel, dim3(1), dim3(kBoundsThreads), 0, stream(), indices, count, stride, per, slot);
        KD_LAUNCH_CHECK();
    } else {
        Workspace ws;  // held until bounds_combine_kernel is enqueued
        if (int rc = workspace(ws, static_cast<size_t>(blocks) * 2 * sizeof(int64_t))) return rc;
        hipLaunchKernelGGL(bounds_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kBoundsThreads), 0, stream(), indices,
                           count, stride, per, static_cast<int64_t*>(ws.ptr));
        KD_LAUNCH_CHECK();
        hipLaunchKernelGGL(bounds_combine_kernel, dim3(1), dim3(kBoundsThreads), 0, stream(),
                           static_cast<const int64_t*>(ws.ptr), blocks, slot);
        KD_LAUNCH_CHECK();
    }
    KD_HIP(hipStreamSynchronize(stream()));
    bounds[0] = slot[0];
    bounds[1] = slot[1];
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

extern "C" int kd_index_bounds(const int64_t* indices, int64_t count, int64_t stride, int64_t* bounds) {
    if (indices == nullptr || bounds == nullptr || count <= 0)
        return fail(KD_E_INVALID, "kd_index_bounds: needs indices, a bounds pair and count > 0");
    if (int rc = ensure_device()) return rc;
    return index_bounds(indices, count, stride, bounds);
}

extern "C" int kd_gather(int dtype, void* out, const void* data, const int64_t* indices, const kd_index_layout* layout) {
    if (layout == nullptr) return fail(KD_E_INVALID, "kd_gather: null layout");
    if (layout->count == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    switch (dtype) {
    case KD_F32: return gather_typed<float>(out, data, indices, *layout);
    case KD_F64: return gather_typed<double>(out, data, indices, *layout);
    case KD_I64: return gather_typed<int64_t>(out, data, indices, *layout);
    case KD_BOOL: return gather_typed<uint8_t>(out, data, indices, *layout);
    }
    return fail(KD_E_INVALID, "kd_gather: unknown dtype");
}

extern "C" int kd_scatter_add(int dtype, void* data, const int64_t* indices, const void* source,
                              const kd_index_layout* layout) {
    if (layout == nullptr) return fail(KD_E_INVALID, "kd_scatter_add: null layout");
    if (layout->count == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    switch (dtype) {
    case KD_F32: return scatter_typed<float>(data, indices, source, *layout);
    case KD_F64: return scatter_typed<double>(data, indices, source, *layout);
    case KD_I64: return scatter_typed<int64_t>(data, indices, source, *layout);
    }
    return fail(KD_E_UNSUPPORTED, "kd_scatter_add: dtype must be f32, f64 or i64");
}
