// kd_reduce.hip - row reductions (sum / max / min) over contiguous chunks for gfx950.
//
// Contract of reference src/cuda/kernels.inl:426-445: results[r] = op over
// data[r*chunk .. (r+1)*chunk). Sum accumulates in double for f32/f64 inputs and stores the
// input dtype; for i64/bool it accumulates wrapping int64 and stores int64. Max/Min are
// NaN-propagating (element_functions.h:27-43) and store the input dtype.
//
// The reference runs one thread per row (uncoalesced) and, for rows longer than 4096, a host
// loop of per-row launches with cudaMalloc'd scratch (kernels.inl:278-307). Here:
//   group  rows of <= 512 elements: a group of G lanes per row (G a power of two), so a wave
//          covers 64/G rows with coalesced loads; group reduction with cross-lane shuffles.
//   block  many long rows: one 256-lane workgroup per row, 16-byte loads, wave shuffles + LDS.
//   split  few long rows: each row is cut into S segments reduced by separate workgroups into
//          a persistent workspace, then combined in a fixed order by a second launch.
// Every path reduces in an order fixed by (chunk, rows), so results are deterministic.
//
// The same machinery serves reductions kael runs on the host today: prod (double / wrapping
// int64 accumulation, src/ops/reduce.cpp:202-219,362-369), all / any (:285-295,442-469) and
// argmax / argmin (first extreme, first NaN wins: :236-268,399-421), plus cumsum
// (src/ops/sequence.cpp:95-117) as a segmented scan.
#include <algorithm>
#include <climits>
#include <limits>
#include <cfloat>
#include <mutex>
#include <string>

#include "kd_internal.h"

namespace kd {

namespace {

constexpr int kBlock = 256;

template <int Op, typename In> struct ReduceTraits;

template <typename In> struct SumAcc {
    using type = std::conditional_t<std::is_floating_point_v<In>, double, int64_t>;
};

template <int Op, typename In> struct Combiner {
    static constexpr bool kDescending = false;  // lanes scan their elements in increasing position
    static constexpr bool kArith = Op == KD_REDUCE_SUM || Op == KD_REDUCE_PROD;
    static constexpr bool kLogical = Op == KD_REDUCE_ALL || Op == KD_REDUCE_ANY;
    using Acc = std::conditional_t<kArith, typename SumAcc<In>::type, std::conditional_t<kLogical, uint8_t, In>>;
    using Out = std::conditional_t<kArith, std::conditional_t<std::is_floating_point_v<In>, In, int64_t>,
                                   std::conditional_t<kLogical, uint8_t, In>>;
    __device__ __forceinline__ static Acc identity() {
        if constexpr (Op == KD_REDUCE_SUM || Op == KD_REDUCE_ANY) {
            return Acc(0);
        } else if constexpr (Op == KD_REDUCE_PROD || Op == KD_REDUCE_ALL) {
            return Acc(1);
        } else if constexpr (std::is_floating_point_v<In>) {
            return Op == KD_REDUCE_MAX ? static_cast<In>(-INFINITY) : static_cast<In>(INFINITY);
        } else if constexpr (std::is_same_v<In, int64_t>) {
            return Op == KD_REDUCE_MAX ? INT64_MIN : INT64_MAX;
        } else {
            return Op == KD_REDUCE_MAX ? uint8_t{0} : uint8_t{255};
        }
    }
    // `index` (the element's position in its chunk) matters only to ArgCombiner.
    __device__ __forceinline__ static Acc load(In v, int64_t) {
        if constexpr (kLogical) return v != In(0) ? uint8_t{1} : uint8_t{0};
        else return static_cast<Acc>(v);
    }
    __device__ __forceinline__ static Acc combine(Acc a, Acc b) {
        if constexpr (Op == KD_REDUCE_SUM) {
            if constexpr (std::is_same_v<Acc, int64_t>) return wrap_add(a, b);
            else return a + b;
        } else if constexpr (Op == KD_REDUCE_PROD) {
            if constexpr (std::is_same_v<Acc, int64_t>) return wrap_mul(a, b);
            else return a * b;
        } else if constexpr (Op == KD_REDUCE_ALL) {
            return a & b;
        } else if constexpr (Op == KD_REDUCE_ANY) {
            return a | b;
        } else if constexpr (Op == KD_REDUCE_MAX) {
            return max_na(a, b);
        } else {
            return min_na(a, b);
        }
    }
    __device__ __forceinline__ static Out finish(Acc a) { return static_cast<Out>(a); }
};

// (value, position) of the first extreme of a chunk: the first NaN wins, then the larger
// (Largest) or smaller value, then the smaller position - the rule of reference
// best_position, which is order independent, so every reduction tree gives the same index.
template <typename In, typename I> struct ArgAcc {
    In v;
    I i;
};

// I: the position type. Positions are relative to the chunk, so int32 serves every chunk below
// 2^31 elements (cheaper index arithmetic and one select instead of two per element); int64
// otherwise.
template <bool Largest, typename In, typename I = int64_t> struct ArgCombiner {
    using Acc = ArgAcc<In, I>;
    using Index = I;
    using Out = int64_t;
    // Each lane scans its own elements from the highest position down (block_range_down), so
    // the element being added always lies before everything the accumulator has seen: it wins
    // ties and every NaN replaces the accumulator, which leaves the first extreme (or first NaN)
    // in one compare and two selects per element instead of a full combine.
    static constexpr bool kDescending = true;
    static constexpr I kNone = std::numeric_limits<I>::max();
    __device__ __forceinline__ static Acc identity() {
        if constexpr (std::is_floating_point_v<In>) {
            return Acc{static_cast<In>(Largest ? -INFINITY : INFINITY), kNone};
        } else if constexpr (std::is_same_v<In, int64_t>) {
            return Acc{Largest ? INT64_MIN : INT64_MAX, kNone};
        } else {
            return Acc{static_cast<In>(Largest ? 0 : 255), kNone};
        }
    }
    __device__ __forceinline__ static Acc load(In v, int64_t index) { return Acc{v, static_cast<I>(index)}; }
    __device__ __forceinline__ static Acc combine(Acc a, Acc b) {
        if constexpr (std::is_floating_point_v<In>) {
            const bool an = a.v != a.v, bn = b.v != b.v;
            if (an || bn) return (an && (!bn || a.i < b.i)) ? a : b;
        }
        if (Largest ? a.v > b.v : a.v < b.v) return a;
        if (Largest ? b.v > a.v : b.v < a.v) return b;
        return a.i < b.i ? a : b;
    }
    // `a` is the identity or holds an element at a position above `index`.
    __device__ __forceinline__ static Acc step_down(Acc a, In x, I index) {
        bool take;
        if constexpr (std::is_floating_point_v<In>) take = x != x || (Largest ? x >= a.v : x <= a.v);
        else take = Largest ? x >= a.v : x <= a.v;
        return take ? Acc{x, index} : a;
    }
    __device__ __forceinline__ static Out finish(Acc a) { return static_cast<Out>(a.i); }
};

template <typename T> __device__ __forceinline__ T shfl_xor(T v, int mask) {
    if constexpr (std::is_same_v<T, uint8_t>) {
        return static_cast<uint8_t>(__shfl_xor(static_cast<int>(v), mask, 64));
    } else {
        return __shfl_xor(v, mask, 64);
    }
}

template <typename In, typename I> __device__ __forceinline__ ArgAcc<In, I> shfl_xor(ArgAcc<In, I> v, int mask) {
    return ArgAcc<In, I>{shfl_xor(v.v, mask), __shfl_xor(v.i, mask, 64)};
}

// Reduces within aligned groups of `G` lanes (G a power of two <= 64).
template <typename C, int G>
__device__ __forceinline__ typename C::Acc group_reduce(typename C::Acc v) {
#pragma unroll
    for (int m = G / 2; m > 0; m /= 2) v = C::combine(v, shfl_xor(v, m));
    return v;
}

// Whole-workgroup reduction; the result is valid in thread 0.
template <typename C>
__device__ __forceinline__ typename C::Acc block_reduce(typename C::Acc v) {
    using Acc = typename C::Acc;
    __shared__ Acc partial[kBlock / 64];
    v = group_reduce<C, 64>(v);
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    if (lane == 0) partial[wave] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        v = partial[0];
#pragma unroll
        for (int w = 1; w < kBlock / 64; ++w) v = C::combine(v, partial[w]);
    }
    __syncthreads();
    return v;
}

template <typename In> struct alignas(16) Vec16 {
    In v[16 / sizeof(In)];
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename In> __device__ __forceinline__ Vec16<In> nt_load(const Vec16<In>* p) {
    const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    Vec16<In> out;
    __builtin_memcpy(&out, &r, 16);
    return out;
}

template <typename T> __device__ __forceinline__ void nt_store(Vec16<T>* p, const Vec16<T>& v) {
    u32x4 r;
    __builtin_memcpy(&r, &v, 16);
    __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
}

// block_range for combiners with kDescending: the same lanes take the same elements, but every
// lane visits them from its highest position down - the scalar tail, its 16-byte vectors four
// at a time from the top, then the scalar head.
template <typename C, typename In>
__device__ __forceinline__ typename C::Acc block_range_down(const In* data, int64_t begin64, int64_t end64) {
    using Acc = typename C::Acc;
    using I = typename C::Index;  // positions within the chunk: the dispatch picks a type that holds them
    constexpr int V = 16 / sizeof(In);
    Acc acc = C::identity();
    const I begin = static_cast<I>(begin64);
    const I end = static_cast<I>(end64);
    const I misalign = static_cast<I>((reinterpret_cast<uintptr_t>(data + begin64) % 16) / sizeof(In));
    const I head_end = misalign != 0 ? std::min<I>(end, begin + (V - misalign)) : begin;
    const I i = head_end;
    const I vectors = (end - i) / V;
    const I t = static_cast<I>(threadIdx.x);
    for (I j = i + vectors * V + t; j < end; j += kBlock) acc = C::step_down(acc, data[j], j);  // <= 1 per lane
    const Vec16<In>* vp = reinterpret_cast<const Vec16<In>*>(data + i);
    I m = t < vectors ? (vectors - 1 - t) / kBlock + 1 : 0;  // this lane's vectors: t, t + kBlock, ...
    for (; m >= 4; m -= 4) {
        Vec16<In> x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = nt_load(vp + t + (m - 1 - u) * kBlock);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const I first = i + (t + (m - 1 - u) * kBlock) * V;
#pragma unroll
            for (int e = V - 1; e >= 0; --e) acc = C::step_down(acc, x[u].v[e], first + e);
        }
    }
    for (; m >= 1; --m) {
        const Vec16<In> x = nt_load(vp + t + (m - 1) * kBlock);
        const I first = i + (t + (m - 1) * kBlock) * V;
#pragma unroll
        for (int e = V - 1; e >= 0; --e) acc = C::step_down(acc, x.v[e], first + e);
    }
    for (I j = begin + t; j < head_end; j += kBlock) acc = C::step_down(acc, data[j], j);  // <= 1 per lane
    return block_reduce<C>(acc);
}

// Reduces data[begin, end) with all lanes of the block; 16-byte loads when `data + begin` is
// 16-byte aligned. Lane-level order is fixed by the block size.
template <typename C, typename In>
__device__ __forceinline__ typename C::Acc block_range(const In* data, int64_t begin, int64_t end) {
    if constexpr (C::kDescending) return block_range_down<C, In>(data, begin, end);
    using Acc = typename C::Acc;
    constexpr int V = 16 / sizeof(In);
    Acc acc = C::identity();
    int64_t i = begin;
    // Scalar head up to 16-byte alignment.
    const int64_t misalign = (reinterpret_cast<uintptr_t>(data + begin) % 16) / sizeof(In);
    if (misalign != 0) {
        const int64_t head_end = std::min<int64_t>(end, begin + (V - misalign));
        for (int64_t j = begin + threadIdx.x; j < head_end; j += kBlock) acc = C::combine(acc, C::load(data[j], j));
        i = head_end;
    }
    const int64_t vectors = (end - i) / V;
    const Vec16<In>* vp = reinterpret_cast<const Vec16<In>*>(data + i);
    // Four nontemporal 16-byte loads in flight per lane (the data is read exactly once).
    int64_t k = threadIdx.x;
    for (; k + 3 * kBlock < vectors; k += 4 * kBlock) {
        Vec16<In> x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = nt_load(vp + k + u * kBlock);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < V; ++e) acc = C::combine(acc, C::load(x[u].v[e], i + (k + u * kBlock) * V + e));
    }
    for (; k < vectors; k += kBlock) {
        const Vec16<In> x = nt_load(vp + k);
#pragma unroll
        for (int e = 0; e < V; ++e) acc = C::combine(acc, C::load(x.v[e], i + k * V + e));
    }
    for (int64_t j = i + vectors * V + threadIdx.x; j < end; j += kBlock) acc = C::combine(acc, C::load(data[j], j));
    return block_reduce<C>(acc);
}

template <typename C, typename In>
__global__ __launch_bounds__(kBlock) void block_kernel(typename C::Out* results, const In* data, int64_t chunk,
                                                       int64_t rows) {
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const typename C::Acc v = block_range<C, In>(data + r * chunk, 0, chunk);
        if (threadIdx.x == 0) results[r] = C::finish(v);
    }
}

template <typename C, typename In, int G>
__global__ __launch_bounds__(kBlock) void group_kernel(typename C::Out* results, const In* data, int64_t chunk,
                                                       int64_t rows) {
    constexpr int rows_per_block = kBlock / G;
    const int g = threadIdx.x / G;
    const int lane = threadIdx.x % G;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * rows_per_block; base < rows;
         base += static_cast<int64_t>(gridDim.x) * rows_per_block) {
        const int64_t r = base + g;
        typename C::Acc acc = C::identity();
        if (r < rows) {
            const In* row = data + r * chunk;
            if constexpr (C::kDescending) {
                using I = typename C::Index;
                if (lane < chunk)
                    for (I j = static_cast<I>(lane + (chunk - 1 - lane) / G * G); j >= 0; j -= G)
                        acc = C::step_down(acc, row[j], j);
            } else {
                for (int64_t j = lane; j < chunk; j += G) acc = C::combine(acc, C::load(row[j], j));
            }
        }
        acc = group_reduce<C, G>(acc);
        if (lane == 0 && r < rows) results[r] = C::finish(acc);
    }
}

template <typename C, typename In>
__global__ __launch_bounds__(kBlock) void split_kernel(typename C::Acc* partial, const In* data, int64_t chunk,
                                                       int64_t segments, int64_t segment) {
    const int64_t r = blockIdx.y;
    const int64_t s = blockIdx.x;
    const int64_t begin = s * segment;
    const int64_t end = std::min<int64_t>(chunk, begin + segment);
    const typename C::Acc v = block_range<C, In>(data + r * chunk, begin, end);
    if (threadIdx.x == 0) partial[r * segments + s] = v;
}

template <typename C>
__global__ __launch_bounds__(kBlock) void combine_kernel(typename C::Out* results, const typename C::Acc* partial,
                                                         int64_t segments) {
    // One workgroup per row: a fixed tree over the segment partials. Lane t combines partials
    // t, t + kBlock, t + 2 kBlock, ... in that order; the loads of a batch are all issued before
    // the first combine, so the partials (just written by other XCDs, read from memory) cost one
    // round trip per batch instead of one per partial.
    constexpr int kBatch = 16;
    using Acc = typename C::Acc;
    const Acc* row = partial + static_cast<int64_t>(blockIdx.x) * segments;
    Acc acc = C::identity();
    for (int64_t s0 = threadIdx.x; s0 < segments; s0 += int64_t{kBlock} * kBatch) {
        Acc v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int64_t s = s0 + int64_t{u} * kBlock;
            if (s < segments) v[u] = row[s];
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (s0 + int64_t{u} * kBlock < segments) acc = C::combine(acc, v[u]);
    }
    const int64_t r = blockIdx.x;
    acc = block_reduce<C>(acc);
    if (threadIdx.x == 0) results[r] = C::finish(acc);
}

// ---- column reductions ------------------------------------------------------------------------
//
// results[j] = op over i < outer of data[i * inner + j] for j < inner: a contiguous tensor reduced
// over its leading dims, read in place (kael's plan_reduction moves the reduced dims last with a
// transposed copy, src/ops/reduce.cpp:118-153). Workgroup (cb, s): the 64 columns [64 cb, 64 cb + 64),
// one per lane (each row read coalesced), over the segment's rows [r0, r1); wave w scans the
// contiguous rows [r0 + w q, r0 + w q + q) in increasing order, 16 loads in flight, and the four
// wave partials combine in wave order, so every column is reduced in increasing row order in
// contiguous runs (max / min keep the first NaN and the first extreme). One segment writes the
// result; several write partial[s * inner + j], which column_combine_kernel combines in segment
// order. Sums accumulate in double for f32 / f64, as kd_reduce's do.
template <typename C, typename In>
__global__ __launch_bounds__(kBlock) void column_kernel(typename C::Out* results, typename C::Acc* partial,
                                                        const In* data, int64_t outer, int64_t inner,
                                                        int64_t seg_rows, int64_t segments) {
    using Acc = typename C::Acc;
    constexpr int kWaves = kBlock / 64;
    __shared__ Acc waves[kWaves][64];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 64 + lane;
    const int64_t s = blockIdx.y;
    const int64_t r0 = s * seg_rows;
    const int64_t r1 = std::min<int64_t>(outer, r0 + seg_rows);
    const int64_t q = (r1 - r0 + kWaves - 1) / kWaves;
    const int64_t w0 = std::min<int64_t>(r1, r0 + wave * q);
    const int64_t w1 = std::min<int64_t>(r1, w0 + q);
    Acc acc = C::identity();
    if (j < inner) {
        constexpr int kRows = 16;  // loads in flight per lane
        const In* col = data + j;
        for (int64_t i0 = w0; i0 < w1; i0 += kRows) {
            In v[kRows];
#pragma unroll
            for (int u = 0; u < kRows; ++u)
                if (i0 + u < w1) v[u] = col[(i0 + u) * inner];
#pragma unroll
            for (int u = 0; u < kRows; ++u)
                if (i0 + u < w1) acc = C::combine(acc, C::load(v[u], i0 + u));
        }
    }
    waves[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && j < inner) {
        Acc v = waves[0][lane];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v = C::combine(v, waves[w][lane]);
        if (segments == 1) results[j] = C::finish(v);
        else partial[s * inner + j] = v;
    }
}

// Combines the segment partials of 64 columns per workgroup: wave w takes the contiguous segments
// [w q, w q + q) with up to 16 loads in flight per lane (the partials were just written by other
// XCDs, so each round of loads costs a trip past the L2), and the four wave results combine in
// wave order: every column in segment order.
template <typename C>
__global__ __launch_bounds__(kBlock) void column_combine_kernel(typename C::Out* results, const typename C::Acc* partial,
                                                                int64_t segments, int64_t inner) {
    constexpr int kBatch = 16;
    constexpr int kWaves = kBlock / 64;
    using Acc = typename C::Acc;
    __shared__ Acc waves[kWaves][64];
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 64 + lane;
    const int64_t q = (segments + kWaves - 1) / kWaves;
    const int64_t s_begin = std::min<int64_t>(segments, wave * q);
    const int64_t s_end = std::min<int64_t>(segments, s_begin + q);
    Acc v = C::identity();
    if (j < inner) {
        for (int64_t s0 = s_begin; s0 < s_end; s0 += kBatch) {
            Acc x[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (s0 + u < s_end) x[u] = partial[(s0 + u) * inner + j];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (s0 + u < s_end) v = C::combine(v, x[u]);
        }
    }
    waves[wave][lane] = v;
    __syncthreads();
    if (wave == 0 && j < inner) {
        Acc r = waves[0][lane];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) r = C::combine(r, waves[w][lane]);
        results[j] = C::finish(r);
    }
}

template <typename C, typename In>
int columns_with(void* results, const void* data_v, int64_t outer, int64_t inner) {
    using Acc = typename C::Acc;
    auto* out = static_cast<typename C::Out*>(results);
    const In* data = static_cast<const In*>(data_v);
    const int cus = compute_units();
    const int64_t col_blocks = (inner + 63) / 64;
    // about 4 workgroups per CU, segments of at least 64 rows
    int64_t segments = std::max<int64_t>(1, (int64_t{cus} * 4 + col_blocks - 1) / col_blocks);
    segments = std::min<int64_t>(segments, std::max<int64_t>(1, outer / 64));
    const int64_t seg_rows = std::max<int64_t>(1, (outer + segments - 1) / segments);
    segments = outer == 0 ? 1 : (outer + seg_rows - 1) / seg_rows;
    if (col_blocks > int64_t{1} << 31 || segments > 65535) return fail(KD_E_INVALID, "kd_reduce_columns: too large");
    const dim3 grid(static_cast<uint32_t>(col_blocks), static_cast<uint32_t>(segments));
    if (segments == 1) {
        hipLaunchKernelGGL((column_kernel<C, In>), grid, dim3(kBlock), 0, stream(), out, static_cast<Acc*>(nullptr), data,
                           outer, inner, seg_rows, segments);
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    Workspace ws;  // held until column_combine_kernel is enqueued
    if (int rc = workspace(ws, static_cast<size_t>(segments * inner) * sizeof(Acc))) return rc;
    Acc* partial = static_cast<Acc*>(ws.ptr);
    hipLaunchKernelGGL((column_kernel<C, In>), grid, dim3(kBlock), 0, stream(), out, partial, data, outer, inner, seg_rows,
                       segments);
    KD_LAUNCH_CHECK();
    hipLaunchKernelGGL((column_combine_kernel<C>), dim3(static_cast<uint32_t>(col_blocks)), dim3(kBlock), 0, stream(), out,
                       static_cast<const Acc*>(partial), segments, inner);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <int Op> int columns_dtype(int in, void* results, const void* data, int64_t outer, int64_t inner) {
    switch (in) {
    case KD_F32: return columns_with<Combiner<Op, float>, float>(results, data, outer, inner);
    case KD_F64: return columns_with<Combiner<Op, double>, double>(results, data, outer, inner);
    case KD_I64: return columns_with<Combiner<Op, int64_t>, int64_t>(results, data, outer, inner);
    case KD_BOOL: return columns_with<Combiner<Op, uint8_t>, uint8_t>(results, data, outer, inner);
    }
    return fail(KD_E_INVALID, "kd_reduce_columns: unknown dtype");
}

// ---- cumsum ------------------------------------------------------------------------------------

constexpr int kScanPer = 8;  // elements scanned in registers by one lane per tile

template <typename Acc> __device__ __forceinline__ Acc scan_add(Acc a, Acc b) {
    if constexpr (std::is_same_v<Acc, int64_t>) return wrap_add(a, b);
    else return a + b;
}

// Exclusive scan of one value per lane across the workgroup (waves by shuffles, then the wave
// totals through LDS); `total` receives the workgroup sum.
template <typename Acc> __device__ __forceinline__ Acc block_exclusive_scan(Acc v, Acc& total) {
    __shared__ Acc wave_sum[kBlock / 64];
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    Acc x = v;
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {
        const Acc y = __shfl_up(x, d, 64);
        if (lane >= d) x = scan_add(x, y);
    }
    Acc excl = __shfl_up(x, 1, 64);
    if (lane == 0) excl = Acc(0);
    if (lane == 63) wave_sum[wave] = x;
    __syncthreads();
    Acc before = Acc(0);
    total = Acc(0);
#pragma unroll
    for (int w = 0; w < kBlock / 64; ++w) {
        if (w < wave) before = scan_add(before, wave_sum[w]);
        total = scan_add(total, wave_sum[w]);
    }
    __syncthreads();  // wave_sum is reused by the next tile
    return scan_add(before, excl);
}

// Exclusive scans of C values per lane across the workgroup in one pass (one pair of barriers
// for all C); total[c] receives the workgroup sum of value c.
template <typename Acc, int C>
__device__ __forceinline__ void block_exclusive_scan_n(const Acc (&v)[C], Acc (&excl)[C], Acc (&total)[C]) {
    __shared__ Acc wave_sum[kBlock / 64][C];
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    Acc x[C];
#pragma unroll
    for (int c = 0; c < C; ++c) x[c] = v[c];
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const Acc y = __shfl_up(x[c], d, 64);
            if (lane >= d) x[c] = scan_add(x[c], y);
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const Acc e = __shfl_up(x[c], 1, 64);
        excl[c] = lane == 0 ? Acc(0) : e;
        if (lane == 63) wave_sum[wave][c] = x[c];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < C; ++c) {
        Acc before = Acc(0);
        Acc sum = Acc(0);
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) {
            if (w < wave) before = scan_add(before, wave_sum[w][c]);
            sum = scan_add(sum, wave_sum[w][c]);
        }
        excl[c] = scan_add(before, excl[c]);
        total[c] = sum;
    }
    __syncthreads();  // wave_sum is reused by the next tile
}

// Workgroup (s, r) scans segment s of row r (all of it when segments == 1), starting from the
// sum of the row's earlier segments (their totals come from split_kernel), in tiles of
// kBlock * kScanPer elements.
//  scalar: lane t takes kScanPer consecutive elements, scans them in registers and adds the
//          exclusive scan of the lane totals and the running carry.
//  Vec:    rows start 16-byte aligned for In and Out (of equal size) and hold a whole number
//          of 16-byte vectors (segments are multiples of them). A tile is kScanPer / V chunks of
//          kBlock vectors (V elements each) and lane t holds vector t of every chunk, so each
//          load and store instruction moves one contiguous kBlock * 16 bytes; one block scan of
//          the per-chunk lane totals serves the whole tile. The data is streamed once, with
//          nontemporal loads and stores.
template <typename In, typename Out, typename Acc, bool Vec>
__global__ __launch_bounds__(kBlock) void scan_kernel(Out* out, const In* data, int64_t size, int64_t rows,
                                                      const Acc* seg_totals, int64_t segments, int64_t segment) {
    __shared__ Acc carry_in;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const int64_t s = blockIdx.x;
        const int64_t begin = s * segment;
        const int64_t end = std::min<int64_t>(size, begin + segment);
        const In* row = data + r * size;
        Out* orow = out + r * size;
        if (segments > 1) {
            Acc c = Acc(0);
            for (int64_t k = threadIdx.x; k < s; k += kBlock) c = scan_add(c, seg_totals[r * segments + k]);
            c = block_reduce<Combiner<KD_REDUCE_SUM, In>>(c);
            if (threadIdx.x == 0) carry_in = c;
        } else if (threadIdx.x == 0) {
            carry_in = Acc(0);
        }
        __syncthreads();
        Acc carry = carry_in;
        for (int64_t base = begin; base < end; base += int64_t{kBlock} * kScanPer) {
            if constexpr (Vec) {
                constexpr int V = 16 / sizeof(In);
                constexpr int kChunks = kScanPer / V;
                Acc vals[kChunks][V];
                Acc lane_total[kChunks];
#pragma unroll
                for (int c = 0; c < kChunks; ++c) {
                    const int64_t first = base + (int64_t{c} * kBlock + threadIdx.x) * V;
                    Acc run = Acc(0);
                    if (first < end) {  // whole vector: end is a multiple of V
                        const Vec16<In> g = nt_load(reinterpret_cast<const Vec16<In>*>(row + first));
#pragma unroll
                        for (int e = 0; e < V; ++e) {
                            run = scan_add(run, static_cast<Acc>(g.v[e]));
                            vals[c][e] = run;
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < V; ++e) vals[c][e] = Acc(0);
                    }
                    lane_total[c] = run;
                }
                Acc excl[kChunks], total[kChunks];
                block_exclusive_scan_n<Acc, kChunks>(lane_total, excl, total);
#pragma unroll
                for (int c = 0; c < kChunks; ++c) {
                    const int64_t first = base + (int64_t{c} * kBlock + threadIdx.x) * V;
                    const Acc offset = scan_add(carry, excl[c]);
                    if (first < end) {
                        Vec16<Out> g;
#pragma unroll
                        for (int e = 0; e < V; ++e) g.v[e] = static_cast<Out>(scan_add(offset, vals[c][e]));
                        nt_store(reinterpret_cast<Vec16<Out>*>(orow + first), g);
                    }
                    carry = scan_add(carry, total[c]);
                }
            } else {
                const int64_t first = base + static_cast<int64_t>(threadIdx.x) * kScanPer;
                Acc vals[kScanPer];
                Acc run = Acc(0);
#pragma unroll
                for (int e = 0; e < kScanPer; ++e) {
                    const int64_t j = first + e;
                    run = scan_add(run, j < end ? static_cast<Acc>(row[j]) : Acc(0));
                    vals[e] = run;
                }
                Acc total;
                const Acc offset = scan_add(carry, block_exclusive_scan(run, total));
#pragma unroll
                for (int e = 0; e < kScanPer; ++e) {
                    const int64_t j = first + e;
                    if (j < end) orow[j] = static_cast<Out>(scan_add(offset, vals[e]));
                }
                carry = scan_add(carry, total);
            }
        }
        __syncthreads();  // carry_in is rewritten for the next row
    }
}

template <typename In> int cumsum_typed(void* out_v, const void* data_v, int64_t size, int64_t rows) {
    using Acc = typename SumAcc<In>::type;
    using Out = std::conditional_t<std::is_floating_point_v<In>, In, int64_t>;
    Out* out = static_cast<Out*>(out_v);
    const In* data = static_cast<const In*>(data_v);
    const int cus = compute_units();
    constexpr int64_t kTile = int64_t{kBlock} * kScanPer;
    // Coalesced 16-byte vectors: aligned rows holding a whole number of them, In and Out of one
    // size (f32, f64, i64).
    constexpr bool kVecType = sizeof(In) == sizeof(Out) && kScanPer * sizeof(In) % 16 == 0;
    const bool vec = kVecType && reinterpret_cast<uintptr_t>(data) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 16 == 0 && size % static_cast<int64_t>(16 / sizeof(In)) == 0;
    const auto launch = [&](dim3 grid, const Acc* totals, int64_t segments, int64_t segment) {
        if constexpr (kVecType) {
            if (vec) {
                hipLaunchKernelGGL((scan_kernel<In, Out, Acc, true>), grid, dim3(kBlock), 0, stream(), out, data, size,
                                   rows, totals, segments, segment);
                return;
            }
        }
        hipLaunchKernelGGL((scan_kernel<In, Out, Acc, false>), grid, dim3(kBlock), 0, stream(), out, data, size, rows,
                           totals, segments, segment);
    };
    if (rows >= 2 * cus || size <= 16 * kTile) {
        launch(dim3(1, static_cast<uint32_t>(std::min<int64_t>(rows, 65535))), nullptr, 1, size);
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    // Few long rows: segment totals first (the sum reduction's split kernel), then every segment
    // scans from the total of the segments before it.
    int64_t segments = std::max<int64_t>(1, (int64_t{cus} * 4 + rows - 1) / rows);
    int64_t segment = (size + segments - 1) / segments;
    segment = (std::max<int64_t>(segment, 4 * kTile) + kTile - 1) / kTile * kTile;
    segments = (size + segment - 1) / segment;
    if (rows > 65535) return fail(KD_E_INVALID, "kd_cumsum: too many rows for the split path");
    Workspace ws;  // held until the scan that reads the segment totals is enqueued
    if (int rc = workspace(ws, static_cast<size_t>(rows * segments) * sizeof(Acc))) return rc;
    const dim3 grid(static_cast<uint32_t>(segments), static_cast<uint32_t>(rows));
    hipLaunchKernelGGL((split_kernel<Combiner<KD_REDUCE_SUM, In>, In>), grid, dim3(kBlock), 0, stream(),
                       static_cast<Acc*>(ws.ptr), data, size, segments, segment);
    KD_LAUNCH_CHECK();
    launch(grid, static_cast<const Acc*>(ws.ptr), segments, segment);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

// `fixed` (non-null): the split path's partials go there, up to `fixed_bytes`, instead of the
// workspace lease (kd_reduce_noalloc); a larger need is an error.
template <typename C, typename In>
int reduce_with(void* results, const void* data_v, int64_t chunk, int64_t rows, void* fixed = nullptr,
                size_t fixed_bytes = 0) {
    using Out = typename C::Out;
    using Acc = typename C::Acc;
    Out* out = static_cast<Out*>(results);
    const In* data = static_cast<const In*>(data_v);
    const int cus = compute_units();
    if (chunk <= 512) {
        int g = 1;
        while (g < 64 && g * 8 < chunk) g *= 2;
        const int64_t rows_per_block = kBlock / g;
        const int64_t blocks = std::min<int64_t>((rows + rows_per_block - 1) / rows_per_block, int64_t{cus} * 64);
        const dim3 grid(static_cast<uint32_t>(std::max<int64_t>(blocks, 1)));
        switch (g) {
#define KD_GROUP_CASE(G)                                                                                   \
    case G:                                                                                                \
        hipLaunchKernelGGL((group_kernel<C, In, G>), grid, dim3(kBlock), 0, stream(), out, data, chunk, rows); \
        break;
            KD_GROUP_CASE(1) KD_GROUP_CASE(2) KD_GROUP_CASE(4) KD_GROUP_CASE(8) KD_GROUP_CASE(16)
            KD_GROUP_CASE(32) KD_GROUP_CASE(64)
#undef KD_GROUP_CASE
        }
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    // Enough rows to fill the device: one workgroup per row.
    if (rows >= 2 * cus || chunk < 16384) {
        const int64_t blocks = std::min<int64_t>(rows, int64_t{cus} * 64);
        hipLaunchKernelGGL((block_kernel<C, In>), dim3(static_cast<uint32_t>(blocks)), dim3(kBlock), 0, stream(), out,
                           data, chunk, rows);
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    // Few long rows: split each row so that about 4 workgroups per CU are busy.
    int64_t segments = std::max<int64_t>(1, (int64_t{cus} * 4 + rows - 1) / rows);
    int64_t segment = (chunk + segments - 1) / segments;
    segment = std::max<int64_t>(segment, 8192);
    segment = (segment + 63) / 64 * 64;
    segments = (chunk + segment - 1) / segment;
    if (rows > 65535) return fail(KD_E_INVALID, "kd_reduce: too many rows for the split path");
    const size_t partial_bytes = static_cast<size_t>(rows * segments) * sizeof(Acc);
    Workspace ws;  // held until combine_kernel is enqueued
    Acc* partial = static_cast<Acc*>(fixed);
    if (fixed != nullptr) {
        if (partial_bytes > fixed_bytes)
            return fail(KD_E_INVALID, "kd_reduce_noalloc: the split path needs " + std::to_string(partial_bytes) +
                                          " bytes of scratch, above the " + std::to_string(fixed_bytes) +
                                          "-byte static buffer");
    } else {
        if (int rc = workspace(ws, partial_bytes)) return rc;
        partial = static_cast<Acc*>(ws.ptr);
    }
    hipLaunchKernelGGL((split_kernel<C, In>), dim3(static_cast<uint32_t>(segments), static_cast<uint32_t>(rows)),
                       dim3(kBlock), 0, stream(), partial, data, chunk, segments, segment);
    KD_LAUNCH_CHECK();
    hipLaunchKernelGGL((combine_kernel<C>), dim3(static_cast<uint32_t>(rows)), dim3(kBlock), 0, stream(), out,
                       static_cast<const Acc*>(partial), segments);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <int Op>
int reduce_dtype(int in, void* results, const void* data, int64_t chunk, int64_t rows, void* fixed = nullptr,
                 size_t fixed_bytes = 0) {
    switch (in) {
    case KD_F32: return reduce_with<Combiner<Op, float>, float>(results, data, chunk, rows, fixed, fixed_bytes);
    case KD_F64: return reduce_with<Combiner<Op, double>, double>(results, data, chunk, rows, fixed, fixed_bytes);
    case KD_I64: return reduce_with<Combiner<Op, int64_t>, int64_t>(results, data, chunk, rows, fixed, fixed_bytes);
    case KD_BOOL: return reduce_with<Combiner<Op, uint8_t>, uint8_t>(results, data, chunk, rows, fixed, fixed_bytes);
    }
    return fail(KD_E_INVALID, "kd_reduce: unknown dtype");
}

// Entry body shared by kd_reduce and kd_reduce_noalloc.
int reduce_entry(const char* name, int op, int in_dtype, void* results, const void* data, int64_t chunk_size,
                 int64_t output_count, void* fixed, size_t fixed_bytes) {
    if (chunk_size < 0 || output_count < 0) return fail(KD_E_INVALID, std::string(name) + ": negative size");
    if (dtype_size(in_dtype) == 0) return fail(KD_E_INVALID, std::string(name) + ": unknown dtype");
    if (output_count == 0) return KD_OK;
    if (chunk_size == 0 && (op == KD_REDUCE_MAX || op == KD_REDUCE_MIN))
        return fail(KD_E_INVALID, std::string(name) + ": max/min of an empty chunk");
    switch (op) {
#define KD_REDUCE_CASE(OP) \
    case OP: return reduce_dtype<OP>(in_dtype, results, data, chunk_size, output_count, fixed, fixed_bytes);
        KD_REDUCE_CASE(KD_REDUCE_SUM) KD_REDUCE_CASE(KD_REDUCE_MAX) KD_REDUCE_CASE(KD_REDUCE_MIN)
        KD_REDUCE_CASE(KD_REDUCE_PROD) KD_REDUCE_CASE(KD_REDUCE_ALL) KD_REDUCE_CASE(KD_REDUCE_ANY)
#undef KD_REDUCE_CASE
    }
    return fail(KD_E_INVALID, std::string(name) + ": unknown op");
}

template <bool Largest, typename I> int arg_typed(int in, int64_t* results, const void* data, int64_t chunk, int64_t rows) {
    switch (in) {
    case KD_F32: return reduce_with<ArgCombiner<Largest, float, I>, float>(results, data, chunk, rows);
    case KD_F64: return reduce_with<ArgCombiner<Largest, double, I>, double>(results, data, chunk, rows);
    case KD_I64: return reduce_with<ArgCombiner<Largest, int64_t, I>, int64_t>(results, data, chunk, rows);
    case KD_BOOL: return reduce_with<ArgCombiner<Largest, uint8_t, I>, uint8_t>(results, data, chunk, rows);
    }
    return fail(KD_E_INVALID, "kd_arg_reduce: unknown dtype");
}

// Positions in int32 when the chunk (plus a block of lanes past its end) fits, else int64.
template <bool Largest> int arg_dtype(int in, int64_t* results, const void* data, int64_t chunk, int64_t rows) {
    if (chunk < (int64_t{1} << 31) - 4 * kBlock) return arg_typed<Largest, int32_t>(in, results, data, chunk, rows);
    return arg_typed<Largest, int64_t>(in, results, data, chunk, rows);
}

} // namespace

} // namespace kd

// Scratch of kd_reduce_noalloc: the split path's segment partials (at most rows * segments <
// 4 * CUs + 2 * CUs values of at most 8 bytes: 12 KiB on 256 CUs). Every GPU the library runs on
// holds its own copy until the process ends. Host code never passes `scratch` itself to a kernel
// (in host code its name is only a stand-in): it uses the device address that
// hipGetSymbolAddress returns for the current device (static_scratch below).
constexpr size_t kStaticScratchBytes = size_t{64} << 10;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace kd {

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Who used a device's scratch last. A call holds its device's lock from before its split kernel
// until its combine kernel is enqueued, so calls from several host threads on one stream enqueue
// their launch pairs whole, one pair after another; when the stream differs from the previous
// call's, that stream is drained first, so calls on different streams never overlap either.
struct ScratchUse {
    std::mutex mutex;
    hipStream_t last = nullptr;
    bool used = false;
};
ScratchUse g_scratch_use[kMaxDevices];

// The device address of `scratch` on the current device, looked up once per device (with that
// device current) and kept.
int static_scratch(void** out) {
    int dev = 0;
    KD_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(KD_E_UNSUPPORTED, "kd_reduce_noalloc: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        KD_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (ptr == nullptr) return fail(KD_E_RUNTIME, "kd_reduce_noalloc: no device address for the static scratch");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

extern "C" int kd_reduce(int op, int out_dtype, int in_dtype, void* results, const void* data, int64_t chunk_size,
                         int64_t output_count) {
    (void)out_dtype;  // implied by op and input dtype, as in the reference (kernels.inl:444)
    if (output_count > 0) {
        if (int rc = ensure_device()) return rc;
    }
    return reduce_entry("kd_reduce", op, in_dtype, results, data, chunk_size, output_count, nullptr, 0);
}

extern "C" int kd_reduce_noalloc(int op, int out_dtype, int in_dtype, void* results, const void* data,
                                 int64_t chunk_size, int64_t output_count) {
    (void)out_dtype;
    // Sizes that launch nothing (no output, a negative size) return from reduce_entry before any
    // scratch is used; every other call takes the static scratch, never the workspace lease.
    void* ptr = nullptr;
    if (output_count > 0 && chunk_size >= 0) {
        if (int rc = ensure_device()) return rc;
        if (int rc = static_scratch(&ptr)) return rc;
        int dev = 0;
        KD_HIP(hipGetDevice(&dev));  // static_scratch checked the ordinal
        ScratchUse& use = g_scratch_use[dev];
        std::lock_guard<std::mutex> lock(use.mutex);
        hipStream_t current = stream();
        if (use.used && use.last != current) KD_HIP(hipStreamSynchronize(use.last));
        const int rc = reduce_entry("kd_reduce_noalloc", op, in_dtype, results, data, chunk_size, output_count, ptr,
                                    kStaticScratchBytes);
        use.last = current;
        use.used = true;
        return rc;
    }
    return reduce_entry("kd_reduce_noalloc", op, in_dtype, results, data, chunk_size, output_count, nullptr,
                        kStaticScratchBytes);
}

extern "C" int kd_arg_reduce(int largest, int in_dtype, int64_t* results, const void* data, int64_t chunk_size,
                             int64_t output_count) {
    if (chunk_size < 0 || output_count < 0) return fail(KD_E_INVALID, "kd_arg_reduce: negative size");
    if (dtype_size(in_dtype) == 0) return fail(KD_E_INVALID, "kd_arg_reduce: unknown dtype");
    if (output_count == 0) return KD_OK;
    if (chunk_size == 0) return fail(KD_E_INVALID, "kd_arg_reduce: argmax/argmin of an empty chunk");
    if (int rc = ensure_device()) return rc;
    return largest ? arg_dtype<true>(in_dtype, results, data, chunk_size, output_count)
                   : arg_dtype<false>(in_dtype, results, data, chunk_size, output_count);
}

extern "C" int kd_cumsum(int in_dtype, void* out, const void* in, int64_t size, int64_t rows) {
    if (size < 0 || rows < 0) return fail(KD_E_INVALID, "kd_cumsum: negative size");
    if (size == 0 || rows == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    switch (in_dtype) {
    case KD_F32: return cumsum_typed<float>(out, in, size, rows);
    case KD_F64: return cumsum_typed<double>(out, in, size, rows);
    case KD_I64: return cumsum_typed<int64_t>(out, in, size, rows);
    case KD_BOOL: return cumsum_typed<uint8_t>(out, in, size, rows);
    }
    return fail(KD_E_INVALID, "kd_cumsum: unknown dtype");
}

extern "C" int kd_reduce_columns(int op, int out_dtype, int in_dtype, void* results, const void* data, int64_t outer,
                                 int64_t inner) {
    (void)out_dtype;  // implied by op and input dtype, as for kd_reduce
    if (outer < 0 || inner < 0) return fail(KD_E_INVALID, "kd_reduce_columns: negative size");
    if (dtype_size(in_dtype) == 0) return fail(KD_E_INVALID, "kd_reduce_columns: unknown dtype");
    if (inner == 0) return KD_OK;
    if (outer == 0 && (op == KD_REDUCE_MAX || op == KD_REDUCE_MIN))
        return fail(KD_E_INVALID, "kd_reduce_columns: max/min of an empty chunk");
    if (int rc = ensure_device()) return rc;
    switch (op) {
#define KD_COLUMNS_CASE(OP) \
    case OP: return columns_dtype<OP>(in_dtype, results, data, outer, inner);
        KD_COLUMNS_CASE(KD_REDUCE_SUM) KD_COLUMNS_CASE(KD_REDUCE_MAX) KD_COLUMNS_CASE(KD_REDUCE_MIN)
        KD_COLUMNS_CASE(KD_REDUCE_PROD) KD_COLUMNS_CASE(KD_REDUCE_ALL) KD_COLUMNS_CASE(KD_REDUCE_ANY)
#undef KD_COLUMNS_CASE
    }
    return fail(KD_E_INVALID, "kd_reduce_columns: unknown op");
}
