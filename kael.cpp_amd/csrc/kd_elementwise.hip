// kd_elementwise.hip - strided elementwise ops, dtype conversion and fill for gfx950.
//
// Replaces the reference's one-thread-per-element `Element` task with div/mod index decode
// (src/cuda/kernels.inl:15-47, launched by backend.cu:45-53). Semantics (op functors, casts,
// operand order: operand 0 is the output) are those of kernels.inl:254-424; the layouts are
// the ones kael's TensorIterator produces (src/iterator.cpp:112-132). Three kernel families:
//
//  vec   the innermost dim is contiguous (or broadcast, stride 0) for every operand: each
//        lane moves 16-byte vectors; outer dims are decoded once per vector with a
//        multiply-high division. Covers contiguous tensors and row/column broadcasts.
//  tile  an input is contiguous along the second-innermost dim only (a transposed view):
//        64x64 tiles are staged through LDS so that both the transposed read and the
//        output write are coalesced. Covers `a.T() + b` and `contiguous()` of a transpose.
//  nd    anything else: one element per lane, all dims decoded with multiply-high division.
#include <algorithm>

#include "kd_internal.h"

namespace kd {

namespace {

constexpr int kBlock = 256;

// Functor for an ElementOp on dtype T.
template <int Op, typename T> struct OpFn {
    using In = T;
    using Out = op_out_t<Op, T>;
    static constexpr int inputs = op_inputs(Op);
    Params<T> p;
    // The result always passes through cast_value<Out>, which normalises bool outputs to 0/1
    // (reference kernels.inl:39-45 applies it to every functor result).
    __device__ __forceinline__ Out operator()(T a, T b, T c) const {
        return cast_value<Out>(apply_op<Op, T>(a, b, c, p));
    }
};

// Functor for `convert`: Identity followed by cast_value (kernels.inl:323-331).
template <typename OutT, typename InT> struct CastFn {
    using In = InT;
    using Out = OutT;
    static constexpr int inputs = 1;
    __device__ __forceinline__ Out operator()(In a, In, In) const { return cast_value<Out>(a); }
};

// Byte offsets of the operands for a decoded outer position.
struct Decode {
    int dims;                       // number of dims decoded (outer dims for vec/tile)
    FastDiv div[KD_MAX_DIMS];       // divisors, innermost decoded dim first
    int64_t stride[KD_MAX_OPERANDS][KD_MAX_DIMS];  // matching byte strides, same order
};

template <int Operands>
__device__ __forceinline__ void decode(const Decode& d, uint32_t index, int64_t (&off)[KD_MAX_OPERANDS]) {
#pragma unroll
    for (int op = 0; op < Operands; ++op) off[op] = 0;
    for (int k = 0; k < d.dims; ++k) {
        const uint32_t q = d.div[k].div(index);
        const uint32_t pos = index - q * d.div[k].divisor;
        index = q;
#pragma unroll
        for (int op = 0; op < Operands; ++op) off[op] += static_cast<int64_t>(pos) * d.stride[op][k];
    }
}

struct Bases {
    char* p[KD_MAX_OPERANDS];
};

// ---- vec family ----------------------------------------------------------------------------

template <typename T, int N> struct alignas(sizeof(T) * N) Vec {
    T v[N];
};

// Loads and stores of 1..32-byte aggregates, optionally with the nontemporal hint (streaming
// data that is touched once: measured ~6.4 TB/s versus ~5.5 TB/s with default caching).
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT, typename T> __device__ __forceinline__ T ld(const T* p) {
    if constexpr (!NT) {
        return *p;
    } else {
        T out;
        if constexpr (sizeof(T) == 16) {
            const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
            __builtin_memcpy(&out, &r, 16);
        } else if constexpr (sizeof(T) == 32) {
            const u32x4 r0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
            const u32x4 r1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + 1);
            __builtin_memcpy(&out, &r0, 16);
            __builtin_memcpy(reinterpret_cast<char*>(&out) + 16, &r1, 16);
        } else if constexpr (sizeof(T) == 8) {
            const u32x2 r = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
            __builtin_memcpy(&out, &r, 8);
        } else if constexpr (sizeof(T) == 4) {
            const unsigned r = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(p));
            __builtin_memcpy(&out, &r, 4);
        } else {
            out = *p;
        }
        return out;
    }
}

template <bool NT, typename T> __device__ __forceinline__ void st(T* p, const T& v) {
    if constexpr (!NT) {
        *p = v;
    } else if constexpr (sizeof(T) == 16) {
        u32x4 r;
        __builtin_memcpy(&r, &v, 16);
        __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
    } else if constexpr (sizeof(T) == 32) {
        u32x4 r0, r1;
        __builtin_memcpy(&r0, &v, 16);
        __builtin_memcpy(&r1, reinterpret_cast<const char*>(&v) + 16, 16);
        __builtin_nontemporal_store(r0, reinterpret_cast<u32x4*>(p));
        __builtin_nontemporal_store(r1, reinterpret_cast<u32x4*>(p) + 1);
    } else if constexpr (sizeof(T) == 8) {
        u32x2 r;
        __builtin_memcpy(&r, &v, 8);
        __builtin_nontemporal_store(r, reinterpret_cast<u32x2*>(p));
    } else if constexpr (sizeof(T) == 4) {
        unsigned r;
        __builtin_memcpy(&r, &v, 4);
        __builtin_nontemporal_store(r, reinterpret_cast<unsigned*>(p));
    } else {
        *p = v;
    }
}

// Outer1: at most one outer dim (contiguous tensors, row and column broadcasts): the outer
// strides are loop invariants held in scalar registers, instead of a per-vector decode loop
// whose dynamically indexed kernel arguments cost a scalar-load round trip per vector.
// Mask >= 0 fixes the broadcast mask at compile time (no per-vector branch on it); -1 reads it
// from `broadcast_mask`.
template <typename F, int VEC, bool NT, bool Outer1, int Mask>
__device__ __forceinline__ void vec_loop(F f, const Bases& bases, const Decode& outer, uint32_t inner_vectors,
                                         FastDiv inner_div, uint32_t total_vectors, uint32_t broadcast_mask) {
    using In = typename F::In;
    using Out = typename F::Out;
    constexpr int N = F::inputs;
    if constexpr (Mask >= 0) broadcast_mask = static_cast<uint32_t>(Mask);
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < total_vectors; v += stride) {
        const uint32_t row = inner_div.div(v);
        const uint32_t col = v - row * inner_vectors;
        int64_t off[KD_MAX_OPERANDS];
        if constexpr (Outer1) {
#pragma unroll
            for (int op = 0; op <= N; ++op) off[op] = static_cast<int64_t>(row) * outer.stride[op][0];
        } else {
            decode<N + 1>(outer, row, off);
        }
        Vec<In, VEC> in[3];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const char* base = bases.p[i + 1] + off[i + 1];
            if (broadcast_mask & (1u << (i + 1))) {
                const In s = *reinterpret_cast<const In*>(base);
#pragma unroll
                for (int e = 0; e < VEC; ++e) in[i].v[e] = s;
            } else {
                in[i] = ld<NT>(reinterpret_cast<const Vec<In, VEC>*>(base) + col);
            }
        }
        Vec<Out, VEC> out;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            out.v[e] = f(in[0].v[e], N > 1 ? in[1].v[e] : In{}, N > 2 ? in[2].v[e] : In{});
        }
        st<NT>(reinterpret_cast<Vec<Out, VEC>*>(bases.p[0] + off[0]) + col, out);
    }
}

// The contiguous path's common broadcast patterns (none, or one input broadcast along the last
// dim, e.g. a[4096,4096] + b[4096,1]) get loops with the mask fixed at compile time: the
// runtime test on it inside the loop cost ~5 % of HBM bandwidth on that shape.
template <typename F, int VEC, bool NT, bool Outer1>
__global__ __launch_bounds__(kBlock) void vec_kernel(F f, Bases bases, Decode outer,
                                                     uint32_t inner_vectors, FastDiv inner_div,
                                                     uint32_t total_vectors, uint32_t broadcast_mask) {
    constexpr int N = F::inputs;
    if constexpr (Outer1 && N <= 2) {
        if (broadcast_mask == 0)
            return vec_loop<F, VEC, NT, Outer1, 0>(f, bases, outer, inner_vectors, inner_div, total_vectors, 0);
        if (broadcast_mask == 2u)
            return vec_loop<F, VEC, NT, Outer1, 2>(f, bases, outer, inner_vectors, inner_div, total_vectors, 2u);
        if constexpr (N == 2) {
            if (broadcast_mask == 4u)
                return vec_loop<F, VEC, NT, Outer1, 4>(f, bases, outer, inner_vectors, inner_div, total_vectors, 4u);
        }
    }
    vec_loop<F, VEC, NT, Outer1, -1>(f, bases, outer, inner_vectors, inner_div, total_vectors, broadcast_mask);
}

// ---- tile family ------------------------------------------------------------------------------

constexpr int kTile = 64;

// Tile (tr, tc) visited by workgroup `id` of a 1-D grid over `tiles` tiles, `tiles_c` per tile
// row. Workgroups are dispatched round-robin over the 8 XCDs, so id % 8 names the XCD; each XCD
// walks its own contiguous run of tiles, columns fastest, so that the tiles in flight on one XCD
// write neighbouring segments of the same output rows. On a[4096,4096].T() + b this order moves
// 80 % of HBM peak against 71 % for the plain row-major tile order.
__device__ __forceinline__ void tile_of(uint32_t id, uint32_t tiles_c, uint32_t tiles, uint32_t& tr, uint32_t& tc) {
    const uint32_t full = tiles - tiles % 8;
    const uint32_t lin = id < full ? (id % 8) * (full / 8) + id / 8 : id;
    tr = lin / tiles_c;
    tc = lin - tr * tiles_c;
}

// Tile of rows (dim d-2) x cols (dim d-1). `transposed_mask` marks the inputs read through LDS
// (contiguous along rows); other inputs and the output are read/written along cols.
template <typename F>
__global__ __launch_bounds__(kBlock) void tile_kernel(F f, Bases bases, Decode outer, int64_t rows,
                                                      int64_t cols, int64_t rs0, int64_t rs1, int64_t rs2,
                                                      int64_t rs3, int64_t cs0, int64_t cs1, int64_t cs2,
                                                      int64_t cs3, uint32_t transposed_mask, uint32_t tiles_c,
                                                      uint32_t tiles) {
    using In = typename F::In;
    using Out = typename F::Out;
    constexpr int N = F::inputs;
    __shared__ In stage[N][kTile][kTile + 1];
    const int64_t rstride[4] = {rs0, rs1, rs2, rs3};
    const int64_t cstride[4] = {cs0, cs1, cs2, cs3};

    int64_t off[KD_MAX_OPERANDS];
    decode<N + 1>(outer, blockIdx.z, off);
    uint32_t tr, tc;
    tile_of(blockIdx.x, tiles_c, tiles, tr, tc);
    const int64_t r0 = static_cast<int64_t>(tr) * kTile;
    const int64_t c0 = static_cast<int64_t>(tc) * kTile;
    const int tx = threadIdx.x % kTile;
    const int ty = threadIdx.x / kTile;  // 0..3

    // Load the transposed inputs: consecutive lanes walk rows (their contiguous dim).
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (!(transposed_mask & (1u << (i + 1)))) continue;
        const char* base = bases.p[i + 1] + off[i + 1];
        const int64_t r = r0 + tx;
        for (int j = ty; j < kTile; j += kBlock / kTile) {
            const int64_t c = c0 + j;
            if (r < rows && c < cols) {
                stage[i][j][tx] = *reinterpret_cast<const In*>(base + r * rstride[i + 1] + c * cstride[i + 1]);
            }
        }
    }
    __syncthreads();

    const int64_t c = c0 + tx;
    if (c >= cols) return;
    for (int j = ty; j < kTile; j += kBlock / kTile) {
        const int64_t r = r0 + j;
        if (r >= rows) break;
        In in[3] = {};
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (transposed_mask & (1u << (i + 1))) {
                in[i] = stage[i][tx][j];
            } else {
                in[i] = *reinterpret_cast<const In*>(bases.p[i + 1] + off[i + 1] + r * rstride[i + 1] +
                                                      c * cstride[i + 1]);
            }
        }
        *reinterpret_cast<Out*>(bases.p[0] + off[0] + r * rstride[0] + c * cstride[0]) =
            f(in[0], in[1], in[2]);
    }
}

// Vectorized tile family: 64x64 tiles of (rows = dim d-2, cols = dim d-1). Transposed inputs
// (contiguous along rows) are loaded with VEC-wide vectors along their contiguous dim and
// staged in LDS; the output and inner-contiguous inputs move VEC-wide vectors along cols;
// broadcast inputs (stride 0 along cols) are read once per row. Needs rows % VEC == 0,
// cols % VEC == 0 and VEC-aligned bases and strides for every vector access (checked on the
// host). Inputs are read with ordinary loads: a tile reads 256-byte row segments, for which the
// nontemporal hint cost 15 % of bandwidth; the output takes the hint (NT) when streaming.
template <typename F, int VEC, bool NT>
__global__ __launch_bounds__(kBlock) void tile_vec_kernel(F f, Bases bases, Decode outer, int64_t rows, int64_t cols,
                                                          int64_t rs0, int64_t rs1, int64_t rs2, int64_t rs3, int64_t cs1,
                                                          int64_t cs2, int64_t cs3, uint32_t transposed_mask,
                                                          uint32_t broadcast_mask, uint32_t tiles_c, uint32_t tiles) {
    using In = typename F::In;
    using Out = typename F::Out;
    constexpr int N = F::inputs;
    // stage[slot][c][r] for the transposed inputs only (slot order = input order)
    extern __shared__ __align__(16) unsigned char tile_lds[];
    auto stage = reinterpret_cast<In(*)[kTile][kTile + VEC]>(tile_lds);
    int slot_of[3] = {0, 0, 0};
    {
        int next = 0;
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (transposed_mask & (1u << (i + 1))) slot_of[i] = next++;
    }
    const int64_t rstride[4] = {rs0, rs1, rs2, rs3};
    const int64_t cstride[4] = {static_cast<int64_t>(sizeof(Out)), cs1, cs2, cs3};
    int64_t off[KD_MAX_OPERANDS];
    decode<N + 1>(outer, blockIdx.z, off);
    uint32_t tr, tc;
    tile_of(blockIdx.x, tiles_c, tiles, tr, tc);
    const int64_t r0 = static_cast<int64_t>(tr) * kTile;
    const int64_t c0 = static_cast<int64_t>(tc) * kTile;
    const char* tile_base[3];
#pragma unroll
    for (int i = 0; i < N; ++i) tile_base[i] = bases.p[i + 1] + off[i + 1] + r0 * rstride[i + 1] + c0 * cstride[i + 1];
    char* out_base = bases.p[0] + off[0] + r0 * rstride[0] + c0 * static_cast<int64_t>(sizeof(Out));
    constexpr int per_line = kTile / VEC;  // vectors along one tile edge

#pragma unroll
    for (int i = 0; i < N; ++i) {
        if (!(transposed_mask & (1u << (i + 1)))) continue;
        for (int idx = threadIdx.x; idx < kTile * per_line; idx += kBlock) {
            const int c = idx / per_line, rv = idx % per_line;
            if (c0 + c < cols && r0 + VEC * rv < rows) {
                const Vec<In, VEC> v = ld<false>(reinterpret_cast<const Vec<In, VEC>*>(
                    tile_base[i] + c * cstride[i + 1] + static_cast<int64_t>(VEC * rv) * sizeof(In)));
#pragma unroll
                for (int e = 0; e < VEC; ++e) stage[slot_of[i]][c][VEC * rv + e] = v.v[e];
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < kTile * per_line; idx += kBlock) {
        const int r = idx / per_line, cv = idx % per_line;
        if (r0 + r >= rows || c0 + VEC * cv >= cols) continue;
        Vec<In, VEC> in[3];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            if (transposed_mask & (1u << (i + 1))) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) in[i].v[e] = stage[slot_of[i]][VEC * cv + e][r];
            } else if (broadcast_mask & (1u << (i + 1))) {
                const In s = *reinterpret_cast<const In*>(tile_base[i] + r * rstride[i + 1]);
#pragma unroll
                for (int e = 0; e < VEC; ++e) in[i].v[e] = s;
            } else {
                in[i] = ld<false>(reinterpret_cast<const Vec<In, VEC>*>(tile_base[i] + r * rstride[i + 1]) + cv);
            }
        }
        Vec<Out, VEC> o;
#pragma unroll
        for (int e = 0; e < VEC; ++e) o.v[e] = f(in[0].v[e], N > 1 ? in[1].v[e] : In{}, N > 2 ? in[2].v[e] : In{});
        st<NT>(reinterpret_cast<Vec<Out, VEC>*>(out_base + r * rstride[0]) + cv, o);
    }
}

// ---- nd family ---------------------------------------------------------------------------------

template <typename F>
__global__ __launch_bounds__(kBlock) void nd_kernel(F f, Bases bases, Decode all, uint32_t count) {
    using In = typename F::In;
    using Out = typename F::Out;
    constexpr int N = F::inputs;
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t e = blockIdx.x * kBlock + threadIdx.x; e < count; e += stride) {
        int64_t off[KD_MAX_OPERANDS];
        decode<N + 1>(all, e, off);
        In in[3] = {};
#pragma unroll
        for (int i = 0; i < N; ++i) in[i] = *reinterpret_cast<const In*>(bases.p[i + 1] + off[i + 1]);
        *reinterpret_cast<Out*>(bases.p[0] + off[0]) = f(in[0], in[1], in[2]);
    }
}

// 64-bit fallback for more than 2^31 - 1 elements (same decode as kernels.inl:15-28).
template <typename F>
__global__ __launch_bounds__(kBlock) void nd64_kernel(F f, kd_element_layout layout) {
    using In = typename F::In;
    using Out = typename F::Out;
    constexpr int N = F::inputs;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; e < layout.count; e += stride) {
        int64_t off[KD_MAX_OPERANDS] = {0, 0, 0, 0};
        int64_t rem = e;
        for (int d = layout.dims - 1; d >= 0; --d) {
            const int64_t pos = rem % layout.shape[d];
            rem /= layout.shape[d];
#pragma unroll
            for (int op = 0; op <= N; ++op) off[op] += pos * layout.strides[op][d];
        }
        In in[3] = {};
#pragma unroll
        for (int i = 0; i < N; ++i) in[i] = *reinterpret_cast<const In*>(static_cast<char*>(layout.base[i + 1]) + off[i + 1]);
        *reinterpret_cast<Out*>(static_cast<char*>(layout.base[0]) + off[0]) = f(in[0], in[1], in[2]);
    }
}

// ---- host-side planning ------------------------------------------------------------------------

int grid_for(int64_t work) {
    const int64_t blocks = (work + kBlock - 1) / kBlock;
    const int64_t cap = int64_t{1} << 20;
    return static_cast<int>(std::max<int64_t>(1, std::min(blocks, cap)));
}

// Fills `d` with dims [first, last) of the layout, innermost first.
void make_decode(const kd_element_layout& l, int operands, int first, int last, Decode& d) {
    d.dims = 0;
    for (int dim = last - 1; dim >= first; --dim) {
        d.div[d.dims] = FastDiv(static_cast<uint32_t>(l.shape[dim]));
        for (int op = 0; op < operands; ++op) d.stride[op][d.dims] = l.strides[op][dim];
        ++d.dims;
    }
}

// Streaming hint for operands too large to stay in cache between kernels (>= 32 MiB moved).
bool streaming(const kd_element_layout& l, int64_t out_size, int64_t in_size, int operands) {
    return l.count * (out_size + in_size * (operands - 1)) >= (int64_t{32} << 20);
}

template <typename F> int launch(const F& f, const kd_element_layout& l) {
    using In = typename F::In;
    using Out = typename F::Out;
    constexpr int N = F::inputs;
    constexpr int operands = N + 1;
    const int64_t in_size = sizeof(In);
    const int64_t out_size = sizeof(Out);
    if (l.operands != operands) return fail(KD_E_INVALID, "layout operand count does not match the op");
    if (l.dims < 1 || l.dims > KD_MAX_DIMS) return fail(KD_E_INVALID, "layout dims out of range");
    if (l.count == 0) return KD_OK;
    int64_t product = 1;
    for (int d = 0; d < l.dims; ++d) {
        if (l.shape[d] <= 0) return fail(KD_E_INVALID, "layout has a non-positive dim with count > 0");
        product *= l.shape[d];
    }
    if (product != l.count) return fail(KD_E_INVALID, "layout count does not match its shape");

    Bases bases;
    for (int op = 0; op < KD_MAX_OPERANDS; ++op) bases.p[op] = op < operands ? static_cast<char*>(l.base[op]) : nullptr;

    const bool small = l.count < (int64_t{1} << 31);
    const int last = l.dims - 1;

    if (small) {
        // vec family
        constexpr int VEC = sizeof(In) >= 8 ? 2 : (sizeof(In) == 4 ? 4 : 16);
        bool vec_ok = l.shape[last] % VEC == 0 && l.strides[0][last] == out_size;
        uint32_t broadcast_mask = 0;
        const auto aligned = [&](int op, int64_t esize) {
            const int64_t bytes = esize * VEC;
            if (reinterpret_cast<uintptr_t>(l.base[op]) % bytes != 0) return false;
            for (int d = 0; d < last; ++d)
                if (l.strides[op][d] % bytes != 0) return false;
            return true;
        };
        if (vec_ok) vec_ok = aligned(0, out_size);
        for (int i = 1; i <= N && vec_ok; ++i) {
            if (l.strides[i][last] == 0) {
                broadcast_mask |= 1u << i;
            } else if (l.strides[i][last] != in_size || !aligned(i, in_size)) {
                vec_ok = false;
            }
        }
        if (vec_ok) {
            Decode outer{};
            make_decode(l, operands, 0, last, outer);
            const uint32_t inner_vectors = static_cast<uint32_t>(l.shape[last] / VEC);
            const uint32_t total = static_cast<uint32_t>(l.count / VEC);
            const bool nt = streaming(l, out_size, in_size, operands);
            const dim3 grid(grid_for(total));
            const FastDiv inner_div(inner_vectors);
            // With no outer dim the row is always 0; the zeroed strides make every offset 0.
            if (outer.dims <= 1) {
                if (nt)
                    hipLaunchKernelGGL((vec_kernel<F, VEC, true, true>), grid, dim3(kBlock), 0, stream(), f, bases,
                                       outer, inner_vectors, inner_div, total, broadcast_mask);
                else
                    hipLaunchKernelGGL((vec_kernel<F, VEC, false, true>), grid, dim3(kBlock), 0, stream(), f, bases,
                                       outer, inner_vectors, inner_div, total, broadcast_mask);
            } else {
                if (nt)
                    hipLaunchKernelGGL((vec_kernel<F, VEC, true, false>), grid, dim3(kBlock), 0, stream(), f, bases,
                                       outer, inner_vectors, inner_div, total, broadcast_mask);
                else
                    hipLaunchKernelGGL((vec_kernel<F, VEC, false, false>), grid, dim3(kBlock), 0, stream(), f, bases,
                                       outer, inner_vectors, inner_div, total, broadcast_mask);
            }
            KD_LAUNCH_CHECK();
            return KD_OK;
        }

        // tile family: some input contiguous along dim d-2 but strided along d-1
        if (l.dims >= 2) {
            const int r = l.dims - 2;
            uint32_t tmask = 0;
            bool tile_ok = l.strides[0][last] == out_size;
            for (int i = 1; i <= N; ++i) {
                const int64_t cs = l.strides[i][last];
                if (cs == in_size || cs == 0) continue;
                if (l.strides[i][r] == in_size) tmask |= 1u << i;
            }
            const int64_t outer_count = l.count / (l.shape[r] * l.shape[last]);
            const int64_t tile_count = ((l.shape[last] + kTile - 1) / kTile) * ((l.shape[r] + kTile - 1) / kTile);
            if (tile_ok && tmask != 0 && outer_count < 65536 && tile_count * kBlock < (int64_t{1} << 32)) {
                Decode outer;
                make_decode(l, operands, 0, r, outer);
                int64_t rs[4] = {0, 0, 0, 0}, cs[4] = {0, 0, 0, 0};
                for (int op = 0; op < operands; ++op) {
                    rs[op] = l.strides[op][r];
                    cs[op] = l.strides[op][last];
                }
                const uint32_t tiles_c = static_cast<uint32_t>((l.shape[last] + kTile - 1) / kTile);
                const uint32_t tiles = static_cast<uint32_t>(tile_count);
                const dim3 grid(tiles, 1, static_cast<uint32_t>(outer_count));
                // Vectorized tile when every vector access is aligned and whole.
                constexpr int TV = sizeof(In) >= 8 ? 2 : (sizeof(In) == 4 ? 4 : 16);
                bool tv_ok = l.shape[r] % TV == 0 && l.shape[last] % TV == 0 && sizeof(Out) * TV <= 32;
                uint32_t bmask = 0;
                const auto vec_aligned = [&](int op, int64_t esize, bool along_rows) {
                    const int64_t bytes = esize * TV;
                    if (reinterpret_cast<uintptr_t>(l.base[op]) % bytes != 0) return false;
                    for (int dd = 0; dd < l.dims; ++dd) {
                        if ((along_rows ? dd == r : dd == last)) continue;
                        if (l.strides[op][dd] % bytes != 0) return false;
                    }
                    return true;
                };
                if (tv_ok) tv_ok = vec_aligned(0, out_size, false);
                for (int i = 1; i <= N && tv_ok; ++i) {
                    if (tmask & (1u << i)) {
                        tv_ok = vec_aligned(i, in_size, true);
                    } else if (l.strides[i][last] == 0) {
                        bmask |= 1u << i;
                    } else if (l.strides[i][last] == in_size) {
                        tv_ok = vec_aligned(i, in_size, false);
                    } else {
                        tv_ok = false;
                    }
                }
                if (tv_ok) {
                    const size_t lds = static_cast<size_t>(__builtin_popcount(tmask)) * kTile * (kTile + TV) * sizeof(In);
                    if (streaming(l, out_size, in_size, operands))
                        hipLaunchKernelGGL((tile_vec_kernel<F, TV, true>), grid, dim3(kBlock), lds, stream(), f, bases, outer,
                                           l.shape[r], l.shape[last], rs[0], rs[1], rs[2], rs[3], cs[1], cs[2], cs[3], tmask,
                                           bmask, tiles_c, tiles);
                    else
                        hipLaunchKernelGGL((tile_vec_kernel<F, TV, false>), grid, dim3(kBlock), lds, stream(), f, bases, outer,
                                           l.shape[r], l.shape[last], rs[0], rs[1], rs[2], rs[3], cs[1], cs[2], cs[3], tmask,
                                           bmask, tiles_c, tiles);
                    KD_LAUNCH_CHECK();
                    return KD_OK;
                }
                hipLaunchKernelGGL((tile_kernel<F>), grid, dim3(kBlock), 0, stream(), f, bases, outer,
                                   l.shape[r], l.shape[last], rs[0], rs[1], rs[2], rs[3], cs[0], cs[1],
                                   cs[2], cs[3], tmask, tiles_c, tiles);
                KD_LAUNCH_CHECK();
                return KD_OK;
            }
        }

        Decode all;
        make_decode(l, operands, 0, l.dims, all);
        hipLaunchKernelGGL((nd_kernel<F>), dim3(grid_for(l.count)), dim3(kBlock), 0, stream(), f, bases, all,
                           static_cast<uint32_t>(l.count));
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    hipLaunchKernelGGL((nd64_kernel<F>), dim3(grid_for(l.count)), dim3(kBlock), 0, stream(), f, l);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <int Op, typename T> int run_op(const kd_element_layout& l, const kd_element_parameters& p) {
    OpFn<Op, T> f;
    f.p = Params<T>::make(p);
    return launch(f, l);
}

template <int Op> int run_typed(int dtype, const kd_element_layout& l, const kd_element_parameters& p) {
    if constexpr (is_floating_op(Op)) {
        if (dtype == KD_F32) return run_op<Op, float>(l, p);
        if (dtype == KD_F64) return run_op<Op, double>(l, p);
        return fail(KD_E_INVALID, "floating-point element op on a non-floating dtype");
    } else {
        switch (dtype) {
        case KD_F32: return run_op<Op, float>(l, p);
        case KD_F64: return run_op<Op, double>(l, p);
        case KD_I64: return run_op<Op, int64_t>(l, p);
        case KD_BOOL:
            if constexpr (Op == KD_OP_POWER) return KD_OK;  // nothing is launched: kernels.inl:345-351
            else return run_op<Op, uint8_t>(l, p);
        }
        return fail(KD_E_INVALID, "unknown dtype");
    }
}

template <typename Out> int run_convert_from(int in, const kd_element_layout& l) {
    switch (in) {
    case KD_F32: return launch(CastFn<Out, float>{}, l);
    case KD_F64: return launch(CastFn<Out, double>{}, l);
    case KD_I64: return launch(CastFn<Out, int64_t>{}, l);
    case KD_BOOL: return launch(CastFn<Out, uint8_t>{}, l);
    }
    return fail(KD_E_INVALID, "convert: unknown input dtype");
}

template <typename T>
__global__ __launch_bounds__(kBlock) void fill_kernel(T* target, T value, int64_t count) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) target[i] = value;
}

// 16-byte stores for an aligned body; `pattern` holds 16 bytes of repeated value.
__global__ __launch_bounds__(kBlock) void fill16_kernel(uint4* target, uint4 pattern, int64_t vectors) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < vectors; i += stride) target[i] = pattern;
}

template <typename T> int fill_typed(void* target, int64_t count, const void* value) {
    T v;
    std::memcpy(&v, value, sizeof(T));
    char* p = static_cast<char*>(target);
    // Head up to 16-byte alignment, body with 16-byte stores, tail.
    int64_t head = 0;
    while (head < count && reinterpret_cast<uintptr_t>(p + head * sizeof(T)) % 16 != 0) ++head;
    if (head > 0) {
        hipLaunchKernelGGL((fill_kernel<T>), dim3(1), dim3(kBlock), 0, stream(), reinterpret_cast<T*>(p), v, head);
        KD_LAUNCH_CHECK();
    }
    const int64_t per = 16 / sizeof(T);
    const int64_t vectors = (count - head) / per;
    if (vectors > 0) {
        uint4 pattern;
        T lanes[16 / sizeof(T)];
        for (int64_t i = 0; i < per; ++i) lanes[i] = v;
        std::memcpy(&pattern, lanes, 16);
        hipLaunchKernelGGL(fill16_kernel, dim3(grid_for(vectors)), dim3(kBlock), 0, stream(),
                           reinterpret_cast<uint4*>(p + head * sizeof(T)), pattern, vectors);
        KD_LAUNCH_CHECK();
    }
    const int64_t done = head + vectors * per;
    if (done < count) {
        hipLaunchKernelGGL((fill_kernel<T>), dim3(1), dim3(kBlock), 0, stream(),
                           reinterpret_cast<T*>(p + done * sizeof(T)), v, count - done);
        KD_LAUNCH_CHECK();
    }
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

#define KD_OP_CASE(op) \
    case op: return run_typed<op>(in_dtype, *layout, parameters);

extern "C" int kd_elementwise(int op, int out_dtype, int in_dtype, const kd_element_layout* layout,
                              kd_element_parameters parameters) {
    if (layout == nullptr) return fail(KD_E_INVALID, "kd_elementwise: null layout");
    if (dtype_size(in_dtype) == 0) return fail(KD_E_INVALID, "kd_elementwise: unknown dtype");
    (void)out_dtype;  // implied by the op, as in the reference (kernels.inl:335)
    if (layout->count == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    switch (op) {
        KD_OP_CASE(KD_OP_PLUS)
        KD_OP_CASE(KD_OP_MINUS)
        KD_OP_CASE(KD_OP_TIMES)
        KD_OP_CASE(KD_OP_DIVIDES)
        KD_OP_CASE(KD_OP_POWER)
        KD_OP_CASE(KD_OP_MAXIMUM)
        KD_OP_CASE(KD_OP_MINIMUM)
        KD_OP_CASE(KD_OP_EQUAL)
        KD_OP_CASE(KD_OP_NOT_EQUAL)
        KD_OP_CASE(KD_OP_LESS)
        KD_OP_CASE(KD_OP_LESS_EQUAL)
        KD_OP_CASE(KD_OP_GREATER)
        KD_OP_CASE(KD_OP_GREATER_EQUAL)
        KD_OP_CASE(KD_OP_LOGICAL_AND)
        KD_OP_CASE(KD_OP_LOGICAL_OR)
        KD_OP_CASE(KD_OP_LOGICAL_XOR)
        KD_OP_CASE(KD_OP_IS_ZERO)
        KD_OP_CASE(KD_OP_NEGATE)
        KD_OP_CASE(KD_OP_ABSOLUTE)
        KD_OP_CASE(KD_OP_SIGN)
        KD_OP_CASE(KD_OP_EXP)
        KD_OP_CASE(KD_OP_LOG)
        KD_OP_CASE(KD_OP_LOG1P)
        KD_OP_CASE(KD_OP_EXPM1)
        KD_OP_CASE(KD_OP_SQRT)
        KD_OP_CASE(KD_OP_RSQRT)
        KD_OP_CASE(KD_OP_SIN)
        KD_OP_CASE(KD_OP_COS)
        KD_OP_CASE(KD_OP_TANH)
        KD_OP_CASE(KD_OP_SIGMOID)
        KD_OP_CASE(KD_OP_RELU)
        KD_OP_CASE(KD_OP_GELU_EXACT)
        KD_OP_CASE(KD_OP_GELU_TANH)
        KD_OP_CASE(KD_OP_CLAMP)
        KD_OP_CASE(KD_OP_WHERE)
        KD_OP_CASE(KD_OP_MASKED_FILL)
        KD_OP_CASE(KD_OP_GELU_EXACT_BACKWARD)
        KD_OP_CASE(KD_OP_GELU_TANH_BACKWARD)
    }
    return fail(KD_E_INVALID, "kd_elementwise: unknown op " + std::to_string(op));
}

extern "C" int kd_convert(int out_dtype, int in_dtype, const kd_element_layout* layout) {
    if (layout == nullptr) return fail(KD_E_INVALID, "kd_convert: null layout");
    if (layout->count == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    switch (out_dtype) {
    case KD_F32: return run_convert_from<float>(in_dtype, *layout);
    case KD_F64: return run_convert_from<double>(in_dtype, *layout);
    case KD_I64: return run_convert_from<int64_t>(in_dtype, *layout);
    case KD_BOOL: return run_convert_from<uint8_t>(in_dtype, *layout);
    }
    return fail(KD_E_INVALID, "kd_convert: unknown output dtype");
}

extern "C" int kd_fill(int dtype, void* target, int64_t count, const void* value) {
    if (count < 0) return fail(KD_E_INVALID, "kd_fill: negative count");
    if (count == 0) return KD_OK;
    if (target == nullptr || value == nullptr) return fail(KD_E_INVALID, "kd_fill: null pointer");
    if (int rc = ensure_device()) return rc;
    switch (dtype) {
    case KD_F32: return fill_typed<float>(target, count, value);
    case KD_F64: return fill_typed<double>(target, count, value);
    case KD_I64: return fill_typed<int64_t>(target, count, value);
    case KD_BOOL: return fill_typed<uint8_t>(target, count, value);
    }
    return fail(KD_E_INVALID, "kd_fill: unknown dtype");
}
