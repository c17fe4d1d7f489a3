// kd_matmul.hip - batched matrix products for gfx950.
//
// Contract of reference include/kael/device_kernels.h:111-112 / src/cuda/backend.cu:142-171:
// out[b] = a[b] . b[b] for `batches` row-major matrices, `out` overwritten (never accumulated).
// f32 and f64 are floating point, i64 wraps (kernels.inl:160-169), bool is rejected
// (src/ops/linalg.cpp:72). The reference computes a 4x4 register tile per thread straight from
// global memory (kernels.inl:136-177). Here, per shape:
//
//   mfma   f32, M and N large: 128x128 workgroup tiles, four waves of 64x64, each a 2x2 grid of
//          v_mfma_f32_32x32x2f32 accumulators. K advances 16 at a time through double-buffered
//          LDS; global loads for step k+1 are in flight while step k multiplies.
//   small  f32, few 128x128 tiles and K <= 2048 (C1's 512^3, small MLP layers): 32x32 tiles,
//          one workgroup of 16 waves each, the waves splitting K and reading their operands
//          straight from global memory, their partial tiles added in LDS in wave order.
//   skinny f32, M <= 16 (decode-shaped): lanes own 4 columns each, K is split across the
//          workgroup's waves and, when N alone cannot fill the device, across workgroups whose
//          partial sums land in a workspace and are added in a fixed order by a second launch.
//   rowdot f32, N <= 4 (e.g. the GPT head computing W . x^T): one wave per output row, a
//          coalesced dot product along K.
//   tiled  f64 and i64: 64x64 LDS tiles, 4x4 outputs per lane (exact wrapping for i64).
//
// Every kernel takes per-operand element strides (batch, row, column), which is how
// kd_matmul_strided reads transposed or batch-broadcast operands in place.
#include <algorithm>
#include <type_traits>

#include "kd_internal.h"

namespace kd {

namespace {

struct Strides3 {
    int64_t b, r, c;
};

// Batches address the operands on one level (batch b at b * sa.b) or, with heads > 1, on two:
// b = o * heads + h at o * sa.b + h * ha (attention's [batch, head] views of a [batch, token,
// head, dim] tensor, which no single batch stride describes).
struct MatmulArgs {
    int64_t batches, M, K, N;
    Strides3 sa, sb, so;
    int64_t heads = 1;
    int64_t ha = 0, hb = 0, ho = 0;
    const void* bias = nullptr;  // element n added to column n of every output row (element type)
};

// out = v, or v + bias[col] rounded once (wrapping for i64): the bias add of kael's Linear
// (product + bias) as the epilogue of the product that precedes it.
template <typename T> __device__ __forceinline__ T plus_bias(T v, const void* bias, int64_t col) {
    if (bias == nullptr) return v;
    const T b = static_cast<const T*>(bias)[col];
    if constexpr (std::is_same_v<T, int64_t>) return wrap_add(v, b);
    else return add_sep(v, b);
}

// Element offset of batch `batch` in an operand with outer / head strides `outer` / `inner`.
__host__ __device__ __forceinline__ int64_t batch_offset(const MatmulArgs& p, int64_t batch, int64_t outer,
                                                         int64_t inner) {
    if (p.heads == 1) return batch * outer;
    const int64_t o = static_cast<uint32_t>(batch) / static_cast<uint32_t>(p.heads);
    return o * outer + (batch - o * p.heads) * inner;
}

// Batch addressing of the kernels with 32-bit tile offsets: blockIdx.y = o * heads + h starts
// o * a + h * ha elements into A (likewise B and the output). heads = 1 is a plain batch stride,
// also how split K passes each split's offsets.
struct BatchStrides {
    int64_t a, b, o;
    int64_t ha, hb, ho;
    uint32_t heads;
    const float* bias;  // the epilogue's bias (null: none; split-K partials never take it)
};

BatchStrides batch_strides(int64_t a, int64_t b, int64_t o) { return {a, b, o, 0, 0, 0, 1u, nullptr}; }
BatchStrides batch_strides(const MatmulArgs& p) {
    return {p.sa.b, p.sb.b, p.so.b, p.ha, p.hb, p.ho, static_cast<uint32_t>(p.heads), static_cast<const float*>(p.bias)};
}

// Offsets of this workgroup's batch (blockIdx.y) in A, B and the output.
__device__ __forceinline__ void batch_offsets(const BatchStrides& s, int64_t& oa, int64_t& ob, int64_t& oo) {
    const uint32_t y = blockIdx.y;
    if (s.heads == 1) {
        oa = y * s.a;
        ob = y * s.b;
        oo = y * s.o;
        return;
    }
    const uint32_t o = y / s.heads;
    const uint32_t h = y - o * s.heads;
    oa = o * s.a + h * s.ha;
    ob = o * s.b + h * s.hb;
    oo = o * s.o + h * s.ho;
}

constexpr int kThreads = 256;

// ---- mfma family (f32) ---------------------------------------------------------------------

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 16;
constexpr int kAld = kBK + 4;   // A tile [m][k]: row stride 20 floats, conflict-free 16-byte reads
constexpr int kBld = kBN + 4;   // B tile [k][n]
constexpr int kAsize = kBM * kAld;
constexpr int kBsize = kBK * kBld;

typedef float v16f __attribute__((ext_vector_type(16)));

// Operand access modes, chosen on the host.
//   A: kRowVec = K contiguous (row-major), kColVec = M contiguous (a transposed view)
//   B: kRowVec = N contiguous (row-major), kColVec = K contiguous (a transposed view)
enum { kRowVec = 0, kColVec = 1, kGeneric = 2 };

template <int AMode>
__device__ __forceinline__ void load_a(float (&reg)[8], const float* a, const MatmulArgs& p, int64_t m0, int64_t k0) {
    const int t = threadIdx.x;
    if constexpr (AMode == kRowVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t m = m0 + t / 4 + 64 * i;
            const int64_t k = k0 + 4 * (t % 4);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < p.M && k < p.K) v = *reinterpret_cast<const float4*>(a + m * p.sa.r + k);
            reg[4 * i + 0] = v.x;
            reg[4 * i + 1] = v.y;
            reg[4 * i + 2] = v.z;
            reg[4 * i + 3] = v.w;
        }
    } else if constexpr (AMode == kColVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t m = m0 + 4 * (t % 32);
            const int64_t k = k0 + t / 32 + 8 * i;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < p.M && k < p.K) v = *reinterpret_cast<const float4*>(a + k * p.sa.c + m);
            reg[4 * i + 0] = v.x;
            reg[4 * i + 1] = v.y;
            reg[4 * i + 2] = v.z;
            reg[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = t + kThreads * i;
            const int64_t m = m0 + idx / kBK;
            const int64_t k = k0 + idx % kBK;
            reg[i] = (m < p.M && k < p.K) ? a[m * p.sa.r + k * p.sa.c] : 0.f;
        }
    }
}

template <int AMode> __device__ __forceinline__ void store_a(float* As, const float (&reg)[8]) {
    const int t = threadIdx.x;
    if constexpr (AMode == kRowVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = t / 4 + 64 * i;
            const int k = 4 * (t % 4);
            *reinterpret_cast<float4*>(As + row * kAld + k) =
                make_float4(reg[4 * i], reg[4 * i + 1], reg[4 * i + 2], reg[4 * i + 3]);
        }
    } else if constexpr (AMode == kColVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = 4 * (t % 32);
            const int k = t / 32 + 8 * i;
#pragma unroll
            for (int e = 0; e < 4; ++e) As[(m + e) * kAld + k] = reg[4 * i + e];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = t + kThreads * i;
            As[(idx / kBK) * kAld + idx % kBK] = reg[i];
        }
    }
}

template <int BMode>
__device__ __forceinline__ void load_b(float (&reg)[8], const float* b, const MatmulArgs& p, int64_t k0, int64_t n0) {
    const int t = threadIdx.x;
    if constexpr (BMode == kRowVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t k = k0 + t / 32 + 8 * i;
            const int64_t n = n0 + 4 * (t % 32);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < p.K && n < p.N) v = *reinterpret_cast<const float4*>(b + k * p.sb.r + n);
            reg[4 * i + 0] = v.x;
            reg[4 * i + 1] = v.y;
            reg[4 * i + 2] = v.z;
            reg[4 * i + 3] = v.w;
        }
    } else if constexpr (BMode == kColVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t n = n0 + t / 4 + 64 * i;
            const int64_t k = k0 + 4 * (t % 4);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < p.K && n < p.N) v = *reinterpret_cast<const float4*>(b + n * p.sb.c + k);
            reg[4 * i + 0] = v.x;
            reg[4 * i + 1] = v.y;
            reg[4 * i + 2] = v.z;
            reg[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = t + kThreads * i;
            const int64_t k = k0 + idx / kBN;
            const int64_t n = n0 + idx % kBN;
            reg[i] = (k < p.K && n < p.N) ? b[k * p.sb.r + n * p.sb.c] : 0.f;
        }
    }
}

template <int BMode> __device__ __forceinline__ void store_b(float* Bs, const float (&reg)[8]) {
    const int t = threadIdx.x;
    if constexpr (BMode == kRowVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int k = t / 32 + 8 * i;
            const int n = 4 * (t % 32);
            *reinterpret_cast<float4*>(Bs + k * kBld + n) =
                make_float4(reg[4 * i], reg[4 * i + 1], reg[4 * i + 2], reg[4 * i + 3]);
        }
    } else if constexpr (BMode == kColVec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int n = t / 4 + 64 * i;
            const int k = 4 * (t % 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) Bs[(k + e) * kBld + n] = reg[4 * i + e];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = t + kThreads * i;
            Bs[(idx / kBN) * kBld + idx % kBN] = reg[i];
        }
    }
}

// Full tiles (M % 128 == 0, N % 128 == 0, K % 16 == 0, vector modes): each thread's two 16-byte
// sources per operand stay fixed for the whole K loop and only a uniform offset advances, so a
// K step issues its loads without bounds checks or 64-bit index products (the bounds-checked
// loaders above cost ~8 % of the 4096^3 rate). Register order matches load_a / load_b.
template <int AMode>
__device__ __forceinline__ void a_origin(const float* a, const MatmulArgs& p, int64_t m0, const float* (&src)[2],
                                         int64_t& step) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (AMode == kRowVec) src[i] = a + (m0 + t / 4 + 64 * i) * p.sa.r + 4 * (t % 4);
        else src[i] = a + (t / 32 + 8 * i) * p.sa.c + m0 + 4 * (t % 32);
    }
    step = AMode == kRowVec ? kBK : kBK * p.sa.c;
}

template <int BMode>
__device__ __forceinline__ void b_origin(const float* b, const MatmulArgs& p, int64_t n0, const float* (&src)[2],
                                         int64_t& step) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if constexpr (BMode == kRowVec) src[i] = b + (t / 32 + 8 * i) * p.sb.r + n0 + 4 * (t % 32);
        else src[i] = b + (n0 + t / 4 + 64 * i) * p.sb.c + 4 * (t % 4);
    }
    step = BMode == kRowVec ? kBK * p.sb.r : kBK;
}

__device__ __forceinline__ void load_full(float (&reg)[8], const float* const (&src)[2], int64_t offset) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(src[i] + offset);
        reg[4 * i + 0] = v.x;
        reg[4 * i + 1] = v.y;
        reg[4 * i + 2] = v.z;
        reg[4 * i + 3] = v.w;
    }
}

// Maps the linear workgroup id to a (tile_m, tile_n) pair so that the workgroups that one XCD
// runs (ids congruent mod 8 are dispatched to the same XCD) cover a compact block of tiles,
// sharing A rows and B columns in that XCD's L2.
__device__ __forceinline__ void tile_of(int64_t id, int64_t tiles_m, int64_t tiles_n, int64_t& tm, int64_t& tn) {
    const int64_t total = tiles_m * tiles_n;
    int64_t local = id;
    if (total % 8 == 0) local = (id % 8) * (total / 8) + id / 8;
    // Grouped order: columns of 8 tile-rows walked along N.
    constexpr int64_t kGroup = 8;
    const int64_t group_size = kGroup * tiles_n;
    const int64_t group = local / group_size;
    const int64_t first_m = group * kGroup;
    const int64_t rows_in_group = std::min<int64_t>(kGroup, tiles_m - first_m);
    const int64_t in_group = local % group_size;
    tm = first_m + in_group % rows_in_group;
    tn = in_group / rows_in_group;
}

template <int AMode, int BMode, bool Full, bool Bias = false>
__global__ __launch_bounds__(kThreads) void mfma_f32_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                            float* __restrict__ out, MatmulArgs p) {
    __shared__ float As[2][kAsize];
    __shared__ float Bs[2][kBsize];

    const int64_t tiles_m = (p.M + kBM - 1) / kBM;
    const int64_t tiles_n = (p.N + kBN - 1) / kBN;
    int64_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t batch = blockIdx.y;
    const int64_t m0 = tm * kBM;
    const int64_t n0 = tn * kBN;
    a += batch_offset(p, batch, p.sa.b, p.ha);
    b += batch_offset(p, batch, p.sb.b, p.hb);
    out += batch_offset(p, batch, p.so.b, p.ho);

    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    const int wm = wave / 2;  // wave tile row (0..1), 64 rows each
    const int wn = wave % 2;  // wave tile col (0..1), 64 cols each
    const int li = lane % 32;
    const int lh = lane / 32;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    float ra[8], rb[8];
    const int64_t ksteps = (p.K + kBK - 1) / kBK;
    const float* a_src[2] = {nullptr, nullptr};
    const float* b_src[2] = {nullptr, nullptr};
    int64_t a_step = 0, b_step = 0;
    if constexpr (Full) {
        a_origin<AMode>(a, p, m0, a_src, a_step);
        b_origin<BMode>(b, p, n0, b_src, b_step);
        load_full(ra, a_src, 0);
        load_full(rb, b_src, 0);
    } else {
        load_a<AMode>(ra, a, p, m0, 0);
        load_b<BMode>(rb, b, p, 0, n0);
    }
    store_a<AMode>(As[0], ra);
    store_b<BMode>(Bs[0], rb);
    __syncthreads();

    for (int64_t ks = 0; ks < ksteps; ++ks) {
        const int cur = ks & 1;
        const bool more = ks + 1 < ksteps;
        if (more) {
            if constexpr (Full) {
                load_full(ra, a_src, (ks + 1) * a_step);
                load_full(rb, b_src, (ks + 1) * b_step);
            } else {
                load_a<AMode>(ra, a, p, m0, (ks + 1) * kBK);
                load_b<BMode>(rb, b, p, (ks + 1) * kBK, n0);
            }
        }
        const float* as = As[cur];
        const float* bs = Bs[cur];
        // Raised wave priority while this wave issues its MFMAs: the SIMD's arbiter then
        // prefers waves with matrix work ready over waves issuing loads, which keeps the matrix
        // pipe fed (measured +5 % at 4096^3).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kg = 0; kg < kBK; kg += 8) {
            // Lane (li, lh) feeds k = kg + 4*lh + s to MFMA step s (s = 0..3): the same k for
            // its A element and its B element, so the 2-deep MFMA sums cover k = kg..kg+7.
            float4 af[2];
            float bf[2][4];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const float4*>(as + (wm * 64 + i * 32 + li) * kAld + kg + 4 * lh);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int s = 0; s < 4; ++s) bf[j][s] = bs[(kg + 4 * lh + s) * kBld + wn * 64 + j * 32 + li];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float av = s == 0 ? af[i].x : s == 1 ? af[i].y : s == 2 ? af[i].z : af[i].w;
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bf[j][s], acc[i][j], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
        if (more) {
            store_a<AMode>(As[cur ^ 1], ra);
            store_b<BMode>(Bs[cur ^ 1], rb);
        }
        __syncthreads();
    }

    // Accumulator element r of lane (li, lh) is row 8*(r/4) + 4*lh + r%4, column li of its
    // 32x32 block.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t col = n0 + wn * 64 + j * 32 + li;
            if (!Full && col >= p.N) continue;
            if constexpr (Bias) {
                const float bv = static_cast<const float*>(p.bias)[col];
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = add_sep(acc[i][j][r], bv);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * lh + (r % 4);
                if (Full || row < p.M) out[row * p.so.r + col * p.so.c] = acc[i][j][r];
            }
        }
}

// Row-major A and B whose tiles are all full (M % 128 == 0, N % 128 == 0, K % 16 == 0) with
// every per-batch extent below 2^31 elements: the headline and forward-pass shape. The same
// tiles, LDS layout, MFMA order and wave priority as mfma_f32_kernel, but with 32-bit per-thread
// offsets and leading dimensions, and the loop bound in a scalar register: on 4096^3 this runs
// ~5 % faster than the general kernel's Full path, whose 64-bit index math and argument block
// cost issue slots around the MFMAs. Results are bitwise those of mfma_f32_kernel.
//
// Split K (blockIdx.z = split): workgroup (tile, batch, split) multiplies the K slice that
// starts split_a columns into A and split_b elements into B (K is the slice length) and writes
// its partial product split_o floats further into the output, a workspace that
// split_sum_kernel adds up in split order.
__global__ __launch_bounds__(kThreads) void mfma_f32_rowmajor_kernel(const float* __restrict__ a,
                                                                     const float* __restrict__ b,
                                                                     float* __restrict__ out, int M, int N, int K,
                                                                     int lda, int ldb, int ldo, int64_t batch_a,
                                                                     int64_t batch_b, int64_t batch_o, int64_t split_a,
                                                                     int64_t split_b, int64_t split_o) {
    __shared__ float As[2][kAsize];
    __shared__ float Bs[2][kBsize];
    const int tiles_m = M / kBM;
    const int tiles_n = N / kBN;
    int64_t tm64, tn64;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm64, tn64);
    const int m0 = static_cast<int>(tm64) * kBM;
    const int n0 = static_cast<int>(tn64) * kBN;
    a += blockIdx.y * batch_a + blockIdx.z * split_a;
    b += blockIdx.y * batch_b + blockIdx.z * split_b;
    out += blockIdx.y * batch_o + blockIdx.z * split_o;

    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2;
    const int wn = wave % 2;
    const int li = lane % 32;
    const int lh = lane / 32;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Thread t moves A rows m0 + t/4 + 64i (4 floats at k = 4*(t%4)) and B rows t/32 + 8i (4
    // floats at n = n0 + 4*(t%32)), as load_a / load_b do for the vector modes.
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int a_off[2] = {(m0 + t / 4) * lda + 4 * (t % 4), (m0 + t / 4 + 64) * lda + 4 * (t % 4)};
    const int b_off[2] = {(t / 32) * ldb + n0 + 4 * (t % 32), (t / 32 + 8) * ldb + n0 + 4 * (t % 32)};
    const int as_off[2] = {(t / 4) * kAld + 4 * (t % 4), (t / 4 + 64) * kAld + 4 * (t % 4)};
    const int bs_off[2] = {(t / 32) * kBld + 4 * (t % 32), (t / 32 + 8) * kBld + 4 * (t % 32)};
    f4 ra[2], rb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ra[i] = *reinterpret_cast<const f4*>(a + a_off[i]);
        rb[i] = *reinterpret_cast<const f4*>(b + b_off[i]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        *reinterpret_cast<f4*>(&As[0][as_off[i]]) = ra[i];
        *reinterpret_cast<f4*>(&Bs[0][bs_off[i]]) = rb[i];
    }
    __syncthreads();

    const int ksteps = K / kBK;
    for (int ks = 0; ks < ksteps; ++ks) {
        const int cur = ks & 1;
        const bool more = ks + 1 < ksteps;
        if (more) {
            const int ka = (ks + 1) * kBK;
            const int kb = ka * ldb;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                ra[i] = *reinterpret_cast<const f4*>(a + a_off[i] + ka);
                rb[i] = *reinterpret_cast<const f4*>(b + b_off[i] + kb);
            }
        }
        const float* as = As[cur];
        const float* bs = Bs[cur];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kg = 0; kg < kBK; kg += 8) {
            f4 af[2];
            float bf[2][4];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const f4*>(as + (wm * 64 + i * 32 + li) * kAld + kg + 4 * lh);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4) bf[j][s4] = bs[(kg + 4 * lh + s4) * kBld + wn * 64 + j * 32 + li];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s4], bf[j][s4], acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        if (more) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                *reinterpret_cast<f4*>(&As[cur ^ 1][as_off[i]]) = ra[i];
                *reinterpret_cast<f4*>(&Bs[cur ^ 1][bs_off[i]]) = rb[i];
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + li;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * lh + (r % 4);
                out[row * ldo + col] = acc[i][j][r];
            }
        }
}

// Whole-tile products with A and/or B read through a transposed view, 32-bit offsets: A
// M-contiguous (AT: the weight gradient X^T . g of a Linear layer, reference
// src/autograd/functions_linalg.cpp:44) and/or B K-contiguous (BT: the forward x . W^T,
// src/nn/layers.cpp:43). The general kernel's transposed loaders store each 16-byte load as four
// scalars down an LDS column (8-way bank conflicts for A). Here waves 0-1 load the A tile and
// waves 2-3 the B tile, four 16-byte loads per thread: a transposed operand as a 4 x 4 block
// (four consecutive rows of its contiguous dim, coalesced across lanes) that the thread writes
// transposed as four 16-byte rows of the [m][k] / [k][n] LDS tile; a row-major operand as four
// 16-byte rows. With AT the A tile's 16-byte column groups are XOR-swizzled by (row / 16) % 4,
// which makes those transposed writes conflict-free; the MFMA reads apply the same swizzle. MFMA
// order and results are those of mfma_f32_rowmajor_kernel (bit for bit). `lda` / `ldb` / `ldo`
// are the strides between consecutive rows of the stored operands: of A's k (AT) or m rows, of
// B's n (BT) or k rows, of the output's m rows.
template <bool AT, bool BT, bool Bias = false, bool Deep = false>
__global__ __launch_bounds__(kThreads) void mfma_f32_trans_kernel(const float* __restrict__ a,
                                                                  const float* __restrict__ b,
                                                                  float* __restrict__ out, int M, int N, int K,
                                                                  int lda, int ldb, int ldo, BatchStrides bs) {
    __shared__ float As[2][kAsize];
    __shared__ float Bs[2][kBsize];
    const int tiles_m = M / kBM;
    const int tiles_n = N / kBN;
    int64_t tm64, tn64;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm64, tn64);
    const int m0 = static_cast<int>(tm64) * kBM;
    const int n0 = static_cast<int>(tn64) * kBN;
    {
        int64_t oa, ob, oo;
        batch_offsets(bs, oa, ob, oo);
        a += oa;
        b += ob;
        out += oo;
    }

    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2;
    const int wn = wave % 2;
    const int li = lane % 32;
    const int lh = lane / 32;

    v16f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    typedef float f4 __attribute__((ext_vector_type(4)));
    // Column (in floats) of 16-byte group `c4` of A tile row `row` after the swizzle.
    const auto aswz = [](int row, int c4) { return AT ? c4 ^ (4 * ((row / 16) % 4)) : c4; };
    const bool loads_a = t < kThreads / 2;
    const int u = loads_a ? t : t - kThreads / 2;
    // Per-thread source offset (element) of load j = 0..3 at K step 0, and the step per load j.
    int g_off, g_row;
    if (loads_a) {
        if (AT) {  // A^T rows k = 4*(u/32) + j, columns m0 + 4*(u%32) .. +3
            g_off = 4 * (u / 32) * lda + m0 + 4 * (u % 32);
            g_row = lda;
        } else {   // A rows m0 + u/4 + 32*j, columns k = 4*(u%4) .. +3
            g_off = (m0 + u / 4) * lda + 4 * (u % 4);
            g_row = 32 * lda;
        }
    } else {
        if (BT) {  // B^T rows n0 + 4*(u/4) + j, columns k = 4*(u%4) .. +3
            g_off = (n0 + 4 * (u / 4)) * ldb + 4 * (u % 4);
            g_row = ldb;
        } else {   // B rows k = 4*(u/32) + j, columns n0 + 4*(u%32) .. +3
            g_off = 4 * (u / 32) * ldb + n0 + 4 * (u % 32);
            g_row = ldb;
        }
    }
    const int g_step = loads_a ? (AT ? kBK * lda : kBK) : (BT ? kBK : kBK * ldb);
    const float* src = loads_a ? a : b;
    const auto fetch = [&](f4 (&r)[4], int ks) {
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = *reinterpret_cast<const f4*>(src + g_off + ks * g_step + j * g_row);
    };
    const auto stash = [&](const f4 (&r)[4], int buf) {
        if (loads_a) {
            if (AT) {
                // r[j][e] = A[m0 + 4*(u%32) + e][4*(u/32) + j]
                const int c4 = 4 * (u / 32);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = 4 * (u % 32) + e;
                    *reinterpret_cast<f4*>(&As[buf][row * kAld + aswz(row, c4)]) = f4{r[0][e], r[1][e], r[2][e], r[3][e]};
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<f4*>(&As[buf][(u / 4 + 32 * j) * kAld + 4 * (u % 4)]) = r[j];
            }
        } else {
            if (BT) {
                // r[j][e] = B[4*(u%4) + e][n0 + 4*(u/4) + j]
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    *reinterpret_cast<f4*>(&Bs[buf][(4 * (u % 4) + e) * kBld + 4 * (u / 4)]) = f4{r[0][e], r[1][e], r[2][e], r[3][e]};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<f4*>(&Bs[buf][(4 * (u / 32) + j) * kBld + 4 * (u % 32)]) = r[j];
            }
        }
    };
    // This lane's A tile reads (rows wm*64 + i*32 + li, 16-byte groups kg + 4*lh) as LDS offsets.
    int a_rd[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = wm * 64 + i * 32 + li;
            a_rd[i][h] = row * kAld + aswz(row, 8 * h + 4 * lh);
        }
    const auto step = [&](int cur) {
        const float* as = As[cur];
        const float* bs = Bs[cur];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kg = 0; kg < kBK; kg += 8) {
            f4 af[2];
            float bf[2][4];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const f4*>(as + a_rd[i][kg / 8]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4) bf[j][s4] = bs[(kg + 4 * lh + s4) * kBld + wn * 64 + j * 32 + li];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s4], bf[j][s4], acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    };
    const int ksteps = K / kBK;
    if constexpr (Deep) {
        // Grids of at most one workgroup per CU: a wave per SIMD cannot hide one step's load
        // latency behind other waves, so the global loads run two K steps ahead (step s fetched
        // into register set s % 2 at the start of step s - 2, written to LDS buffer s % 2 at the
        // end of step s - 1). Same MFMA order, same results.
        f4 r0[4], r1[4];
        fetch(r0, 0);
        if (ksteps > 1) fetch(r1, 1);
        stash(r0, 0);
        __syncthreads();
        int ks = 0;
        for (; ks + 1 < ksteps; ks += 2) {
            if (ks + 2 < ksteps) fetch(r0, ks + 2);
            step(0);
            stash(r1, 1);
            __syncthreads();
            if (ks + 3 < ksteps) fetch(r1, ks + 3);
            step(1);
            if (ks + 2 < ksteps) stash(r0, 0);
            __syncthreads();
        }
        if (ks < ksteps) step(0);  // an odd step count's last step
    } else {
        f4 r[4];
        fetch(r, 0);
        stash(r, 0);
        __syncthreads();
        for (int ks = 0; ks < ksteps; ++ks) {
            const int cur = ks & 1;
            const bool more = ks + 1 < ksteps;
            if (more) fetch(r, ks + 1);
            step(cur);
            if (more) stash(r, cur ^ 1);
            __syncthreads();
        }
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + wn * 64 + j * 32 + li;
            // the bias variant is its own instantiation: a runtime test here costs the
            // headline kernel registers (116 -> 164 VGPRs, one wave per SIMD less)
            const float bv = Bias ? bs.bias[col] : 0.f;
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (rr / 4) + 4 * lh + (rr % 4);
                if constexpr (Bias) out[row * ldo + col] = add_sep(acc[i][j][rr], bv);
                else out[row * ldo + col] = acc[i][j][rr];
            }
        }
}

// ---- 64x64 tiles (f32, grids too small for 128x128 tiles) ---------------------------------------

constexpr int kT64 = 64;
constexpr int kT64K = 32;           // K per LDS stage
constexpr int kT64Ald = kT64K + 4;  // A tile [m][k], row stride 36 floats
constexpr int kT64Bld = kT64 + 4;   // B tile [k][n], row stride 68 floats

// Whole 64x64 output tiles for products whose 128x128 grid would not give every CU a workgroup:
// attention-sized batched products (128 x 128 x 64 per head), x . W^T with N = 256 over a folded
// batch, split-K weight gradients. Four waves, each one 32x32 v_mfma_f32_32x32x2f32 accumulator of
// the 2x2 wave grid; K advances 32 at a time through double-buffered LDS. Waves 0-1 load the A
// tile and waves 2-3 the B tile, four 16-byte loads per thread, coalesced along each operand's
// contiguous dim; a transposed operand (A^T: M contiguous, B^T: K contiguous) is written
// transposed into the [m][k] / [k][n] LDS tile, A^T's 16-byte column groups XOR-swizzled by
// (row / 4) % 8 so that those writes do not collide. Each output element accumulates K in the same
// (k, k + 4) MFMA pairs and order as the 128x128 kernels, so without split K the results are
// theirs bit for bit. Batches (or K splits: their offsets as batch strides) take blockIdx.y.
// Ragged: M a multiple of 4 but not of 64 (the tied LM head's 96-row weight gradient): the last
// tile row loads zeros past M and stores only rows below it.
template <bool AT, bool BT, bool Ragged = false>
__global__ __launch_bounds__(kThreads) void mfma_f32_t64_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                                float* __restrict__ out, int M, int N, int K, int lda,
                                                                int ldb, int ldo, BatchStrides bs) {
    __shared__ float As[2][kT64 * kT64Ald];
    __shared__ float Bs[2][kT64K * kT64Bld];
    const int tiles_m = (M + kT64 - 1) / kT64;
    const int tiles_n = N / kT64;
    int64_t tm64, tn64;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm64, tn64);
    const int m0 = static_cast<int>(tm64) * kT64;
    const int n0 = static_cast<int>(tn64) * kT64;
    {
        int64_t oa, ob, oo;
        batch_offsets(bs, oa, ob, oo);
        a += oa;
        b += ob;
        out += oo;
    }

    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2;
    const int wn = wave % 2;
    const int li = lane % 32;
    const int lh = lane / 32;

    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;

    typedef float f4 __attribute__((ext_vector_type(4)));
    // Column (in floats) of 16-byte group `c4` of A tile row `row` after the swizzle.
    const auto aswz = [](int row, int c4) { return AT ? c4 ^ (4 * ((row / 4) % 8)) : c4; };
    const bool loads_a = t < kThreads / 2;
    const int u = loads_a ? t : t - kThreads / 2;
    // Per-thread source offset (element) of load j = 0..3 at K step 0, and the step per load j.
    int g_off, g_row;
    if (loads_a) {
        if (AT) {  // A^T rows k = 4*(u/16) + j, columns m0 + 4*(u%16) .. +3
            g_off = 4 * (u / 16) * lda + m0 + 4 * (u % 16);
            g_row = lda;
        } else {   // A rows m0 + u/8 + 16*j, columns k = 4*(u%8) .. +3
            g_off = (m0 + u / 8) * lda + 4 * (u % 8);
            g_row = 16 * lda;
        }
    } else {
        if (BT) {  // B^T rows n0 + 4*(u/8) + j, columns k = 4*(u%8) .. +3
            g_off = (n0 + 4 * (u / 8)) * ldb + 4 * (u % 8);
            g_row = ldb;
        } else {   // B rows k = 4*(u/16) + j, columns n0 + 4*(u%16) .. +3
            g_off = 4 * (u / 16) * ldb + n0 + 4 * (u % 16);
            g_row = ldb;
        }
    }
    const int g_step = loads_a ? (AT ? kT64K * lda : kT64K) : (BT ? kT64K : kT64K * ldb);
    const float* src = loads_a ? a : b;
    // Ragged: whether load j of this thread stays inside A's M rows (A^T: its four columns, all in or
    // all out as M is a multiple of 4; A: its row)
    const auto inside = [&](int j) {
        if constexpr (!Ragged) return true;
        else if (!loads_a) return true;
        else if (AT) return m0 + 4 * (u % 16) < M;
        else return m0 + u / 8 + 16 * j < M;
    };
    const auto fetch = [&](f4 (&r)[4], int ks) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            r[j] = inside(j) ? *reinterpret_cast<const f4*>(src + g_off + ks * g_step + j * g_row) : f4{0.f, 0.f, 0.f, 0.f};
    };
    const auto stash = [&](const f4 (&r)[4], int buf) {
        if (loads_a) {
            if (AT) {
                // r[j][e] = A[m0 + 4*(u%16) + e][4*(u/16) + j]
                const int c4 = 4 * (u / 16);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = 4 * (u % 16) + e;
                    *reinterpret_cast<f4*>(&As[buf][row * kT64Ald + aswz(row, c4)]) = f4{r[0][e], r[1][e], r[2][e], r[3][e]};
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<f4*>(&As[buf][(u / 8 + 16 * j) * kT64Ald + 4 * (u % 8)]) = r[j];
            }
        } else {
            if (BT) {
                // r[j][e] = B[4*(u%8) + e][n0 + 4*(u/8) + j]
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    *reinterpret_cast<f4*>(&Bs[buf][(4 * (u % 8) + e) * kT64Bld + 4 * (u / 8)]) = f4{r[0][e], r[1][e], r[2][e], r[3][e]};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) *reinterpret_cast<f4*>(&Bs[buf][(4 * (u / 16) + j) * kT64Bld + 4 * (u % 16)]) = r[j];
            }
        }
    };
    // This lane's A tile reads (row wm*32 + li, 16-byte groups kg + 4*lh) as LDS offsets.
    const int arow = wm * 32 + li;
    int a_rd[kT64K / 8];
#pragma unroll
    for (int h = 0; h < kT64K / 8; ++h) a_rd[h] = arow * kT64Ald + aswz(arow, 8 * h + 4 * lh);
    const auto step = [&](int cur) {
        const float* as = As[cur];
        const float* bs = Bs[cur];
#pragma unroll
        for (int kg = 0; kg < kT64K; kg += 8) {
            const f4 af = *reinterpret_cast<const f4*>(as + a_rd[kg / 8]);
            float bf[4];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) bf[s4] = bs[(kg + 4 * lh + s4) * kT64Bld + wn * 32 + li];
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[s4], bf[s4], acc, 0, 0, 0);
        }
    };
    // Global loads run two K steps ahead of the MFMAs: a grid of at most a few workgroups per CU
    // has too few waves to cover one step's load latency with the others' work. Step s is
    // fetched into register set s % 2 at the start of step s - 2 and written to LDS buffer s % 2
    // at the end of step s - 1.
    const int ksteps = K / kT64K;
    f4 r0[4], r1[4];
    fetch(r0, 0);
    if (ksteps > 1) fetch(r1, 1);
    stash(r0, 0);
    __syncthreads();
    int ks = 0;
    for (; ks + 1 < ksteps; ks += 2) {
        if (ks + 2 < ksteps) fetch(r0, ks + 2);
        step(0);
        stash(r1, 1);
        __syncthreads();
        if (ks + 3 < ksteps) fetch(r1, ks + 3);
        step(1);
        if (ks + 2 < ksteps) stash(r0, 0);
        __syncthreads();
    }
    if (ks < ksteps) step(0);  // an odd step count's last step

    const int col = n0 + wn * 32 + li;
    if (bs.bias == nullptr) {
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const int row = m0 + wm * 32 + 8 * (rr / 4) + 4 * lh + (rr % 4);
            if (!Ragged || row < M) out[row * ldo + col] = acc[rr];
        }
    } else {
        const float bv = bs.bias[col];
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const int row = m0 + wm * 32 + 8 * (rr / 4) + 4 * lh + (rr % 4);
            if (!Ragged || row < M) out[row * ldo + col] = add_sep(acc[rr], bv);
        }
    }
}

// ---- small family (f32, few output tiles) -----------------------------------------------------

constexpr int kSmallTile = 32;
constexpr int kSmallWaves = 16;

// Products whose 128x128 tiles would leave most CUs idle (C1's 512^3 has 16 of them) and whose K
// is moderate: one workgroup of 16 waves per 32x32 output tile. Wave w multiplies the 8-deep K
// groups g = w, w + 16, ... straight from global memory - lane (li, lh) reads row li of A and
// column li of B at k = 8g + 4lh .. 8g + 4lh + 3, the operands of four v_mfma_f32_32x32x2f32
// steps - with the next group's loads in flight during the current group's MFMAs. The 16
// partial tiles are then added through LDS in wave order, so the result does not depend on
// timing. One launch and no workspace, where the split-K path needs a second launch to add its
// partial products. AVec: A is K-contiguous with 16-byte aligned rows (one 16-byte load per
// lane and group).
template <bool AVec>
__global__ __launch_bounds__(kSmallWaves * 64) void small_kernel(const float* __restrict__ a,
                                                                 const float* __restrict__ b,
                                                                 float* __restrict__ out, MatmulArgs p) {
    __shared__ float red[kSmallWaves][16 * 64];
    typedef float f4 __attribute__((ext_vector_type(4)));
    const int64_t batch = blockIdx.z;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kSmallTile;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kSmallTile;
    const int lane = threadIdx.x % 64;
    const int w = threadIdx.x / 64;
    const int li = lane % 32;
    const int lh = lane / 32;
    // K steps in 32-bit element offsets (the host checks that K times the K strides fits).
    const int K = static_cast<int>(p.K);
    const int a_k = static_cast<int>(p.sa.c);
    const int b_k = static_cast<int>(p.sb.r);
    const int groups = (K + 7) / 8;
    const int64_t m = m0 + li;
    const int64_t n = n0 + li;
    const bool mok = m < p.M;
    const bool nok = n < p.N;
    const float* arow = a + batch_offset(p, batch, p.sa.b, p.ha) + (mok ? m : 0) * p.sa.r;
    const float* bcol = b + batch_offset(p, batch, p.sb.b, p.hb) + (nok ? n : 0) * p.sb.c;
    // Group g's operands, zero past the edges of A, B and K.
    const auto load = [&](int g, f4& av, f4& bv) {
        av = f4{0.f, 0.f, 0.f, 0.f};
        bv = f4{0.f, 0.f, 0.f, 0.f};
        if (g >= groups) return;
        const int k = g * 8 + 4 * lh;
        if (AVec && k + 3 < K) {
            if (mok) av = *reinterpret_cast<const f4*>(arow + k);
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                if (mok && k + s < K) av[s] = arow[(k + s) * a_k];
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
            if (nok && k + s < K) bv[s] = bcol[(k + s) * b_k];
    };
    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    f4 ca, cb, na, nb;
    load(w, ca, cb);
    for (int g = w; g < groups; g += kSmallWaves) {
        load(g + kSmallWaves, na, nb);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[s], cb[s], acc, 0, 0, 0);
        ca = na;
        cb = nb;
    }
    // Accumulator element r of lane (li, lh) is row 8*(r/4) + 4*lh + r%4, column li of the tile.
#pragma unroll
    for (int r = 0; r < 16; ++r) red[w][r * 64 + lane] = acc[r];
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * 64; e += kSmallWaves * 64) {
        float v = red[0][e];
#pragma unroll
        for (int q = 1; q < kSmallWaves; ++q) v += red[q][e];
        const int r = e / 64;
        const int l = e % 64;
        const int64_t row = m0 + 8 * (r / 4) + 4 * (l / 32) + (r % 4);
        const int64_t col = n0 + l % 32;
        if (row < p.M && col < p.N)
            out[batch_offset(p, batch, p.so.b, p.ho) + row * p.so.r + col * p.so.c] = plus_bias(v, p.bias, col);
    }
}

// ---- skinny family (f32, small M) ------------------------------------------------------------

constexpr int kSkinnyMaxM = 16;
constexpr int kSkinnyCols = 256;  // 64 lanes x 4 columns

// Partial sums of rows [0, M) x columns [n0, n0+256) over k in [k_begin, k_end): the four waves
// take interleaved k, then combine in LDS in wave order. `partial` (if non-null) receives the
// workgroup's sum for split index blockIdx.y; otherwise the result goes to `out` directly.
template <int MT, bool BVec>
__global__ __launch_bounds__(kThreads) void skinny_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ out, float* __restrict__ partial,
                                                          MatmulArgs p, int64_t k_chunk) {
    __shared__ float red[4][MT][kSkinnyCols];
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    const int64_t batch = blockIdx.z;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kSkinnyCols + lane * 4;
    const int64_t k_begin = static_cast<int64_t>(blockIdx.y) * k_chunk;
    const int64_t k_end = std::min<int64_t>(p.K, k_begin + k_chunk);
    a += batch_offset(p, batch, p.sa.b, p.ha);
    b += batch_offset(p, batch, p.sb.b, p.hb);

    float acc[MT][4];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[m][c] = 0.f;

    for (int64_t k = k_begin + wave; k < k_end; k += 4) {
        float bv[4];
        if (BVec && n0 + 3 < p.N) {
            const float4 v = *reinterpret_cast<const float4*>(b + k * p.sb.r + n0);
            bv[0] = v.x;
            bv[1] = v.y;
            bv[2] = v.z;
            bv[3] = v.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) bv[c] = n0 + c < p.N ? b[k * p.sb.r + (n0 + c) * p.sb.c] : 0.f;
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < p.M) {
                const float av = a[m * p.sa.r + k * p.sa.c];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[m][c] += av * bv[c];
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) red[wave][m][lane * 4 + c] = acc[m][c];
    __syncthreads();
    for (int idx = threadIdx.x; idx < MT * kSkinnyCols; idx += kThreads) {
        const int m = idx / kSkinnyCols;
        const int col = idx % kSkinnyCols;
        const int64_t n = static_cast<int64_t>(blockIdx.x) * kSkinnyCols + col;
        if (m >= p.M || n >= p.N) continue;
        const float v = ((red[0][m][col] + red[1][m][col]) + red[2][m][col]) + red[3][m][col];
        if (partial != nullptr) {
            partial[((batch * gridDim.y + blockIdx.y) * p.M + m) * p.N + n] = v;
        } else {
            out[batch_offset(p, batch, p.so.b, p.ho) + m * p.so.r + n * p.so.c] = plus_bias(v, p.bias, n);
        }
    }
}

// Adds the split partials in split order and writes the output.
__global__ __launch_bounds__(kThreads) void split_sum_kernel(const float* __restrict__ partial, float* __restrict__ out,
                                                             MatmulArgs p, int64_t splits) {
    const int64_t per_batch = p.M * p.N;
    const int64_t total = p.batches * per_batch;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t batch = idx / per_batch;
        const int64_t mn = idx % per_batch;
        // The partials come from memory (written by other XCDs): a batch of them is loaded before
        // the first add, one round trip per batch (C4's products split K at most 16 ways); they
        // are added in split order.
        constexpr int kBatch = 16;
        float v = 0.f;
        for (int64_t s0 = 0; s0 < splits; s0 += kBatch) {
            float x[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (s0 + u < splits) x[u] = partial[(batch * splits + s0 + u) * per_batch + mn];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (s0 + u < splits) v += x[u];
        }
        const int64_t m = mn / p.N;
        const int64_t n = mn % p.N;
        out[batch_offset(p, batch, p.so.b, p.ho) + m * p.so.r + n * p.so.c] = plus_bias(v, p.bias, n);
    }
}

// ---- rowdot family (f32, small N) ---------------------------------------------------------------

constexpr int kRowdotMaxN = 4;

// One wave per (batch, row); lanes stride along K.
template <bool AVec>
__global__ __launch_bounds__(kThreads) void rowdot_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ out, MatmulArgs p) {
    const int lane = threadIdx.x % 64;
    const int64_t row_id = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + threadIdx.x / 64;
    if (row_id >= p.batches * p.M) return;
    const int64_t batch = row_id / p.M;
    const int64_t m = row_id % p.M;
    const float* arow = a + batch_offset(p, batch, p.sa.b, p.ha) + m * p.sa.r;
    const float* bb = b + batch_offset(p, batch, p.sb.b, p.hb);
    float acc[kRowdotMaxN] = {0.f, 0.f, 0.f, 0.f};
    if (AVec) {
        const int64_t vecs = p.K / 4;
        for (int64_t v = lane; v < vecs; v += 64) {
            const float4 x = *reinterpret_cast<const float4*>(arow + 4 * v);
            const int64_t k = 4 * v;
#pragma unroll
            for (int n = 0; n < kRowdotMaxN; ++n) {
                if (n < p.N) {
                    const float* bc = bb + n * p.sb.c;
                    acc[n] += x.x * bc[k * p.sb.r] + x.y * bc[(k + 1) * p.sb.r] + x.z * bc[(k + 2) * p.sb.r] +
                              x.w * bc[(k + 3) * p.sb.r];
                }
            }
        }
        for (int64_t k = vecs * 4 + lane; k < p.K; k += 64) {
#pragma unroll
            for (int n = 0; n < kRowdotMaxN; ++n)
                if (n < p.N) acc[n] += arow[k] * bb[k * p.sb.r + n * p.sb.c];
        }
    } else {
        for (int64_t k = lane; k < p.K; k += 64) {
            const float x = arow[k * p.sa.c];
#pragma unroll
            for (int n = 0; n < kRowdotMaxN; ++n)
                if (n < p.N) acc[n] += x * bb[k * p.sb.r + n * p.sb.c];
        }
    }
#pragma unroll
    for (int n = 0; n < kRowdotMaxN; ++n) {
#pragma unroll
        for (int off = 32; off > 0; off /= 2) acc[n] += __shfl_xor(acc[n], off, 64);
    }
    if (lane == 0) {
#pragma unroll
        for (int n = 0; n < kRowdotMaxN; ++n)
            if (n < p.N) out[batch_offset(p, batch, p.so.b, p.ho) + m * p.so.r + n * p.so.c] = plus_bias(acc[n], p.bias, n);
    }
}

// ---- tiled family (f64 / i64) ----------------------------------------------------------------------

constexpr int kTT = 64;  // tile edge
constexpr int kTK = 16;

template <typename T> __device__ __forceinline__ T mul_add(T acc, T x, T y) {
    if constexpr (std::is_same_v<T, int64_t>) return wrap_add(acc, wrap_mul(x, y));
    else return acc + x * y;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void tiled_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                         T* __restrict__ out, MatmulArgs p) {
    __shared__ T As[kTK][kTT + 1];
    __shared__ T Bs[kTK][kTT + 1];
    const int64_t batch = blockIdx.z;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kTT;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kTT;
    a += batch_offset(p, batch, p.sa.b, p.ha);
    b += batch_offset(p, batch, p.sb.b, p.hb);
    const int tr = threadIdx.x / 16;  // 0..15 -> rows tr*4 .. +3
    const int tc = threadIdx.x % 16;  // cols tc + 16*j
    T acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = T(0);
    for (int64_t k0 = 0; k0 < p.K; k0 += kTK) {
        for (int idx = threadIdx.x; idx < kTK * kTT; idx += kThreads) {
            const int kk = idx % kTK;
            const int mm = idx / kTK;
            const int64_t m = m0 + mm, k = k0 + kk;
            As[kk][mm] = (m < p.M && k < p.K) ? a[m * p.sa.r + k * p.sa.c] : T(0);
            const int nn = idx % kTT;
            const int kb = idx / kTT;
            const int64_t n = n0 + nn, k2 = k0 + kb;
            Bs[kb][nn] = (n < p.N && k2 < p.K) ? b[k2 * p.sb.r + n * p.sb.c] : T(0);
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kTK; ++kk) {
            T av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = As[kk][tr * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tc + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mul_add(acc[i][j], av[i], bv[j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + tr * 4 + i;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t n = n0 + tc + 16 * j;
            if (n < p.N) out[batch_offset(p, batch, p.so.b, p.ho) + m * p.so.r + n * p.so.c] = plus_bias(acc[i][j], p.bias, n);
        }
    }
}

// ---- dispatch ----------------------------------------------------------------------------------

bool aligned16(const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }

// Status of the launch just issued (KD_LAUNCH_CHECK for callers that report through a pointer).
int launch_status() {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? KD_OK : ::kd::hip_fail(e, "kernel launch", __FILE__, __LINE__);
}

// 64x64 tiles (mfma_f32_t64_kernel) for whole-tile products (M, N multiples of 64, K of 32,
// 32-bit offsets) whose 128x128 grid, batch included, would not give every CU a workgroup, or whose
// M or N is not a multiple of 128 (the alternative is the bounds-checked general kernel). Measured
// on C4's products: the attention batches (128 x 128 x 128 x 64) 6.5 us against 16.2 on the general
// kernel, x . W^T over the folded batch with N = 256 22-29 us against 27-31 with split K. When
// even the 64x64 grid fills at most half the CUs and K >= 512, K is split over the kernel's batch
// slot into a workspace that split_sum_kernel adds in split order. Returns false when the product
// does not take this path.
template <bool AT, bool BT> bool launch_t64(const float* a, const float* b, float* out, const MatmulArgs& p, int* rc) {
    constexpr int64_t kMax = int64_t{1} << 31;
    const int64_t lda = AT ? p.sa.c : p.sa.r;
    const int64_t ldb = BT ? p.sb.c : p.sb.r;
    const int64_t a_extent = AT ? p.K * lda + p.M : p.M * lda + p.K;
    const int64_t b_extent = BT ? p.N * ldb + p.K : p.K * ldb + p.N;
    // a ragged last tile row (M a multiple of 4, one product): the tied LM head's 96 x 4096 x 256
    // weight gradient, 20 us on the general kernel's split K
    const bool ragged = p.M % kT64 != 0;
    if ((ragged && (p.M % 4 != 0 || p.batches != 1)) || p.N % kT64 != 0 || p.K % kT64K != 0 || p.K == 0 ||
        p.so.c != 1 || a_extent >= kMax || b_extent >= kMax || p.M * p.so.r + p.N >= kMax)
        return false;
    const int cus = compute_units();
    const bool whole128 = p.M % kBM == 0 && p.N % kBN == 0 && p.K % kBK == 0;
    // the batch folds into M when the batches share B and lie back to back in A and the output
    const bool fold = !AT && p.heads == 1 && p.sb.b == 0 && p.sa.b == p.M * lda && p.so.b == p.M * p.so.r;
    const int64_t rows = fold ? p.M * p.batches : p.M;
    const int64_t batches = fold ? 1 : p.batches;
    if (fold && (rows * lda >= kMax || rows * p.so.r >= kMax)) return false;
    const int64_t tiles128 = (rows / kBM) * (p.N / kBN);
    if (whole128 && tiles128 * batches >= cus) return false;
    // One product with 5 or more 128x128 tiles splits K on them (C4's 256 x 4096 x 768 weight
    // gradient: 28.7 us against 32.1 on 64x64 tiles split 4 ways); with at most 4 the 64x64 grid
    // wins (256 x 4096 x 256: 13 us against 21).
    if (whole128 && p.batches == 1 && tiles128 > 4) return false;
    const int64_t tiles = (rows + kT64 - 1) / kT64 * (p.N / kT64);
    if (batches > 65535) return false;
    if (batches == 1 && tiles * 2 <= cus && p.K >= 512) {
        int64_t splits = std::min<int64_t>(p.K / 256, (cus + tiles - 1) / tiles);
        while (splits > 1 && p.K % (splits * kT64K) != 0) --splits;
        const int64_t per = rows * p.N;
        if (splits > 1 && splits * per < kMax) {
            Workspace ws;  // held until split_sum_kernel is enqueued
            if ((*rc = workspace(ws, static_cast<size_t>(splits * per) * sizeof(float)))) return true;
            const int64_t kc = p.K / splits;
            const dim3 grid(static_cast<uint32_t>(tiles), static_cast<uint32_t>(splits));
            const BatchStrides bs = batch_strides(AT ? kc * lda : kc, BT ? kc : kc * ldb, per);
            if (ragged)
                hipLaunchKernelGGL((mfma_f32_t64_kernel<AT, BT, true>), grid, dim3(kThreads), 0, stream(), a, b,
                                   static_cast<float*>(ws.ptr), static_cast<int>(rows), static_cast<int>(p.N),
                                   static_cast<int>(kc), static_cast<int>(lda), static_cast<int>(ldb),
                                   static_cast<int>(p.N), bs);
            else
                hipLaunchKernelGGL((mfma_f32_t64_kernel<AT, BT>), grid, dim3(kThreads), 0, stream(), a, b,
                                   static_cast<float*>(ws.ptr), static_cast<int>(rows), static_cast<int>(p.N),
                                   static_cast<int>(kc), static_cast<int>(lda), static_cast<int>(ldb),
                                   static_cast<int>(p.N), bs);
            if ((*rc = launch_status())) return true;
            MatmulArgs flat = p;
            flat.batches = 1;
            flat.M = rows;
            const int64_t blocks = std::min<int64_t>((per + kThreads - 1) / kThreads, int64_t{cus} * 16);
            hipLaunchKernelGGL(split_sum_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream(),
                               static_cast<const float*>(ws.ptr), out, flat, splits);
            *rc = launch_status();
            return true;
        }
    }
    const dim3 grid(static_cast<uint32_t>(tiles), static_cast<uint32_t>(batches));
    if (ragged)
        hipLaunchKernelGGL((mfma_f32_t64_kernel<AT, BT, true>), grid, dim3(kThreads), 0, stream(), a, b, out,
                           static_cast<int>(rows), static_cast<int>(p.N), static_cast<int>(p.K), static_cast<int>(lda),
                           static_cast<int>(ldb), static_cast<int>(p.so.r), batch_strides(p));
    else
        hipLaunchKernelGGL((mfma_f32_t64_kernel<AT, BT>), grid, dim3(kThreads), 0, stream(), a, b, out,
                           static_cast<int>(rows), static_cast<int>(p.N), static_cast<int>(p.K), static_cast<int>(lda),
                           static_cast<int>(ldb), static_cast<int>(p.so.r), batch_strides(p));
    *rc = launch_status();
    return true;
}

// mfma_f32_trans_kernel on `grid`: the instantiation that keeps two K steps of loads in flight
// where the grid leaves at most two workgroups per CU (C4's products: 192-256 workgroups, one wave
// per SIMD), the one-step pipeline (fewer registers, four waves per SIMD) otherwise.
template <bool AT, bool BT, bool Bias = false>
void launch_trans(dim3 grid, const float* a, const float* b, float* out, int64_t M, int64_t N, int64_t K, int64_t lda,
                  int64_t ldb, int64_t ldo, const BatchStrides& bs) {
    const int64_t groups = int64_t{grid.x} * grid.y * grid.z;
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    const int la = static_cast<int>(lda), lb = static_cast<int>(ldb), lo = static_cast<int>(ldo);
    if (groups <= 2 * int64_t{compute_units()})
        hipLaunchKernelGGL((mfma_f32_trans_kernel<AT, BT, Bias, true>), grid, dim3(kThreads), 0, stream(), a, b, out, m,
                           n, k, la, lb, lo, bs);
    else
        hipLaunchKernelGGL((mfma_f32_trans_kernel<AT, BT, Bias, false>), grid, dim3(kThreads), 0, stream(), a, b, out, m,
                           n, k, la, lb, lo, bs);
}

template <int AMode, int BMode> int launch_mfma(const float* a, const float* b, float* out, const MatmulArgs& p) {
    const int64_t tiles = ((p.M + kBM - 1) / kBM) * ((p.N + kBN - 1) / kBN);
    if (p.batches > 65535) return fail(KD_E_INVALID, "kd_matmul: too many batches");
    const dim3 grid(static_cast<uint32_t>(tiles), static_cast<uint32_t>(p.batches));
    if constexpr (AMode != kGeneric && BMode != kGeneric) {
        int rc = KD_OK;
        if (launch_t64<AMode == kColVec, BMode == kColVec>(a, b, out, p, &rc)) return rc;
    }
    if constexpr (AMode == kRowVec && BMode == kRowVec) {
        constexpr int64_t kMax = int64_t{1} << 31;
        const bool small = p.M * p.sa.r < kMax && p.K * p.sb.r < kMax && p.M * p.so.r < kMax && p.so.c == 1;
        if (small && p.M % kBM == 0 && p.N % kBN == 0 && p.K % kBK == 0) {
            // Too few tiles to occupy the device (C1's 512^3 has 16): split K so that about one
            // workgroup per CU is busy, partial products into the workspace, summed in split order.
            const int cus = compute_units();
            int64_t splits = 1;
            if (p.heads == 1 && tiles * p.batches * 2 <= cus && p.K >= 256 &&
                p.M * p.N * p.batches * (cus / tiles) < kMax) {
                splits = std::min<int64_t>(p.K / 64, (cus + tiles * p.batches - 1) / (tiles * p.batches));
                while (splits > 1 && p.K % (splits * kBK) != 0) --splits;
            }
            if (splits > 1) {
                Workspace ws;  // held until split_sum_kernel is enqueued
                const int64_t per = p.M * p.N;
                if (int rc = workspace(ws, static_cast<size_t>(splits * p.batches * per) * sizeof(float))) return rc;
                const int64_t kc = p.K / splits;
                hipLaunchKernelGGL(mfma_f32_rowmajor_kernel,
                                   dim3(static_cast<uint32_t>(tiles), static_cast<uint32_t>(p.batches),
                                        static_cast<uint32_t>(splits)),
                                   dim3(kThreads), 0, stream(), a, b, static_cast<float*>(ws.ptr), static_cast<int>(p.M),
                                   static_cast<int>(p.N), static_cast<int>(kc), static_cast<int>(p.sa.r),
                                   static_cast<int>(p.sb.r), static_cast<int>(p.N), p.sa.b, p.sb.b, splits * per, kc,
                                   kc * p.sb.r, per);
                KD_LAUNCH_CHECK();
                const int64_t total = p.batches * per;
                const int64_t blocks = std::min<int64_t>((total + kThreads - 1) / kThreads, int64_t{cus} * 16);
                hipLaunchKernelGGL(split_sum_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream(),
                                   static_cast<const float*>(ws.ptr), out, p, splits);
                KD_LAUNCH_CHECK();
                return KD_OK;
            }
            // Whole tiles without split K: the same tiles and MFMA order on the loader of the
            // transposed-operand family (waves 0-1 load A, waves 2-3 load B, four 16-byte loads
            // each), which measured ~1 % faster than mfma_f32_rowmajor_kernel at 4096^3 with
            // bit-identical results. The bounds checked above cover its 32-bit offsets.
            if (p.bias != nullptr)
                launch_trans<false, false, true>(grid, a, b, out, p.M, p.N, p.K, p.sa.r, p.sb.r, p.so.r, batch_strides(p));
            else
                launch_trans<false, false>(grid, a, b, out, p.M, p.N, p.K, p.sa.r, p.sb.r, p.so.r, batch_strides(p));
            KD_LAUNCH_CHECK();
            return KD_OK;
        }
    }
    if constexpr ((AMode == kColVec || BMode == kColVec) && AMode != kGeneric && BMode != kGeneric) {
        // A transposed and/or B transposed, whole tiles, 32-bit offsets: the conflict-free loaders.
        constexpr bool at = AMode == kColVec;
        constexpr bool bt = BMode == kColVec;
        constexpr int64_t kMax = int64_t{1} << 31;
        const int64_t lda = at ? p.sa.c : p.sa.r;
        const int64_t ldb = bt ? p.sb.c : p.sb.r;
        const int64_t a_extent = at ? p.K * lda + p.M : p.M * lda + p.K;
        const int64_t b_extent = bt ? p.N * ldb + p.K : p.K * ldb + p.N;
        if (a_extent < kMax && b_extent < kMax && p.M * p.so.r + p.N < kMax && p.so.c == 1 && p.M % kBM == 0 &&
            p.N % kBN == 0 && p.K % kBK == 0) {
            // Too few tiles to occupy the device, for one product (C4's weight gradient X^T . g:
            // 256 x 768 outputs, 12 tiles, K = 4096) or for x . W^T over a batch with one shared
            // weight (kael's Linear: B broadcast, A and the output batches back to back; C4's
            // 4096 x 256 outputs have 64), whose batch folds into M: K is split, the splits
            // taking the kernel's batch slot (their K offsets as batch strides) and writing
            // partial products that split_sum_kernel adds in split order.
            const int cus = compute_units();
            const int64_t rows = p.M * p.batches;
            const int64_t flat_tiles = (rows / kBM) * (p.N / kBN);
            const bool fold = !at && p.heads == 1 && p.sb.b == 0 && p.sa.b == p.M * lda && p.so.b == p.M * p.so.r;
            {
                if ((p.batches == 1 || fold) && flat_tiles * 2 <= cus && p.K >= 256 &&
                    (at || rows * lda < kMax) && rows * p.so.r < kMax) {
                    int64_t splits = std::min<int64_t>(p.K / 64, (cus + flat_tiles - 1) / flat_tiles);
                    while (splits > 1 && p.K % (splits * kBK) != 0) --splits;
                    const int64_t per = rows * p.N;
                    if (splits > 1 && splits * per < kMax) {
                        Workspace ws;  // held until split_sum_kernel is enqueued
                        if (int rc = workspace(ws, static_cast<size_t>(splits * per) * sizeof(float))) return rc;
                        const int64_t kc = p.K / splits;
                        launch_trans<at, bt>(dim3(static_cast<uint32_t>(flat_tiles), static_cast<uint32_t>(splits)), a, b,
                                             static_cast<float*>(ws.ptr), rows, p.N, kc, lda, ldb, p.N,
                                             batch_strides(at ? kc * lda : kc, bt ? kc : kc * ldb, per));
                        KD_LAUNCH_CHECK();
                        MatmulArgs flat = p;
                        flat.batches = 1;
                        flat.M = rows;
                        const int64_t blocks = std::min<int64_t>((per + kThreads - 1) / kThreads, int64_t{cus} * 16);
                        hipLaunchKernelGGL(split_sum_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0,
                                           stream(), static_cast<const float*>(ws.ptr), out, flat, splits);
                        KD_LAUNCH_CHECK();
                        return KD_OK;
                    }
                }
            }
            if (p.bias != nullptr)
                launch_trans<at, bt, true>(grid, a, b, out, p.M, p.N, p.K, lda, ldb, p.so.r, batch_strides(p));
            else
                launch_trans<at, bt>(grid, a, b, out, p.M, p.N, p.K, lda, ldb, p.so.r, batch_strides(p));
            KD_LAUNCH_CHECK();
            return KD_OK;
        }
    }
    {
        // Few tiles and a long K on the general kernel (a ragged M or N, any strides; C4's tied
        // LM-head weight gradient, 96 x 256 outputs over K = 4096 tokens, is 2 tiles): K is split so
        // that about one workgroup per CU is busy, the splits taking the kernel's batch slot (their
        // K offsets as batch strides) and writing partial products that split_sum_kernel adds in
        // split order, bias included.
        const int cus = compute_units();
        const int64_t per = p.M * p.N;
        if (p.batches == 1 && p.heads == 1 && tiles * 2 <= cus && p.K >= 1024) {
            int64_t splits = std::min<int64_t>(p.K / 64, cus / tiles);
            while (splits > 1 && p.K % (splits * kBK) != 0) --splits;
            if (splits > 1 && splits * per < (int64_t{1} << 31)) {
                Workspace ws;  // held until split_sum_kernel is enqueued
                if (int rc = workspace(ws, static_cast<size_t>(splits * per) * sizeof(float))) return rc;
                MatmulArgs part = p;
                part.batches = splits;
                part.K = p.K / splits;
                part.sa.b = part.K * p.sa.c;
                part.sb.b = part.K * p.sb.r;
                part.so = Strides3{per, p.N, 1};
                part.bias = nullptr;
                hipLaunchKernelGGL((mfma_f32_kernel<AMode, BMode, false>),
                                   dim3(static_cast<uint32_t>(tiles), static_cast<uint32_t>(splits)), dim3(kThreads), 0,
                                   stream(), a, b, static_cast<float*>(ws.ptr), part);
                KD_LAUNCH_CHECK();
                const int64_t blocks = std::min<int64_t>((per + kThreads - 1) / kThreads, int64_t{cus} * 16);
                hipLaunchKernelGGL(split_sum_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream(),
                                   static_cast<const float*>(ws.ptr), out, p, splits);
                KD_LAUNCH_CHECK();
                return KD_OK;
            }
        }
    }
    bool full = false;
    if constexpr (AMode != kGeneric && BMode != kGeneric) full = p.M % kBM == 0 && p.N % kBN == 0 && p.K % kBK == 0;
    const bool bias = p.bias != nullptr;
    if (full) {
        if constexpr (AMode != kGeneric && BMode != kGeneric) {
            if (bias) hipLaunchKernelGGL((mfma_f32_kernel<AMode, BMode, true, true>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
            else hipLaunchKernelGGL((mfma_f32_kernel<AMode, BMode, true>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
        }
    } else {
        if (bias) hipLaunchKernelGGL((mfma_f32_kernel<AMode, BMode, false, true>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
        else hipLaunchKernelGGL((mfma_f32_kernel<AMode, BMode, false>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
    }
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <int AMode> int launch_mfma_b(const float* a, const float* b, float* out, const MatmulArgs& p, int bmode) {
    switch (bmode) {
    case kRowVec: return launch_mfma<AMode, kRowVec>(a, b, out, p);
    case kColVec: return launch_mfma<AMode, kColVec>(a, b, out, p);
    default: return launch_mfma<AMode, kGeneric>(a, b, out, p);
    }
}

int matmul_f32(const float* a, const float* b, float* out, const MatmulArgs& p) {
    const int cus = compute_units();
    if (p.N <= kRowdotMaxN) {
        const bool avec = p.sa.c == 1 && p.sa.r % 4 == 0 && p.sa.b % 4 == 0 && p.ha % 4 == 0 && aligned16(a);
        const int64_t waves = p.batches * p.M;
        const dim3 grid(static_cast<uint32_t>((waves + 3) / 4));
        if (avec) hipLaunchKernelGGL((rowdot_kernel<true>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
        else hipLaunchKernelGGL((rowdot_kernel<false>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    if (p.M <= kSkinnyMaxM) {
        const bool bvec = p.sb.c == 1 && p.sb.r % 4 == 0 && p.sb.b % 4 == 0 && p.hb % 4 == 0 && aligned16(b);
        const int64_t col_blocks = (p.N + kSkinnyCols - 1) / kSkinnyCols;
        int64_t splits = 1;
        const int64_t want = 2 * int64_t{cus};
        if (col_blocks * p.batches < want) {
            splits = std::min<int64_t>((want + col_blocks * p.batches - 1) / (col_blocks * p.batches),
                                       std::max<int64_t>(1, p.K / 32));
        }
        const int64_t k_chunk = (p.K + splits - 1) / splits;
        splits = (p.K + k_chunk - 1) / k_chunk;
        if (splits < 1) splits = 1;
        float* partial = nullptr;
        Workspace ws;  // held (when split) until split_sum_kernel is enqueued
        if (splits > 1) {
            if (int rc = workspace(ws, static_cast<size_t>(p.batches * splits * p.M * p.N) * sizeof(float))) return rc;
            partial = static_cast<float*>(ws.ptr);
        }
        if (p.batches > 65535 || splits > 65535) return fail(KD_E_INVALID, "kd_matmul: grid too large");
        const dim3 grid(static_cast<uint32_t>(col_blocks), static_cast<uint32_t>(splits), static_cast<uint32_t>(p.batches));
#define KD_SKINNY(MT)                                                                                               \
    if (bvec) hipLaunchKernelGGL((skinny_kernel<MT, true>), grid, dim3(kThreads), 0, stream(), a, b, out, partial, p, k_chunk); \
    else hipLaunchKernelGGL((skinny_kernel<MT, false>), grid, dim3(kThreads), 0, stream(), a, b, out, partial, p, k_chunk);
        if (p.M <= 1) { KD_SKINNY(1) }
        else if (p.M <= 4) { KD_SKINNY(4) }
        else if (p.M <= 8) { KD_SKINNY(8) }
        else { KD_SKINNY(16) }
#undef KD_SKINNY
        KD_LAUNCH_CHECK();
        if (splits > 1) {
            const int64_t total = p.batches * p.M * p.N;
            const int64_t blocks = std::min<int64_t>((total + kThreads - 1) / kThreads, int64_t{cus} * 16);
            hipLaunchKernelGGL(split_sum_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kThreads), 0, stream(), partial,
                               out, p, splits);
            KD_LAUNCH_CHECK();
        }
        return KD_OK;
    }
    {
        // Few 128x128 tiles (at most half the CUs busy) and K <= 2048: 32x32 tiles in one launch
        // (512^3: 6.1 us against 15.6 us with split K; 64x784x128: 7.6 us against 65 us on one
        // 128x128 tile). Longer K with few tiles stays with split K (128x4096x128: 25 us against
        // 31 us), and so do grids of more than 2 small tiles per CU (1024^3: 32 us with split K).
        const int64_t big = ((p.M + kBM - 1) / kBM) * ((p.N + kBN - 1) / kBN) * p.batches;
        const int64_t gm = (p.M + kSmallTile - 1) / kSmallTile;
        const int64_t gn = (p.N + kSmallTile - 1) / kSmallTile;
        const bool fits32 = p.K * std::abs(p.sa.c) < (int64_t{1} << 31) && p.K * std::abs(p.sb.r) < (int64_t{1} << 31);
        if (big * 2 <= cus && gm * gn * p.batches <= 2 * int64_t{cus} && p.K <= 2048 && fits32) {
            if (p.batches > 65535 || gm > 65535) return fail(KD_E_INVALID, "kd_matmul: grid too large");
            const dim3 grid(static_cast<uint32_t>(gn), static_cast<uint32_t>(gm), static_cast<uint32_t>(p.batches));
            const bool avec = p.sa.c == 1 && p.sa.r % 4 == 0 && p.sa.b % 4 == 0 && p.ha % 4 == 0 && aligned16(a);
            if (avec) hipLaunchKernelGGL(small_kernel<true>, grid, dim3(kSmallWaves * 64), 0, stream(), a, b, out, p);
            else hipLaunchKernelGGL(small_kernel<false>, grid, dim3(kSmallWaves * 64), 0, stream(), a, b, out, p);
            KD_LAUNCH_CHECK();
            return KD_OK;
        }
    }
    int amode = kGeneric, bmode = kGeneric;
    if (p.sa.c == 1 && p.sa.r % 4 == 0 && p.sa.b % 4 == 0 && p.ha % 4 == 0 && p.K % 4 == 0 && aligned16(a)) amode = kRowVec;
    else if (p.sa.r == 1 && p.sa.c % 4 == 0 && p.sa.b % 4 == 0 && p.ha % 4 == 0 && p.M % 4 == 0 && aligned16(a)) amode = kColVec;
    if (p.sb.c == 1 && p.sb.r % 4 == 0 && p.sb.b % 4 == 0 && p.hb % 4 == 0 && p.N % 4 == 0 && aligned16(b)) bmode = kRowVec;
    else if (p.sb.r == 1 && p.sb.c % 4 == 0 && p.sb.b % 4 == 0 && p.hb % 4 == 0 && p.K % 4 == 0 && aligned16(b)) bmode = kColVec;
    switch (amode) {
    case kRowVec: return launch_mfma_b<kRowVec>(a, b, out, p, bmode);
    case kColVec: return launch_mfma_b<kColVec>(a, b, out, p, bmode);
    default: return launch_mfma_b<kGeneric>(a, b, out, p, bmode);
    }
}

// ---- f64 on the FP64 matrix cores ------------------------------------------------------------
//
// 64x64 output tiles, four waves each a 2x2 grid of 16x16 v_mfma_f64_16x16x4f64 accumulators;
// K advances 16 at a time through double-buffered LDS, the next stage's elements in registers
// while the current one multiplies. Any operand strides (each thread loads 4 elements of A and 4
// of B per stage, one at a time), batches with one or two stride levels, the bias epilogue; Full
// drops the bounds checks for whole tiles. Lane layout of the 16x16x4 f64 MFMA (measured with
// random operands on gfx950): A[i][k] and B[k][j] come from lane i + 16 k (j + 16 k), and
// register r of lane l holds D[l / 16 + 4 r][l % 16].
constexpr int kD = 64;
constexpr int kDK = 16;
constexpr int kDAld = kDK + 1;  // A tile [m][k]: odd stride, the 16 rows a wave reads spread over the banks
constexpr int kDBld = kD + 1;   // B tile [k][n]
typedef double v4d __attribute__((ext_vector_type(4)));

template <bool Full>
__global__ __launch_bounds__(kThreads) void mfma_f64_kernel(const double* __restrict__ a, const double* __restrict__ b,
                                                            double* __restrict__ out, MatmulArgs p) {
    __shared__ double As[2][kD * kDAld];
    __shared__ double Bs[2][kDK * kDBld];
    const int64_t tiles_m = (p.M + kD - 1) / kD;
    const int64_t tiles_n = (p.N + kD - 1) / kD;
    int64_t tm, tn;
    tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t batch = blockIdx.y;
    const int64_t m0 = tm * kD;
    const int64_t n0 = tn * kD;
    a += batch_offset(p, batch, p.sa.b, p.ha);
    b += batch_offset(p, batch, p.sb.b, p.hb);
    out += batch_offset(p, batch, p.so.b, p.ho);

    const int t = threadIdx.x;
    const int lane = t % 64;
    const int wave = t / 64;
    const int wm = wave / 2;
    const int wn = wave % 2;
    const int li = lane % 16;
    const int lk = lane / 16;

    v4d acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};

    double ra[4], rb[4];
    const auto fetch = [&](int64_t k0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = t + kThreads * e;
            const int64_t m = m0 + idx / kDK, ka = k0 + idx % kDK;
            ra[e] = (Full || (m < p.M && ka < p.K)) ? a[m * p.sa.r + ka * p.sa.c] : 0.0;
            const int64_t kb = k0 + idx / kD, n = n0 + idx % kD;
            rb[e] = (Full || (kb < p.K && n < p.N)) ? b[kb * p.sb.r + n * p.sb.c] : 0.0;
        }
    };
    const auto stash = [&](int buf) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int idx = t + kThreads * e;
            As[buf][(idx / kDK) * kDAld + idx % kDK] = ra[e];
            Bs[buf][(idx / kD) * kDBld + idx % kD] = rb[e];
        }
    };
    fetch(0);
    stash(0);
    __syncthreads();
    const int64_t ksteps = (p.K + kDK - 1) / kDK;
    for (int64_t ks = 0; ks < ksteps; ++ks) {
        const int cur = static_cast<int>(ks & 1);
        const bool more = ks + 1 < ksteps;
        if (more) fetch((ks + 1) * kDK);
        const double* as = As[cur];
        const double* bs = Bs[cur];
#pragma unroll
        for (int kk = 0; kk < kDK; kk += 4) {
            double av[2], bv[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = as[(wm * 32 + i * 16 + li) * kDAld + kk + lk];
#pragma unroll
            for (int j = 0; j < 2; ++j) bv[j] = bs[(kk + lk) * kDBld + wn * 32 + j * 16 + li];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[i], bv[j], acc[i][j], 0, 0, 0);
        }
        if (more) stash(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t col = n0 + wn * 32 + j * 16 + li;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * 32 + i * 16 + lk + 4 * r;
                if (Full || (row < p.M && col < p.N))
                    out[row * p.so.r + col * p.so.c] = plus_bias(acc[i][j][r], p.bias, col);
            }
        }
}

int matmul_f64(const double* a, const double* b, double* out, const MatmulArgs& p) {
    if (p.batches > 65535) return fail(KD_E_INVALID, "kd_matmul: too many batches");
    const int64_t tiles = ((p.M + kD - 1) / kD) * ((p.N + kD - 1) / kD);
    if (tiles > (int64_t{1} << 31) - 1) return fail(KD_E_INVALID, "kd_matmul: too many tiles");
    const dim3 grid(static_cast<uint32_t>(tiles), static_cast<uint32_t>(p.batches));
    const bool full = p.M % kD == 0 && p.N % kD == 0 && p.K % kDK == 0;
    if (full) hipLaunchKernelGGL((mfma_f64_kernel<true>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
    else hipLaunchKernelGGL((mfma_f64_kernel<false>), grid, dim3(kThreads), 0, stream(), a, b, out, p);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <typename T> int matmul_tiled(const T* a, const T* b, T* out, const MatmulArgs& p) {
    if (p.batches > 65535) return fail(KD_E_INVALID, "kd_matmul: too many batches");
    const int64_t gm = (p.M + kTT - 1) / kTT, gn = (p.N + kTT - 1) / kTT;
    if (gm > 65535) return fail(KD_E_INVALID, "kd_matmul: too many rows");
    hipLaunchKernelGGL((tiled_kernel<T>), dim3(static_cast<uint32_t>(gn), static_cast<uint32_t>(gm), static_cast<uint32_t>(p.batches)),
                       dim3(kThreads), 0, stream(), a, b, out, p);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void zero_kernel(T* out, MatmulArgs p) {
    const int64_t total = p.batches * p.M * p.N;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t batch = idx / (p.M * p.N);
        const int64_t m = (idx / p.N) % p.M;
        const int64_t n = idx % p.N;
        out[batch_offset(p, batch, p.so.b, p.ho) + m * p.so.r + n * p.so.c] = plus_bias(T(0), p.bias, n);
    }
}

int dispatch(int dtype, const void* a, const void* b, void* out, const MatmulArgs& p) {
    if (dtype == KD_BOOL) return fail(KD_E_UNSUPPORTED, "matmul does not support dtype bool");
    if (dtype_size(dtype) == 0) return fail(KD_E_INVALID, "kd_matmul: unknown dtype");
    if (p.batches < 0 || p.M < 0 || p.K < 0 || p.N < 0) return fail(KD_E_INVALID, "kd_matmul: negative size");
    if (p.batches == 0 || p.M == 0 || p.N == 0) return KD_OK;
    if (int rc = ensure_device()) return rc;
    if (p.K == 0) {
        // An empty inner dimension yields zeros (the reference's accumulators start at zero).
        const int64_t total = p.batches * p.M * p.N;
        const int64_t blocks = std::min<int64_t>((total + kThreads - 1) / kThreads, int64_t{compute_units()} * 16);
        const dim3 grid(static_cast<uint32_t>(blocks));
        if (dtype == KD_F32) hipLaunchKernelGGL((zero_kernel<float>), grid, dim3(kThreads), 0, stream(), static_cast<float*>(out), p);
        else if (dtype == KD_F64) hipLaunchKernelGGL((zero_kernel<double>), grid, dim3(kThreads), 0, stream(), static_cast<double*>(out), p);
        else hipLaunchKernelGGL((zero_kernel<int64_t>), grid, dim3(kThreads), 0, stream(), static_cast<int64_t*>(out), p);
        KD_LAUNCH_CHECK();
        return KD_OK;
    }
    switch (dtype) {
    case KD_F32: return matmul_f32(static_cast<const float*>(a), static_cast<const float*>(b), static_cast<float*>(out), p);
    case KD_F64: return matmul_f64(static_cast<const double*>(a), static_cast<const double*>(b), static_cast<double*>(out), p);
    default: return matmul_tiled<int64_t>(static_cast<const int64_t*>(a), static_cast<const int64_t*>(b), static_cast<int64_t*>(out), p);
    }
}

} // namespace

int matmul_split_parts(const float* a, const float* b, float* parts, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, int64_t splits) {
    constexpr int64_t kMax = int64_t{1} << 31;
    if (M <= 0 || N <= 0 || splits < 1 || M % kT64 != 0 || N % kT64 != 0 || K % (kT64K * splits) != 0 || lda % 4 != 0 ||
        ldb % 4 != 0 || !aligned16(a) || !aligned16(b) || !aligned16(parts) || M * lda >= kMax || K * ldb >= kMax ||
        splits * M * N >= kMax || splits > 65535)
        return fail(KD_E_INVALID, "matmul_split_parts: operands outside the 64x64 split-K kernel's bounds");
    const int64_t tiles = (M / kT64) * (N / kT64);
    const int64_t kc = K / splits;
    hipLaunchKernelGGL((mfma_f32_t64_kernel<false, false>), dim3(static_cast<uint32_t>(tiles), static_cast<uint32_t>(splits)),
                       dim3(kThreads), 0, stream(), a, b, parts, static_cast<int>(M), static_cast<int>(N),
                       static_cast<int>(kc), static_cast<int>(lda), static_cast<int>(ldb), static_cast<int>(N),
                       batch_strides(kc, kc * ldb, M * N));
    return launch_status();
}

} // namespace kd

using namespace kd;

extern "C" int kd_matmul(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes) {
    if (sizes == nullptr) return fail(KD_E_INVALID, "kd_matmul: null sizes");
    MatmulArgs p;
    p.batches = sizes->batches;
    p.M = sizes->rows;
    p.K = sizes->inner;
    p.N = sizes->columns;
    p.sa = {p.M * p.K, p.K, 1};
    p.sb = {p.K * p.N, p.N, 1};
    p.so = {p.M * p.N, p.N, 1};
    return dispatch(dtype, a, b, out, p);
}

extern "C" int kd_matmul_strided(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                                 const kd_matmul_strides* strides) {
    if (sizes == nullptr || strides == nullptr) return fail(KD_E_INVALID, "kd_matmul_strided: null argument");
    MatmulArgs p;
    p.batches = sizes->batches;
    p.M = sizes->rows;
    p.K = sizes->inner;
    p.N = sizes->columns;
    p.sa = {strides->a[0], strides->a[1], strides->a[2]};
    p.sb = {strides->b[0], strides->b[1], strides->b[2]};
    p.so = {strides->out[0], strides->out[1], strides->out[2]};
    return dispatch(dtype, a, b, out, p);
}

extern "C" int kd_matmul_strided_bias(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                                      const kd_matmul_strides* strides, const void* bias) {
    if (sizes == nullptr || strides == nullptr) return fail(KD_E_INVALID, "kd_matmul_strided_bias: null argument");
    if (bias == nullptr && sizes->batches > 0 && sizes->rows > 0 && sizes->columns > 0)
        return fail(KD_E_INVALID, "kd_matmul_strided_bias: null bias");
    MatmulArgs p;
    p.batches = sizes->batches;
    p.M = sizes->rows;
    p.K = sizes->inner;
    p.N = sizes->columns;
    p.sa = {strides->a[0], strides->a[1], strides->a[2]};
    p.sb = {strides->b[0], strides->b[1], strides->b[2]};
    p.so = {strides->out[0], strides->out[1], strides->out[2]};
    p.bias = bias;
    return dispatch(dtype, a, b, out, p);
}

extern "C" int kd_matmul_strided_heads(int dtype, const void* a, const void* b, void* out, const kd_matmul_sizes* sizes,
                                       const kd_matmul_strides* strides, const kd_matmul_heads* heads) {
    if (sizes == nullptr || strides == nullptr || heads == nullptr)
        return fail(KD_E_INVALID, "kd_matmul_strided_heads: null argument");
    if (heads->heads < 1) return fail(KD_E_INVALID, "kd_matmul_strided_heads: heads must be >= 1");
    if (sizes->batches > 0 && sizes->batches % heads->heads != 0)
        return fail(KD_E_INVALID, "kd_matmul_strided_heads: batches is not a multiple of heads");
    if (sizes->batches > (int64_t{1} << 31)) return fail(KD_E_INVALID, "kd_matmul_strided_heads: too many batches");
    MatmulArgs p;
    p.batches = sizes->batches;
    p.M = sizes->rows;
    p.K = sizes->inner;
    p.N = sizes->columns;
    p.sa = {strides->a[0], strides->a[1], strides->a[2]};
    p.sb = {strides->b[0], strides->b[1], strides->b[2]};
    p.so = {strides->out[0], strides->out[1], strides->out[2]};
    if (heads->heads > 1) {
        p.heads = heads->heads;
        p.ha = heads->a;
        p.hb = heads->b;
        p.ho = heads->out;
    }
    return dispatch(dtype, a, b, out, p);
}
