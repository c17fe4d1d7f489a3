// kd_gpt2.hip - GPT-2 decode engine (benchmark config C5) for gfx950.
//
// Workload of reference examples/gpt2_generate.cpp: kael's GPT (src/nn/transformer.cpp:103-237)
// generating with a KV cache (nn::generate, :256-295), greedily or with sample_next's temperature
// (with or without a top-k), batch 1, f32. kael runs it as ~700 device calls per token with blocking host syncs
// (embedding index checks, the pick on the host). This engine keeps kael's parameters in kael's
// layout and its arithmetic, and runs one token per replay of a captured HIP graph:
//
//   embed       x = wte[token] + wpe[pos]                                      (1 launch)
//   per layer   qkv GEMV on ln1(x) (+bias; K/V appended to the cache)
//               -> attention split into 8 key chunks per head (chunk max, double sum of
//                  exponentials, unnormalised weighted values)
//               -> proj GEMV on the combined attention output (+bias, +residual into x)
//               -> fc1 GEMV on ln2(x) (+bias, GELU)
//               -> fc2 GEMV (+bias, +residual into x)                          (5 launches)
//   head        ln_final -> logits = wte . h with per-workgroup best rows (and, sampling, the
//               keys of logits / temperature) -> the pick (the first maximum, or kael's
//               sample_next), which writes the next token and advances the position in device
//               memory                                                        (2 launches)
// The LayerNorm feeding a GEMV is recomputed by each of its workgroups into LDS (768 values):
// cheaper than a separate launch. A "last workgroup finishes" epilogue was measured and
// rejected: same-address device-scope atomics serialise at about 100 ns each on this part.
//
// The prompt goes through a batched prefill instead: all of its positions pass each layer
// together (GEMMs on the MFMA matmul path, per-row epilogues that also compute the next
// LayerNorm, a causal attention kernel), and the last position's logits and token come from the
// same head and pick kernels.
//
// All step-dependent values (position, token) live in device memory, so the graph is static.
// Weights keep kael's [out, in] row-major layout: every Linear is a row-dot GEMV reading whole
// rows with 16-byte loads (the decode step is HBM-bound on ~494 MB of weights per token).
// Rounding follows kael's op sequence: Linear rounds the product and then adds the bias;
// LayerNorm rounds the standardised value, then multiplies, then adds; attention scores are
// divided by sqrt(head_dim); softmax sums exponentials in double (src/ops/nn.cpp:60-71).
#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "kd_internal.h"
#include "../host/kd_safetensors.h"

namespace kd {

namespace {

constexpr int kThreads = 256;

struct Step {
    int64_t pos;     // position processed by the next step
    int64_t forced;  // positions < forced take their token from `seq` (teacher forcing)
};

// The pick's mode: greedy (top_k 0) or kael's sample_next with a temperature and a top-k
// (reference src/nn/transformer.cpp:39-50), one uniform draw per sampled token taken from
// `uniforms` in order. `error` is set when a pick finds a non-finite logit or no draw left.
struct Sampler {
    float temperature;  // kael's scalar in the logits' dtype
    int32_t error;
    int64_t top_k;
    int64_t draw;       // next draw
    int64_t draws;      // draws uploaded
};

// ---- kernels -------------------------------------------------------------------------------

// Whole-workgroup LayerNorm of x[0, d) into h, d <= 4 * kThreads: one read of x into registers,
// the sums of (x - c) and (x - c)^2 in double around the pivot c = x[0] (one pass; the shift
// keeps the variance free of cancellation) with a single workgroup reduction, then mean =
// c + S1/d and the population variance S2/d - (S1/d)^2; each element is standardised in double,
// rounded to float, then * w and + b, each rounded (reference src/ops/nn.cpp:114-129 then
// src/nn/layers.cpp:67).
// Split in two so that a kernel issues the row's loads (ln_load) before its weight loads and
// computes (ln_finish) after them: a wave waits for its loads in issue order, so a row loaded
// after the weights could only be used once the weights had arrived too (measured: 0.8 us per
// LayerNorm GEMV).
constexpr int64_t kMaxLnDim = 4 * kThreads;

// Cross-lane reductions with DPP (data-parallel primitives: lane permutations folded into the
// adding instruction) instead of LDS shuffles, whose latency a lone wave per SIMD cannot hide. Within
// each 16-lane row: quad butterflies (lanes i ^ 1, i ^ 2), then the mirrored lane of each 8-lane
// half and of the row, which after the quad steps holds the sum of the other quad / half. Every
// lane of the row ends with the row's sum.
template <int Ctrl> __device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), Ctrl, 0xf, 0xf, false));
}
template <int Ctrl> __device__ __forceinline__ double dpp_d(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b)), Ctrl, 0xf, 0xf, false));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b >> 32)), Ctrl, 0xf, 0xf, false));
    return __builtin_bit_cast(double, static_cast<uint64_t>(hi) << 32 | lo);
}
constexpr int kDppQuad1 = 0xb1, kDppQuad2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <typename T> __device__ __forceinline__ T dpp_move(T v, int step) {
    if constexpr (sizeof(T) == 8) {
        return step == 0 ? dpp_d<kDppQuad1>(v) : step == 1 ? dpp_d<kDppQuad2>(v) : step == 2 ? dpp_d<kDppHalfMirror>(v) : dpp_d<kDppMirror>(v);
    } else {
        return step == 0 ? dpp_f<kDppQuad1>(v) : step == 1 ? dpp_f<kDppQuad2>(v) : step == 2 ? dpp_f<kDppHalfMirror>(v) : dpp_f<kDppMirror>(v);
    }
}

template <typename T> __device__ __forceinline__ T row16_sum(T v) {
#pragma unroll
    for (int step = 0; step < 4; ++step) v += dpp_move(v, step);
    return v;
}

template <typename T> __device__ __forceinline__ T row16_max(T v) {
#pragma unroll
    for (int step = 0; step < 4; ++step) v = max_na(v, dpp_move(v, step));
    return v;
}

__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ double lane_value(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), lane));
    return __builtin_bit_cast(double, static_cast<uint64_t>(hi) << 32 | lo);
}

// The wave's sum (rows added in order 0..3), the same in every lane.
template <typename T> __device__ __forceinline__ T wave_sum(T v) {
    v = row16_sum(v);
    return ((lane_value(v, 0) + lane_value(v, 16)) + lane_value(v, 32)) + lane_value(v, 48);
}

template <typename T> __device__ __forceinline__ T wave_max(T v) {
    v = row16_max(v);
    return max_na(max_na(max_na(lane_value(v, 0), lane_value(v, 16)), lane_value(v, 32)), lane_value(v, 48));
}

struct LnIn {
    float x[4], w[4], b[4];
    float c;  // the pivot x[0]
};

__device__ __forceinline__ LnIn ln_load(const float* x, int64_t d, const float* w, const float* b) {
    LnIn r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        r.x[j] = i < d ? x[i] : 0.f;
        r.w[j] = i < d ? w[i] : 0.f;
        r.b[j] = i < d ? b[i] : 0.f;
    }
    r.c = x[0];
    return r;
}

__device__ __forceinline__ void ln_finish(const LnIn& r, int64_t d, float* h) {
    __shared__ double sums[2][kThreads / 64];
    const double c = r.c;
    double s1 = 0.0, s2 = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (threadIdx.x + j * kThreads < d) {
            const double t = static_cast<double>(r.x[j]) - c;
            s1 += t;
            s2 += t * t;
        }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const int wave = threadIdx.x / 64;
    if (threadIdx.x % 64 == 0) {
        sums[0][wave] = s1;
        sums[1][wave] = s2;
    }
    __syncthreads();
    s1 = sums[0][0];
    s2 = sums[1][0];
    for (int v = 1; v < kThreads / 64; ++v) {
        s1 += sums[0][v];
        s2 += sums[1][v];
    }
    const double m1 = s1 / static_cast<double>(d);
    const double mean = c + m1;
    const double scale = std::sqrt(s2 / static_cast<double>(d) - m1 * m1 + 1e-5);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        if (i < d) {
            const float y = static_cast<float>((static_cast<double>(r.x[j]) - mean) / scale);
            h[i] = add_sep(mul_sep(y, r.w[j]), r.b[j]);  // two roundings, as kael's * w and + b
        }
    }
}

// x = wte[token] + wpe[pos].
__global__ __launch_bounds__(kThreads) void embed_kernel(const Step* st, const int64_t* seq, const float* wte,
                                                         const float* wpe, float* x, int64_t d) {
    const int64_t pos = st->pos;
    const int64_t tok = seq[pos];
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < d; i += static_cast<int64_t>(gridDim.x) * kThreads)
        x[i] = __fadd_rn(wte[tok * d + i], wpe[pos * d + i]);
}

enum Epilogue { kStore = 0, kGeluTanh = 1, kGeluExact = 2, kResidual = 3, kQkv = 4 };

struct Best {
    float v;
    int64_t i;
};

// `a` wins over `b` if it is NaN-first, larger, or equal with a smaller index: the first
// maximum, with the first NaN winning (reference best_position, src/ops/reduce.cpp:236-254).
__device__ __forceinline__ bool better(const Best& a, const Best& b) {
    const bool an = isnan(a.v), bn = isnan(b.v);
    if (an || bn) return an && (!bn || a.i < b.i);
    return a.v > b.v || (a.v == b.v && a.i < b.i);
}

__device__ __forceinline__ Best wave_best(Best v) {
#pragma unroll
    for (int m = 32; m > 0; m /= 2) {
        Best o{__shfl_xor(v.v, m, 64), __shfl_xor(v.i, m, 64)};
        if (better(o, v)) v = o;
    }
    return v;
}

constexpr int kAttnChunks = 8;
constexpr int kAttnRegs = 8;  // keys per 16-lane group whose rows attention_kernel holds in registers

struct AttnPartials {
    float* m;      // [heads][chunks]
    double* l;     // [heads][chunks]
    float* acc;    // [heads][chunks][head_dim]
};

// Attention output of every head into h[0, heads * head_dim) from the chunk partials: with M the
// maximum over a head's non-empty chunks (an empty chunk reports m = -inf, l = 0),
// out = sum_c exp(m_c - M) acc_c / float(sum_c exp(m_c - M) l_c), the denominator being the
// float rounding of a double sum as in reference src/ops/nn.cpp:60-71. attn_load issues every
// load (this thread's chunk outputs, the chunk maxima, and thread hd's chunk sums for head
// hd < heads) and attn_finish computes: the split lets a kernel issue its weight loads between
// the two (see ln_load).
constexpr int kMaxHeads = 64;
constexpr int kAttnPer = kMaxLnDim / kThreads;                  // output elements per thread
constexpr int kAttnSlots = kMaxHeads * kAttnChunks / kThreads;  // chunk maxima per thread

struct AttnIn {
    float acc[kAttnPer][kAttnChunks];
    float m[kAttnSlots];
    double l[kAttnChunks];
};

__device__ __forceinline__ void attn_load(const AttnPartials& p, int64_t heads, int64_t head_dim, AttnIn& r) {
#pragma unroll
    for (int q = 0; q < kAttnPer; ++q) {
        const int64_t k = threadIdx.x + q * kThreads;
        const int64_t hd = k / head_dim;
        const int64_t e = k - hd * head_dim;
#pragma unroll
        for (int c = 0; c < kAttnChunks; ++c)
            r.acc[q][c] = k < heads * head_dim ? p.acc[(hd * kAttnChunks + c) * head_dim + e] : 0.f;
    }
    const int64_t slots = heads * kAttnChunks;
#pragma unroll
    for (int j = 0; j < kAttnSlots; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        r.m[j] = i < slots ? p.m[i] : 0.f;
    }
    if (threadIdx.x < heads) {
#pragma unroll
        for (int c = 0; c < kAttnChunks; ++c) r.l[c] = p.l[threadIdx.x * kAttnChunks + c];
    }
}

__device__ void attn_finish(const AttnIn& r, int64_t heads, int64_t head_dim, float* h) {
    __shared__ float factor[kMaxHeads * kAttnChunks];
    __shared__ float denom[kMaxHeads];
    const int64_t slots = heads * kAttnChunks;
#pragma unroll
    for (int j = 0; j < kAttnSlots; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        if (i < slots) factor[i] = r.m[j];
    }
    __syncthreads();
    if (threadIdx.x < heads) {  // heads <= kMaxHeads <= kThreads
        const int64_t hd = threadIdx.x;
        float M = -INFINITY;
        bool any = false;
        double lsum = 0.0;
        float w[kAttnChunks];
#pragma unroll
        for (int c = 0; c < kAttnChunks; ++c) {
            const float m = factor[hd * kAttnChunks + c];
            if (!(m == -INFINITY && r.l[c] == 0.0)) {
                M = any ? max_na(M, m) : m;
                any = true;
            }
        }
#pragma unroll
        for (int c = 0; c < kAttnChunks; ++c) {
            const float m = factor[hd * kAttnChunks + c];
            const bool empty = m == -INFINITY && r.l[c] == 0.0;
            w[c] = empty ? 0.f : std::exp(__fsub_rn(m, M));
            if (!empty) lsum += static_cast<double>(w[c]) * r.l[c];
        }
#pragma unroll
        for (int c = 0; c < kAttnChunks; ++c) factor[hd * kAttnChunks + c] = w[c];
        denom[hd] = static_cast<float>(lsum);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kAttnPer; ++q) {
        const int64_t k = threadIdx.x + q * kThreads;
        if (k < heads * head_dim) {
            const int64_t hd = k / head_dim;
            float num = 0.f;
#pragma unroll
            for (int c = 0; c < kAttnChunks; ++c) num += factor[hd * kAttnChunks + c] * r.acc[q][c];
            h[k] = __fdiv_rn(num, denom[hd]);
        }
    }
}

struct GemvArgs {
    const float* W;        // [N, K] row-major
    const float* x;        // input vector [K]
    const float* bias;     // [N] or nullptr
    float* out;            // [N]
    int64_t N, K;
    // With the kLn prologue the input is LayerNorm(x) with this weight and bias, computed by
    // every workgroup into LDS (a 768-vector: cheaper than a separate launch).
    const float* ln_w;
    const float* ln_b;
    // With the kAttn prologue the input is the attention output combined from these chunk partials.
    AttnPartials attn;
    // kQkv: query -> q, key/value rows appended to this layer's cache at the current position
    float* q;
    float* kcache;
    float* vcache;
    int64_t d, head_dim, max_positions;
    // head_kernel: per-workgroup argmax partials (pick_kernel picks the winner)
    float* best_v;
    int64_t* best_i;
    Step* st;
    // head_kernel when the sampler samples (top_k > 0): every row's order key of logit / temperature,
    // and each workgroup's largest and smallest key (key_parts[2g], key_parts[2g + 1])
    const Sampler* sp;
    uint32_t* keys;
    uint32_t* key_parts;
};

constexpr int kMaxK = 4096;

// kael's GELU forms (reference src/internal/element_functions.h:278-288) on a Linear output.
template <int Epi> __device__ __forceinline__ float gelu_of(float y) {
    if constexpr (Epi == kGeluTanh) {
        const float scale = std::sqrt(2 / MathConst<float>::pi);
        return 0.5f * y * (1 + std::tanh(scale * (y + 0.044715f * y * y * y)));
    } else {
        return 0.5f * y * (1 + std::erf(y / MathConst<float>::sqrt2));
    }
}

// Input prologues of gemv_kernel: the input vector as is, LayerNorm(x), or the attention output
// combined from chunk partials.
enum Prologue { kPlain = 0, kLn = 1, kAttn = 2 };

// out[n] = epilogue(W[n, :] . x) for the rows of this workgroup. The input vector is staged in
// LDS. Rows: WavesPerRow == 1 -> each wave owns 2 rows (8 rows per workgroup); WavesPerRow == 4
// -> the workgroup owns 2 rows and each wave a quarter of K, combined through LDS.
// Load order: the prologue's inputs first, then this lane's weights, then the epilogue's
// operands; the prologue's arithmetic runs while the weights are in flight.
template <int Epi, int WavesPerRow, int Pro>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    __shared__ float4 hs4[kMaxK / 4];
    __shared__ float part[4][2];
    float* hs = reinterpret_cast<float*>(hs4);
    const int64_t K = a.K;
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    constexpr int rows_per_block = WavesPerRow == 1 ? 8 : 2;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * rows_per_block + (WavesPerRow == 1 ? 2 * wave : 0);
    const int64_t k4 = K / 4;
    const int64_t kb = WavesPerRow == 1 ? 0 : (k4 * wave) / 4;
    const int64_t ke = WavesPerRow == 1 ? k4 : (k4 * (wave + 1)) / 4;
    const bool has0 = n0 < a.N;
    const bool has1 = n0 + 1 < a.N;
    [[maybe_unused]] LnIn ln;
    [[maybe_unused]] AttnIn attn;
    [[maybe_unused]] float xr[kMaxK / kThreads];
    if constexpr (Pro == kLn) {
        ln = ln_load(a.x, K, a.ln_w, a.ln_b);
    } else if constexpr (Pro == kAttn) {
        attn_load(a.attn, K / a.head_dim, a.head_dim, attn);
    } else {
#pragma unroll
        for (int j = 0; j < kMaxK / kThreads; ++j) {
            const int64_t k = threadIdx.x + j * kThreads;
            xr[j] = k < K ? a.x[k] : 0.f;
        }
    }
    const float4* w0 = reinterpret_cast<const float4*>(a.W + (has0 ? n0 : 0) * K);
    const float4* w1 = reinterpret_cast<const float4*>(a.W + (has1 ? n0 + 1 : (has0 ? n0 : 0)) * K);
    // This lane's first weight loads, in flight during the prologue. A LayerNorm input has
    // K = d <= 1024, so with K split over 4 waves one float4 per row covers a wave's range:
    // the registers this frees hold the LayerNorm row.
    constexpr int kPrefetch = Pro == kLn && WavesPerRow == 4 ? 1 : 4;
    float4 pw0[kPrefetch], pw1[kPrefetch];
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) {
        const int64_t k = kb + lane + 64 * i;
        if (has0 && k < ke) {
            pw0[i] = w0[k];
            pw1[i] = w1[k];
        }
    }
    // Operands of the epilogue, loaded now so that their latency overlaps the prologue and the
    // dot products instead of following them.
    const bool owner = WavesPerRow == 1 || wave == 0;
    const bool active = owner && lane < 2 && (lane == 0 ? has0 : has1);
    const int64_t n = n0 + lane;
    float bias = 0.f, resid = 0.f;
    if (active) {
        bias = a.bias[n];
        if constexpr (Epi == kResidual) resid = a.out[n];
    }
    const int64_t pos = Epi == kQkv ? a.st->pos : 0;
    if constexpr (Pro == kLn) {
        ln_finish(ln, K, hs);
    } else if constexpr (Pro == kAttn) {
        attn_finish(attn, K / a.head_dim, a.head_dim, hs);
    } else {
#pragma unroll
        for (int j = 0; j < kMaxK / kThreads; ++j) {
            const int64_t k = threadIdx.x + j * kThreads;
            if (k < K) hs[k] = xr[j];
        }
    }
    __syncthreads();

    float a0 = 0.f, a1 = 0.f;
    if (has0) {
#pragma unroll
        for (int i = 0; i < kPrefetch; ++i) {
            const int64_t k = kb + lane + 64 * i;
            if (k < ke) {
                const float4 xx = hs4[k];
                a0 += pw0[i].x * xx.x + pw0[i].y * xx.y + pw0[i].z * xx.z + pw0[i].w * xx.w;
                a1 += pw1[i].x * xx.x + pw1[i].y * xx.y + pw1[i].z * xx.z + pw1[i].w * xx.w;
            }
        }
        for (int64_t k = kb + lane + 64 * kPrefetch; k < ke; k += 64) {
            const float4 xx = hs4[k];
            const float4 p = w0[k];
            const float4 r = w1[k];
            a0 += p.x * xx.x + p.y * xx.y + p.z * xx.z + p.w * xx.w;
            a1 += r.x * xx.x + r.y * xx.y + r.z * xx.z + r.w * xx.w;
        }
    }
    a0 = wave_sum(a0);
    a1 = wave_sum(a1);
    if constexpr (WavesPerRow == 4) {
        if (lane == 0) {
            part[wave][0] = a0;
            part[wave][1] = a1;
        }
        __syncthreads();
        a0 = ((part[0][0] + part[1][0]) + part[2][0]) + part[3][0];
        a1 = ((part[0][1] + part[1][1]) + part[2][1]) + part[3][1];
    }
    // lanes 0 and 1 of the owning wave finish rows n0 and n0 + 1
    float y = 0.f;
    if (active) {
        const float dot = lane == 0 ? a0 : a1;
        y = __fadd_rn(dot, bias);
        if constexpr (Epi == kGeluTanh || Epi == kGeluExact) {
            y = gelu_of<Epi>(y);
        } else if constexpr (Epi == kResidual) {
            y = __fadd_rn(resid, y);
        }
        if constexpr (Epi == kQkv) {
            const int64_t part_id = n / a.d;
            const int64_t within = n - part_id * a.d;
            if (part_id == 0) {
                a.q[within] = y;
            } else {
                const int64_t head = within / a.head_dim;
                const int64_t dim = within - head * a.head_dim;
                float* cache = part_id == 1 ? a.kcache : a.vcache;
                cache[(head * a.max_positions + pos) * a.head_dim + dim] = y;
            }
        } else {
            a.out[n] = y;
        }
    }
}

// Logits of the tied head, logits[n] = wte[n, :] . LayerNorm_f(x), and each workgroup's best
// row (first maximum, first NaN; reference src/ops/reduce.cpp:236-254) for pick_kernel.
// A fixed grid of 4 workgroups per CU (its occupancy at 108 VGPRs) streams the [vocab, d] table:
// each wave takes row pairs p, p + stride, ... and issues the next pair's loads before the
// current pair's dot products, so every wave keeps two pairs in flight. The final LayerNorm is
// computed once per workgroup into LDS and then held in registers (one launch fewer than a
// separate LayerNorm, and one argmax partial per workgroup: 1024 instead of one per 8 rows).
// Needs d <= kMaxLnDim (4 float4 per lane). Registers sized to d = 768 (5 workgroups per CU)
// measured no faster (27.4 µs against 27.1).
constexpr int kHeadVec = kMaxLnDim / 256;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte load with the nontemporal hint (the table is read once per token).
// Loads through pointers that the compiler cannot prove global (read from memory, such as the
// per-layer parameter table) are flat loads, which a wave waits for together with its LDS reads.
// These name the global address space, so that a weight prefetch never delays an LDS read.
typedef __attribute__((address_space(1))) const f32x4 global_f32x4;
typedef __attribute__((address_space(1))) const float global_f32;
typedef __attribute__((address_space(1))) float global_f32_out;

// Order-preserving keys of floats for the sampled pick: unsigned order of the keys is the order of
// the floats (-0 and +0 share +0's key, as they compare equal); the finite floats' keys lie in
// [kFiniteKeyLow, kFiniteKeyHigh], the infinities' and NaNs' outside.
__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t b = x == 0.f ? 0u : __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

constexpr uint32_t kFiniteKeyLow = 0x00800000u;   // key of -FLT_MAX
constexpr uint32_t kFiniteKeyHigh = 0xff7fffffu;  // key of FLT_MAX

__device__ __forceinline__ float4 nt_load4(const float4* p) {
    const f32x4 v = __builtin_nontemporal_load((global_f32x4*)(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float4 gload4(const float4* p) {
    const f32x4 v = *(global_f32x4*)(p);
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float gload(const float* p) { return *(global_f32*)(p); }

__device__ __forceinline__ void gstore(float* p, float v) { *(global_f32_out*)(p) = v; }


__global__ __launch_bounds__(kThreads) void head_kernel(GemvArgs a) {
    __shared__ float4 hs4[kMaxLnDim / 4];
    __shared__ float bv[kThreads / 64];
    __shared__ int64_t bi[kThreads / 64];
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    const int64_t N = a.N;
    const int64_t k4 = a.K / 4;
    const int64_t pairs = (N + 1) / 2;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * (kThreads / 64);
    const float4* W4 = reinterpret_cast<const float4*>(a.W);
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    const auto load = [&](int64_t pair, float4 (&r0)[kHeadVec], float4 (&r1)[kHeadVec]) {
        const int64_t n = 2 * pair;
        const bool second = n + 1 < N;
#pragma unroll
        for (int i = 0; i < kHeadVec; ++i) {
            const int64_t j = lane + 64 * i;
            r0[i] = j < k4 ? nt_load4(W4 + n * k4 + j) : zero;
            r1[i] = j < k4 && second ? nt_load4(W4 + (n + 1) * k4 + j) : zero;
        }
    };
    int64_t p = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave;
    const bool keyed = a.sp != nullptr && a.sp->top_k > 0;
    const float temperature = keyed ? a.sp->temperature : 1.f;
    const LnIn ln = ln_load(a.x, a.K, a.ln_w, a.ln_b);
    float4 c0[kHeadVec], c1[kHeadVec];
    if (p < pairs) load(p, c0, c1);
    ln_finish(ln, a.K, reinterpret_cast<float*>(hs4));
    __syncthreads();
    float4 h[kHeadVec];
#pragma unroll
    for (int i = 0; i < kHeadVec; ++i) {
        const int64_t j = lane + 64 * i;
        h[i] = j < k4 ? hs4[j] : zero;
    }
    Best best{-INFINITY, INT64_MAX};
    uint32_t key_hi = 0, key_lo = ~0u;  // sampled: the largest and smallest key this lane writes
    for (; p < pairs; p += stride) {
        float4 n0[kHeadVec], n1[kHeadVec];
        if (p + stride < pairs) load(p + stride, n0, n1);
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int i = 0; i < kHeadVec; ++i) {
            a0 += c0[i].x * h[i].x + c0[i].y * h[i].y + c0[i].z * h[i].z + c0[i].w * h[i].w;
            a1 += c1[i].x * h[i].x + c1[i].y * h[i].y + c1[i].z * h[i].z + c1[i].w * h[i].w;
        }
        a0 = wave_sum(a0);
        a1 = wave_sum(a1);
        const int64_t n = 2 * p;
        if (lane == 0) a.out[n] = a0;
        if (lane == 1 && n + 1 < N) a.out[n + 1] = a1;
        if (keyed) {  // x = logits / temperature as kael's sample_next divides (f32)
            const bool writes = lane == 0 || (lane == 1 && n + 1 < N);
            if (writes) {
                const uint32_t k = order_key(__fdiv_rn(lane == 0 ? a0 : a1, temperature));
                a.keys[n + lane] = k;
                key_hi = max(key_hi, k);
                key_lo = min(key_lo, k);
            }
        }
        const Best o0{a0, n};
        if (better(o0, best)) best = o0;
        if (n + 1 < N) {
            const Best o1{a1, n + 1};
            if (better(o1, best)) best = o1;
        }
#pragma unroll
        for (int i = 0; i < kHeadVec; ++i) {
            c0[i] = n0[i];
            c1[i] = n1[i];
        }
    }
    __shared__ uint32_t khi[kThreads / 64][2], klo[kThreads / 64][2];
    if (lane == 0) {
        bv[wave] = best.v;
        bi[wave] = best.i;
    }
    if (keyed && lane < 2) {
        khi[wave][lane] = key_hi;
        klo[wave][lane] = key_lo;
    }
    __syncthreads();
    if (keyed && threadIdx.x == 0) {  // the workgroup's key extremes, for the sampled pick's bound
        uint32_t hi = 0, lo = ~0u;
        for (int w = 0; w < kThreads / 64; ++w)
            for (int l = 0; l < 2; ++l) {
                hi = max(hi, khi[w][l]);
                lo = min(lo, klo[w][l]);
            }
        a.key_parts[2 * blockIdx.x] = hi;
        a.key_parts[2 * blockIdx.x + 1] = lo;
    }
    if (threadIdx.x == 0) {
        Best r{bv[0], bi[0]};
        for (int w = 1; w < kThreads / 64; ++w) {
            const Best o{bv[w], bi[w]};
            if (better(o, r)) r = o;
        }
        a.best_v[blockIdx.x] = r.v;
        a.best_i[blockIdx.x] = r.i;
    }
}

// Picks the next token, appends it to the sequence unless the next position is teacher-forced,
// and advances the position. One workgroup of 1024 lanes.
//   Greedy (sampler top_k 0): the first maximum among the head's workgroup partials (one per
//   head workgroup: 1024 for GPT-2 small).
//   Sampled: kael's sample_next (reference src/nn/transformer.cpp:39-50) and multinomial
//   (src/random.cpp:106-160): x = logits / temperature (f32 division, in head_kernel, which
//   writes x's order-preserving 32-bit keys and each workgroup's extremes); a lower bound of the
//   k-th largest key from the k-th largest head-workgroup maximum (or, in the full scan, lane
//   maximum), the keys at or above it (about k) listed, the k-th largest among them by rank
//   counting or radix selects (8-bit digits, per-wave histograms); for k > 1024 a radix select
//   over every key; without a top-k (k = vocab, kael's masking skipped) every entry. The kept entries (x >= the k-th largest: masked_fill's
//   complement) are listed in index order with their e = exp(x - max); then, in kael's order, the
//   sum of e in double rounded to f32, p = e / sum, the cumulative double sum of p, point = u *
//   sum, the first kept entry whose cumulative sum exceeds the point (upper_bound; the masked
//   entries add zeros, which leave every partial sum unchanged), or else the last kept entry with
//   p > 0.
constexpr int kPickThreads = 1024;
constexpr int kPickWaves = kPickThreads / 64;
constexpr int kPickSlots = 64;         // keys per lane: sampled vocabularies up to 65536
constexpr int kPickLdsKept = 4096;     // listed entries staged in LDS; more kept go to the global scratch
static_assert(int64_t{kPickThreads} * kPickSlots == KD_GPT_SAMPLE_MAX_VOCAB);
static_assert(kPickLdsKept % kPickThreads == 0 && kPickLdsKept / kPickThreads <= kPickSlots);
constexpr int32_t kRawBufferWord3 = 0x00020000;  // buffer descriptor word 3: 32-bit data format
constexpr int64_t kRankList = 256;  // candidate lists up to this long: k-th key by rank counting
constexpr int kPickParts = 256;     // head workgroups whose rows the pick reads, at most

struct PickArgs {
    Step* st;
    int64_t* seq;
    const float* pv;
    const int64_t* pi;
    int64_t parts;
    const float* logits;
    int64_t vocab;
    Sampler* sp;
    const double* uniforms;
    int32_t* kept;   // [vocab] scratch: kept indices in index order, when more than kPickLdsKept
    float* kept_e;   // [vocab] scratch: their exponentials
    const uint32_t* keys;  // [kPickSlots * kPickThreads] head_kernel's order keys of x = logits /
                           // temperature, zero past the vocabulary
    const uint32_t* key_parts;  // [2 * parts] each head workgroup's largest and smallest key
};

struct alignas(16) PickShared {  // hist rows are read 16 bytes at a time
    uint32_t hist[kPickWaves][256];
    uint32_t counts[kPickSlots * kPickWaves];  // per (item group, wave), then their offsets
    uint32_t wave_items[kPickWaves][2];       // per wave: the item groups any lane keeps
    int64_t wave_totals[kPickWaves];
    uint32_t wave_totals32[kPickWaves];
    uint32_t wmax[kPickWaves];
    uint32_t wmin[kPickWaves];
    uint32_t chosen;
    int64_t remaining;
    int64_t total;
    alignas(16) uint32_t cand_key[kPickLdsKept + 4];  // listed keys >= the lower bound, zeros after them
    alignas(16) int32_t cand_idx[kPickLdsKept + 4];   // their indices
    uint32_t appended;                                // keys appended to the unordered short list
    uint32_t nparts;                                  // head workgroups that may hold candidates
    int32_t cand_parts[kPickParts];
    float kept_e[kPickLdsKept];       // kept entries, when at most kPickLdsKept
    int32_t kept_i[kPickLdsKept];
};

// Inclusive prefix sum of v over the workgroup's first `n` lanes (n a multiple of 64, at most
// kPickThreads); every thread of the workgroup must call it.
__device__ __forceinline__ int64_t block_inclusive_scan(int64_t v, int n, int64_t* wave_totals) {
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t o = __shfl_up(v, off);
        if (lane >= off) v += o;
    }
    if (lane == 63 && tid < n) wave_totals[wave] = v;
    __syncthreads();
    int64_t before = 0;
    for (int w = 0; w < wave && w < n / 64; ++w) before += wave_totals[w];
    __syncthreads();
    return v + before;
}

// Inclusive prefix sum of 32-bit v over the whole workgroup (sums below 2^32); every thread of
// the workgroup must call it.
__device__ __forceinline__ uint32_t block_inclusive_scan32(uint32_t v, uint32_t* wave_totals) {
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(v), off));
        if (lane >= off) v += o;
    }
    if (lane == 63) wave_totals[wave] = v;
    __syncthreads();
    uint32_t before = 0;
    for (int w = 0; w < wave; ++w) before += wave_totals[w];
    __syncthreads();
    return v + before;
}

// Adds 1 to hist[bin] for every active lane. Most logits share their top key bits, and lane-by-lane
// LDS atomics on one address serialise, so the first few distinct bins among the wave's lanes take
// one atomic each (the bin read from the leading lane with readlane); the lanes left, whose bins
// are then spread, add their own.
__device__ __forceinline__ void wave_histogram_add(uint32_t* hist, uint32_t bin, bool active) {
    uint64_t pending = __ballot(active);
    const int lane = threadIdx.x % 64;
    for (int round = 0; round < 4 && pending != 0; ++round) {
        const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
        const uint32_t leader_bin = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bin), leader));
        const uint64_t same = __ballot(active && bin == leader_bin) & pending;
        if (lane == leader) atomicAdd(&hist[leader_bin], static_cast<uint32_t>(__popcll(same)));
        pending &= ~same;
    }
    if ((pending >> lane) & 1) atomicAdd(&hist[bin], 1u);
}

// The rank-th largest (1-based) of the keys the lanes offer: visit(f) calls f(key, counted) for
// each of the lane's keys, equally often in every lane of a wave (with fewer than four digits, its
// top 8 * digits bits and zeros below: a lower bound). 8-bit digits from the top
// with per-wave histograms; wave 0 finds each digit (lane l sums bins 255 - 4l .. 252 - 4l over the
// waves, a scan over the lanes finds the bin where the count from the top reaches the remaining
// rank). Every thread of the workgroup calls it; rank must not exceed the number of counted keys.
template <class Visit>
__device__ __forceinline__ uint32_t radix_select(const Visit& visit, int64_t rank, PickShared& sh, int digits = 4) {
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    if (tid == 0) sh.remaining = rank;
    uint32_t prefix = 0, mask = 0;
#pragma unroll 1
    for (int shift = 24; shift >= 32 - 8 * digits; shift -= 8) {
        for (int b = lane; b < 256; b += 64) sh.hist[wave][b] = 0;
        __syncthreads();
        visit([&](uint32_t key, bool counted) {
            wave_histogram_add(sh.hist[wave], (key >> shift) & 255u, counted && (key & mask) == prefix);
        });
        __syncthreads();
        if (wave == 0) {
            uint4 c = make_uint4(0, 0, 0, 0);  // .w: bin 255 - 4l, .z, .y, .x: the next three down
            for (int w = 0; w < kPickWaves; ++w) {
                const uint4 h = *reinterpret_cast<const uint4*>(&sh.hist[w][252 - 4 * lane]);
                c.x += h.x;
                c.y += h.y;
                c.z += h.z;
                c.w += h.w;
            }
            const uint32_t mine = c.x + c.y + c.z + c.w;
            uint32_t through = mine;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(through), off));
                if (lane >= off) through += o;
            }
            const int64_t need = sh.remaining;
            const int64_t before = through - mine;
            if (before < need && through >= need) {
                const uint32_t bins[4] = {c.w, c.z, c.y, c.x};
                int64_t run = before;
                int q = 0;
                while (q < 3 && run + bins[q] < need) run += bins[q++];
                sh.chosen = static_cast<uint32_t>(255 - 4 * lane - q);
                sh.remaining = need - run;
            }
        }
        __syncthreads();
        prefix |= sh.chosen << shift;
        mask |= 0xffu << shift;
    }
    return prefix;
}

// Lists the lane's items j (item j of lane t stands for j * kPickThreads + t) whose bit j of
// `mine` is set, in item order, which is (j, wave, lane) order: a count per (j, wave) over the
// items any lane of the wave keeps, an exclusive scan of the counts, then each wave's items in
// lane order, emit(j, position, total) writing one. Returns the total; every thread of the
// workgroup calls it.
template <class Emit>
__device__ __forceinline__ int64_t ordered_compact(uint64_t mine, const Emit& emit, PickShared& sh) {
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    static_assert(kPickSlots * kPickWaves == kPickThreads);
    sh.counts[tid] = 0;
    if (lane == 0) sh.wave_items[wave][0] = sh.wave_items[wave][1] = 0;
    __syncthreads();
    if (mine != 0) {  // the wave's union of items: LDS ORs from the (usually few) lanes that keep some
        atomicOr(&sh.wave_items[wave][0], static_cast<uint32_t>(mine));
        atomicOr(&sh.wave_items[wave][1], static_cast<uint32_t>(mine >> 32));
    }
    __syncthreads();
    const uint64_t wave_items = (uint64_t{sh.wave_items[wave][1]} << 32) | sh.wave_items[wave][0];
    for (uint64_t rest = wave_items; rest != 0; rest &= rest - 1) {
        const int j = __ffsll(static_cast<unsigned long long>(rest)) - 1;
        const uint64_t lanes = __ballot((mine >> j) & 1);
        if (lane == 0) sh.counts[j * kPickWaves + wave] = static_cast<uint32_t>(__popcll(lanes));
    }
    __syncthreads();
    const uint32_t c = sh.counts[tid];
    const uint32_t through = block_inclusive_scan32(c, sh.wave_totals32);
    sh.counts[tid] = through - c;
    if (tid == kPickThreads - 1) sh.total = through;
    __syncthreads();
    const int64_t total = sh.total;
    const uint64_t below = (uint64_t{1} << lane) - 1;
    for (uint64_t rest = wave_items; rest != 0; rest &= rest - 1) {
        const int j = __ffsll(static_cast<unsigned long long>(rest)) - 1;
        const bool k = (mine >> j) & 1;
        const uint64_t lanes = __ballot(k);
        if (k) emit(j, sh.counts[j * kPickWaves + wave] + __popcll(lanes & below), total);
    }
    __syncthreads();
    return total;
}

__device__ __forceinline__ void sample_pick(const PickArgs& a, int64_t& token) {
    __shared__ PickShared sh;
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int64_t V = a.vocab;
    const int64_t top_k = a.sp->top_k;
    // this pick's draw, read now so that its loads overlap the selection
    const int64_t draw = a.sp->draw, draws = a.sp->draws;
    const double u = draw < draws ? a.uniforms[draw] : 0.0;
    // The keys, slot s of lane t holding index s * 1024 + t; the buffer holds all 64 slots with
    // zeros past the vocabulary (below every finite x's key), so the loads need no branches and
    // all go out at once. Buffer loads: one lane offset and a scalar offset per slot, where 64
    // global addresses would take 128 registers.
    const __amdgpu_buffer_rsrc_t keys_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.keys), 0,
                                          int32_t{kPickSlots * kPickThreads * sizeof(uint32_t)}, kRawBufferWord3);
    const auto key_at = [&](int s) -> uint32_t {
        return __builtin_amdgcn_raw_buffer_load_b32(keys_rsrc, tid * 4, s * kPickThreads * 4, 0);
    };
    const bool bounded = top_k <= kPickThreads;
    uint32_t kmax = 0, kmin = ~0u, low = 1;
    uint64_t above = 0;  // (the full scan) bit s: slot s's key is at or above the bound
    bool unordered = false, listed = false;
    int64_t listed_n = 0;
    // From the head kernel's workgroup extremes (for k at most the number of its workgroups): the
    // k-th largest workgroup maximum bounds the k-th largest key from below (k workgroups hold a
    // key at least that large), and only the workgroups whose maximum reaches the bound can hold a
    // key at or above it, so only their rows are read (head workgroup g wrote the rows of row
    // pairs g * 4 + w + j * 4 * parts, w < 4). Too many such workgroups or keys: the full scan.
    const int64_t parts = a.parts;
    bool from_parts = top_k <= parts && parts <= kPickThreads;
    if (from_parts) {
        const bool mine = tid < parts;
        const uint32_t phi = mine ? a.key_parts[2 * tid] : 0u;
        const uint32_t plo = mine ? a.key_parts[2 * tid + 1] : ~0u;
        uint32_t wm = phi, wn = plo;
        for (int off = 32; off > 0; off >>= 1) {
            wm = max(wm, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wm), off)));
            wn = min(wn, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wn), off)));
        }
        if (lane == 0) {
            sh.wmax[wave] = wm;
            sh.wmin[wave] = wn;
        }
        if (tid == 0) {
            sh.appended = 0;
            sh.nparts = 0;
        }
        __syncthreads();
        kmax = sh.wmax[0];
        kmin = sh.wmin[0];
        for (int w = 1; w < kPickWaves; ++w) {
            kmax = max(kmax, sh.wmax[w]);
            kmin = min(kmin, sh.wmin[w]);
        }
        kmax = __builtin_amdgcn_readfirstlane(kmax);
        kmin = __builtin_amdgcn_readfirstlane(kmin);
        low = max(1u, radix_select([&](const auto& f) { f(phi, mine); }, top_k, sh, 2));
        if (mine && phi >= low) {
            const uint32_t at = atomicAdd(&sh.nparts, 1u);
            if (at < kPickParts) sh.cand_parts[at] = tid;
        }
        __syncthreads();
        const uint32_t np = __builtin_amdgcn_readfirstlane(sh.nparts);
        if (np <= kPickParts) {
            const int64_t pairs = (V + 1) / 2, stride = parts * (kThreads / 64);
            const int64_t per_part = 2 * (kThreads / 64) * ((pairs + stride - 1) / stride);  // rows, at most
            const int64_t items = int64_t{np} * per_part;
            for (int64_t base = 0; base < items; base += 4 * kPickThreads) {
                uint32_t k[4];
                int64_t n[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {  // four rows' keys in flight
                    const int64_t i = base + q * kPickThreads + tid;
                    n[q] = -1;
                    k[q] = 0;
                    if (i < items) {
                        const int64_t g = sh.cand_parts[i / per_part], r = i % per_part;
                        const int64_t pair = g * (kThreads / 64) + (r / 2) % (kThreads / 64) + r / (2 * (kThreads / 64)) * stride;
                        const int64_t row = 2 * pair + r % 2;
                        if (pair < pairs && row < V) {
                            n[q] = row;
                            k[q] = a.keys[row];
                        }
                    }
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (n[q] >= 0 && k[q] >= low) {
                        const uint32_t at = atomicAdd(&sh.appended, 1u);
                        if (at < kRankList) {
                            sh.cand_key[at] = k[q];
                            sh.cand_idx[at] = static_cast<int32_t>(n[q]);
                        }
                    }
                }
            }
            __syncthreads();
            const uint32_t appended = __builtin_amdgcn_readfirstlane(sh.appended);
            if (appended <= kRankList) {
                unordered = listed = true;
                listed_n = appended;
            }
        }
        from_parts = unordered;
    }
    if (!from_parts) {  // the full scan
        uint32_t key[kPickSlots];
#pragma unroll
        for (int s = 0; s < kPickSlots; ++s) key[s] = key_at(s);
        // the lane's largest key; the smallest over the vocabulary; the keys' top 16 bits, two slots a
        // register (all the bound's test needs below: its low 16 bits are zero)
        uint32_t tmax = 0, tmin = ~0u;
        uint32_t top16[kPickSlots / 2];
#pragma unroll
        for (int s = 0; s < kPickSlots; ++s) {
            tmax = max(tmax, key[s]);
            tmin = min(tmin, int64_t{s} * kPickThreads + tid < V ? key[s] : ~0u);
            if (s % 2 == 0) top16[s / 2] = key[s] >> 16;
            else top16[s / 2] |= key[s] & 0xffff0000u;
        }
        uint32_t wm = tmax, wn = tmin;
        for (int off = 32; off > 0; off >>= 1) {
            wm = max(wm, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wm), off)));
            wn = min(wn, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wn), off)));
        }
        if (lane == 0) {
            sh.wmax[wave] = wm;
            sh.wmin[wave] = wn;
        }
        __syncthreads();
        kmax = sh.wmax[0];
        kmin = sh.wmin[0];
        for (int w = 1; w < kPickWaves; ++w) {
            kmax = max(kmax, sh.wmax[w]);
            kmin = min(kmin, sh.wmin[w]);
        }
        kmax = __builtin_amdgcn_readfirstlane(kmax);  // uniform: scalar registers, not 32 vector ones
        kmin = __builtin_amdgcn_readfirstlane(kmin);  // held until the end
        // a lower bound of the k-th largest key (a key of 0, past the vocabulary or a NaN, is never
        // kept): for k <= 1024 the k-th largest lane maximum; the keys at or above it listed in index
        // order with their indices when they fit the LDS
        low = 1;
        // (two digits: the bound's top 16 bits, enough to leave about k keys above it)
        if (bounded) low = max(low, radix_select([&](const auto& f) { f(tmax, true); }, top_k, sh, 2));
        // The keys at or above the bound, loaded again (holding them across the selection would
        // spill): bit s of `above` for slot s, and, with a bound, appended to an unordered list
        // through an LDS counter (usually about k of them).
        if (tid == 0) sh.appended = 0;
        __syncthreads();
        // key >= low exactly when key's top 16 bits >= low's (low's low 16 bits are zero); a top of 0
        // (past the vocabulary, or a NaN) is never a candidate
        const uint32_t low16 = max(low >> 16, 1u);
#pragma unroll
        for (int s = 0; s < kPickSlots; ++s) {
            const uint32_t t = s % 2 == 0 ? top16[s / 2] & 0xffffu : top16[s / 2] >> 16;
            above |= uint64_t{t >= low16} << s;
        }
        if (bounded) {
            for (uint64_t rest = above; rest != 0; rest &= rest - 1) {  // this lane's few candidates
                const int slot = __ffsll(static_cast<unsigned long long>(rest)) - 1;
                const uint32_t at = atomicAdd(&sh.appended, 1u);
                if (at < kRankList) {
                    sh.cand_key[at] = __builtin_amdgcn_raw_buffer_load_b32(keys_rsrc, (slot * kPickThreads + tid) * 4, 0, 0);
                    sh.cand_idx[at] = slot * kPickThreads + tid;
                }
                if (at >= kRankList) break;  // the list is long: the ordered path takes over
            }
        }
        __syncthreads();
        const uint32_t appended = __builtin_amdgcn_readfirstlane(sh.appended);  // LDS values are uniform
        unordered = bounded && appended <= kRankList;  // the short list, in no order
        if (unordered) {
            listed_n = appended;
            listed = true;
        } else if (bounded) {  // a longer list, in index order
            listed_n = ordered_compact(
                above,
                [&](int s, int64_t at, int64_t total) {
                    if (total <= kPickLdsKept) sh.cand_idx[at] = s * kPickThreads + tid;
                },
                sh);
            listed = listed_n <= kPickLdsKept;
            if (listed)  // the listed keys, all loads at once
                for (int64_t r = tid; r < listed_n; r += kPickThreads) sh.cand_key[r] = a.keys[sh.cand_idx[r]];
        }
    }
    if (listed) {  // zeros after the list to a multiple of 4
        if (tid < 4) sh.cand_key[listed_n + tid] = 0u;
        __syncthreads();
    }
    // the k-th largest key and the kept entries (keys at or above it) in index order
    constexpr int kListGroups = kPickLdsKept / kPickThreads;
    int64_t m;
    int32_t* kept;
    float* kept_e;
    if (listed) {
        const auto listed_key = [&](int j) {
            const int64_t r = int64_t{j} * kPickThreads + tid;
            return r < listed_n ? sh.cand_key[r] : 0u;
        };
        const int groups = static_cast<int>((listed_n + kPickThreads - 1) / kPickThreads);
        uint32_t kth;
        if (listed_n <= kRankList) {
            // Short lists: the k-th largest is the listed key k with #(keys > k) < top_k <=
            // #(keys >= k); every lane holding one counts over the list (broadcast LDS reads, four
            // keys a read; the zeros after the list count in neither).
            if (tid < listed_n) {
                const uint32_t mine = sh.cand_key[tid];
                int64_t gt = 0, ge = 0;
                for (int64_t j = 0; j < listed_n; j += 4) {
                    const uint4 q = *reinterpret_cast<const uint4*>(&sh.cand_key[j]);
                    gt += (q.x > mine) + (q.y > mine) + (q.z > mine) + (q.w > mine);
                    ge += (q.x >= mine) + (q.y >= mine) + (q.z >= mine) + (q.w >= mine);
                }
                if (gt < top_k && top_k <= ge) sh.chosen = mine;  // lanes with equal keys write the same value
            }
            __syncthreads();
            kth = sh.chosen;
        } else {
            kth = radix_select(
                [&](const auto& f) {
                    for (int j = 0; j < groups; ++j) f(listed_key(j), int64_t{j} * kPickThreads + tid < listed_n);
                },
                top_k, sh);
        }
        kept = sh.kept_i;
        kept_e = sh.kept_e;
        if (unordered) {
            // The kept entries of the unordered list in index order: each kept lane's position is
            // the number of kept entries with a smaller index (indices are distinct).
            if (tid < listed_n) {  // the lanes holding entries (the waves past the list skip the loop)
                const uint32_t key_mine = sh.cand_key[tid];
                const int32_t idx_mine = sh.cand_idx[tid];
                uint32_t total = 0, before = 0;
                for (int j = 0; j < static_cast<int>(listed_n); j += 4) {
                    const uint4 kq = *reinterpret_cast<const uint4*>(&sh.cand_key[j]);
                    const int4 iq = *reinterpret_cast<const int4*>(&sh.cand_idx[j]);
                    total += (kq.x >= kth) + (kq.y >= kth) + (kq.z >= kth) + (kq.w >= kth);
                    before += (kq.x >= kth && iq.x < idx_mine) + (kq.y >= kth && iq.y < idx_mine) +
                              (kq.z >= kth && iq.z < idx_mine) + (kq.w >= kth && iq.w < idx_mine);
                }
                if (key_mine >= kth) sh.kept_i[before] = idx_mine;
                if (tid == 0) sh.total = total;
            }
            __syncthreads();
            m = listed_n == 0 ? 0 : sh.total;  // an empty list (every key a NaN) keeps nothing
        } else {
            uint64_t keep = 0;
#pragma unroll
            for (int j = 0; j < kListGroups; ++j)
                keep |= uint64_t{int64_t{j} * kPickThreads + tid < listed_n && listed_key(j) >= kth} << j;
            m = ordered_compact(
                keep, [&](int j, int64_t at, int64_t) { sh.kept_i[at] = sh.cand_idx[j * kPickThreads + tid]; }, sh);
        }
    } else {
        // without a top-k (top_k = the vocabulary) every entry is kept: the cut is the smallest key
        const uint32_t kth = top_k >= V ? kmin
                                        : max(low, radix_select(
                                                       [&](const auto& f) {
#pragma unroll
                                                           for (int s = 0; s < kPickSlots; ++s) {
                                                               const uint32_t k = key_at(s);
                                                               f(k, k >= low);
                                                           }
                                                       },
                                                       top_k, sh));
        uint64_t keep = 0;
#pragma unroll
        for (int s = 0; s < kPickSlots; ++s) keep |= uint64_t{key_at(s) >= kth} << s;
        m = ordered_compact(
            keep,
            [&](int s, int64_t at, int64_t total) {
                (total <= kPickLdsKept ? sh.kept_i : a.kept)[at] = s * kPickThreads + tid;
            },
            sh);
        kept = m <= kPickLdsKept ? sh.kept_i : a.kept;
        kept_e = m <= kPickLdsKept ? sh.kept_e : a.kept_e;
    }
    // softmax's f32 exponentials exp(x - max) of the kept entries (src/ops/nn.cpp:60-71), x divided
    // again as head_kernel divides it; key_value recovers the largest x exactly
    const float temp = a.sp->temperature;
    const float mx = key_value(kmax);
    for (int64_t r = tid; r < m; r += kPickThreads) kept_e[r] = expf(__fdiv_rn(a.logits[kept[r]], temp) - mx);
    __syncthreads();
    int32_t nonfinite = kmax > kFiniteKeyHigh || kmin < kFiniteKeyLow;
    if (wave != 0) return;
    // The sums below run in index order in double, as kael's CPU loops do: wave 0 loads 64 entries
    // at a time, one per lane, and folds them in lane order through readlane, so only one load per
    // 64 entries stands in the dependent chain.
    const auto entry = [](float v, int j) { return static_cast<double>(lane_value(v, j)); };
    Sampler& sp = *a.sp;
    if (nonfinite || draw >= draws) {
        if (lane == 0) sp.error = nonfinite ? 1 : 2;
        token = 0;
        return;
    }
    if (lane == 0) sp.draw = draw + 1;
    m = __builtin_amdgcn_readfirstlane(static_cast<int>(m));  // uniform: the loops below index lanes by it
    if (m <= 64) {
        // One load group, lane j holding entry j. Where every positive value is at least 2^-24 (and
        // at most 1: e = exp(x - max) <= 1, and p = e / sum <= e as sum >= 1), each value is a whole
        // multiple of 2^-47 and every partial sum of at most 64 of them a whole multiple of 2^-47
        // below 2^53 of them, so each double addition is exact and any order gives the sequential
        // sums bit for bit: a wave sum and a wave prefix sum then stand in for the loops. Otherwise
        // the loops run. Lane j's running sum is the walk's sum after entry j, so the first sum
        // past the point and the last positive weight are ballots.
        const bool in = lane < m;
        const auto exact = [&](float v) { return -wave_max(in && v > 0.f ? -v : -1.f) >= 0x1p-24f; };
        const float e = in ? kept_e[lane] : 0.f;
        double sum = 0.0;
        if (exact(e)) {
            sum = wave_sum(static_cast<double>(e));
        } else {
            for (int j = 0; j < m; ++j) sum += entry(e, j);
        }
        const float denominator = static_cast<float>(sum);
        const float p = in ? __fdiv_rn(e, denominator) : 0.f;
        double mine = static_cast<double>(p), cumulative = 0.0;
        if (exact(p)) {
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const double o = __shfl_up(mine, off);
                if (lane >= off) mine += o;
            }
            cumulative = lane_value(mine, static_cast<int>(m) - 1);
        } else {
            for (int j = 0; j < m; ++j) {
                cumulative += entry(p, j);
                if (lane == j) mine = cumulative;
            }
        }
        // multinomial (src/random.cpp:143-151): point = u * total, upper_bound, and the step back
        // to a positive weight when the point is past every sum
        const double point = u * cumulative;
        const int32_t index = in ? kept[lane] : 0;
        const uint64_t past = __ballot(in && mine > point);
        const uint64_t positive = __ballot(in && p > 0.f);
        if (past != 0) token = __builtin_amdgcn_readlane(index, __ffsll(static_cast<unsigned long long>(past)) - 1);
        else if (positive != 0) token = __builtin_amdgcn_readlane(index, 63 - __clzll(static_cast<long long>(positive)));
        else token = kept[0];
        return;
    }
    // Whole groups of 64 fold with the lane index a constant (unrolled: no loop counter or
    // computed lane select in the dependent chain of additions), the last group in a loop. The
    // group is widened to double once, so each entry is two lane reads into scalar registers,
    // off the chain, and one addition.
    const auto fold = [&](float v, int64_t base, auto&& add) {
        const double w = static_cast<double>(v);
        if (m - base >= 64) {
#pragma unroll
            for (int j0 = 0; j0 < 64; j0 += 16) {  // 16 entries read ahead of their additions
                double x[16];
#pragma unroll
                for (int j = 0; j < 16; ++j) x[j] = lane_value(w, j0 + j);
#pragma unroll
                for (int j = 0; j < 16; ++j) add(j0 + j, x[j]);
            }
        } else {
            const int n = static_cast<int>(m - base);
            for (int j = 0; j < n; ++j) add(j, lane_value(w, j));
        }
    };
    // The groups in index order, lane j holding entry base + j (0 past the list): the loads of
    // the next kAhead groups go out before the current kAhead groups fold, since a list longer
    // than the LDS stage lives in global memory, a round trip away. The loads read clamped, always
    // valid, indices, so that no branch separates them.
    constexpr int kAhead = 4;
    const auto groups = [&](auto&& body) {  // body(e, index, base) for each group
        float ec[kAhead], en[kAhead];
        int32_t ic[kAhead], in_[kAhead];
        const auto load = [&](int64_t base, float (&e)[kAhead], int32_t (&ix)[kAhead]) {
#pragma unroll
            for (int g = 0; g < kAhead; ++g) {
                const int64_t i = base + g * 64 + lane;
                const int64_t c = min<int64_t>(i, m - 1);
                e[g] = kept_e[c];
                ix[g] = kept[c];
                if (i >= m) e[g] = 0.f;
            }
        };
        load(0, ec, ic);
        for (int64_t base = 0; base < m; base += kAhead * 64) {
            load(base + kAhead * 64, en, in_);  // (past the list: clamped, unused)
#pragma unroll
            for (int g = 0; g < kAhead; ++g)
                if (base + g * 64 < m && !body(ec[g], ic[g], base + g * 64)) return;
#pragma unroll
            for (int g = 0; g < kAhead; ++g) {
                ec[g] = en[g];
                ic[g] = in_[g];
            }
        }
    };
    // the sum of e in double in index order, rounded to f32
    double sum = 0.0;
    groups([&](float e, int32_t, int64_t base) {
        fold(e, base, [&](int, double x) { sum += x; });
        return true;
    });
    const float denominator = static_cast<float>(sum);
    // multinomial (src/random.cpp:143-151): the cumulative sum in double, point = u * total,
    // upper_bound, and the step back to a positive weight when the point is past every sum
    double cumulative = 0.0;
    groups([&](float e, int32_t, int64_t base) {
        fold(__fdiv_rn(e, denominator), base, [&](int, double x) { cumulative += x; });
        return true;
    });
    const double point = u * cumulative;
    // the walk: each group's running sums are the previous group's end plus a prefix in order,
    // so the first group whose end passes the point holds the pick
    double run = 0.0;
    int64_t pick = -1, last_positive = kept[0];
    groups([&](float e, int32_t index, int64_t base) {
        const float p = __fdiv_rn(e, denominator);  // 0 past the list
        double end = run;
        fold(p, base, [&](int, double x) { end += x; });
        const uint64_t positive = __ballot(p > 0.f);
        if (end > point) {  // the pick is in this group: walk it entry by entry
            const int n = static_cast<int>(min<int64_t>(64, m - base));
            for (int j = 0; j < n; ++j) {
                run += lane_value(static_cast<double>(p), j);
                if (run > point) {
                    pick = __builtin_amdgcn_readlane(index, j);
                    return false;
                }
            }
        }
        run = end;
        if (positive != 0) last_positive = __builtin_amdgcn_readlane(index, 63 - __clzll(static_cast<long long>(positive)));
        return true;
    });
    token = pick >= 0 ? pick : last_positive;
}

__global__ __launch_bounds__(kPickThreads) void pick_kernel(PickArgs a) {
    __shared__ float bv[kPickWaves];
    __shared__ int64_t bi[kPickWaves];
    if (a.sp->top_k > 0) {
        int64_t token = 0;
        sample_pick(a, token);
        if (threadIdx.x == 0) {
            const int64_t pos = a.st->pos;
            if (pos + 1 >= a.st->forced) a.seq[pos + 1] = token;
            a.st->pos = pos + 1;
        }
        return;
    }
    Best r{-INFINITY, INT64_MAX};
    for (int64_t i = threadIdx.x; i < a.parts; i += kPickThreads) {
        Best o{a.pv[i], a.pi[i]};
        if (better(o, r)) r = o;
    }
    r = wave_best(r);
    if (threadIdx.x % 64 == 0) {
        bv[threadIdx.x / 64] = r.v;
        bi[threadIdx.x / 64] = r.i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        Best w{bv[0], bi[0]};
        for (int k = 1; k < kPickWaves; ++k) {
            Best o{bv[k], bi[k]};
            if (better(o, w)) w = o;
        }
        const int64_t pos = a.st->pos;
        if (pos + 1 >= a.st->forced) a.seq[pos + 1] = w.i;
        a.st->pos = pos + 1;
    }
}

// Split attention over the cached keys of one head: workgroup (h, c) takes chunk c of the
// L = pos + 1 keys (the decode query sees every cached key, so no mask applies). Scores are
// q.k / sqrt(head_dim) (16-lane groups, 16-byte loads, group shuffle reduction); the chunk keeps
// its maximum m_c, the double sum l_c of exp(s - m_c) and the unnormalised weighted values
// acc_c = sum exp(s - m_c) v. attn_load() / attn_finish() merge the chunks.
__global__ __launch_bounds__(kThreads) void attention_kernel(const Step* st, const float* __restrict__ q,
                                                             const float* __restrict__ kcache,
                                                             const float* __restrict__ vcache, AttnPartials part,
                                                             int64_t head_dim, int64_t max_positions, float divisor) {
    extern __shared__ float scores[];  // [chunk length]
    __shared__ float red_f[kThreads / 64];
    __shared__ double red_d[kThreads / 64];
    __shared__ float4 acc_part[kThreads / 16][16];
    const int64_t h = blockIdx.x;
    const int64_t c = blockIdx.y;
    const int64_t L = st->pos + 1;
    const int64_t chunk = (L + kAttnChunks - 1) / kAttnChunks;
    const int64_t j0 = c * chunk;
    const int64_t count = j0 < L ? (j0 + chunk < L ? chunk : L - j0) : 0;
    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int sub = tid % 16, group = tid / 16;  // 16 groups of 16 lanes
    const bool dims_ok = 4 * sub < head_dim;
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (dims_ok) qv = *reinterpret_cast<const float4*>(q + h * head_dim + 4 * sub);
    const float* K = kcache + (h * max_positions + j0) * head_dim;
    const float* V = vcache + (h * max_positions + j0) * head_dim;
    // The first kAttnRegs keys of each 16-lane group: key and value rows issued together up
    // front (the value loads need only the position, not the scores).
    float4 kreg[kAttnRegs], vreg[kAttnRegs];
#pragma unroll
    for (int u = 0; u < kAttnRegs; ++u) {
        const int64_t j = group + u * (kThreads / 16);
        const bool ok = dims_ok && j < count;
        kreg[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        vreg[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok) {
            kreg[u] = *reinterpret_cast<const float4*>(K + j * head_dim + 4 * sub);
            vreg[u] = *reinterpret_cast<const float4*>(V + j * head_dim + 4 * sub);
        }
    }
    float local_max = -INFINITY;
    const auto score = [&](int64_t j, float4 k) {
        float sc = qv.x * k.x + qv.y * k.y + qv.z * k.z + qv.w * k.w;
        sc = row16_sum(sc);
        sc = __fdiv_rn(sc, divisor);
        if (sub == 0) scores[j] = sc;
        local_max = max_na(local_max, sc);
    };
#pragma unroll
    for (int u = 0; u < kAttnRegs; ++u) {
        const int64_t j = group + u * (kThreads / 16);
        if (j < count) score(j, kreg[u]);
    }
    for (int64_t j = group + kAttnRegs * (kThreads / 16); j < count; j += kThreads / 16) {
        float4 k = make_float4(0.f, 0.f, 0.f, 0.f);
        if (dims_ok) k = *reinterpret_cast<const float4*>(K + j * head_dim + 4 * sub);
        score(j, k);
    }
    local_max = wave_max(local_max);
    if (lane == 0) red_f[wave] = local_max;
    __syncthreads();
    float largest = red_f[0];
    for (int w = 1; w < kThreads / 64; ++w) largest = max_na(largest, red_f[w]);
    double total = 0.0;
    for (int64_t j = tid; j < count; j += kThreads) {
        const float e = std::exp(__fsub_rn(scores[j], largest));
        scores[j] = e;
        total += static_cast<double>(e);
    }
    total = wave_sum(total);
    if (lane == 0) red_d[wave] = total;
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (dims_ok) {
        const auto accumulate = [&](int64_t j, float4 v) {
            const float w = scores[j];
            acc.x += w * v.x;
            acc.y += w * v.y;
            acc.z += w * v.z;
            acc.w += w * v.w;
        };
#pragma unroll
        for (int u = 0; u < kAttnRegs; ++u) {
            const int64_t j = group + u * (kThreads / 16);
            if (j < count) accumulate(j, vreg[u]);
        }
        for (int64_t j = group + kAttnRegs * (kThreads / 16); j < count; j += kThreads / 16)
            accumulate(j, *reinterpret_cast<const float4*>(V + j * head_dim + 4 * sub));
    }
    acc_part[group][sub] = acc;
    __syncthreads();
    const int64_t slot = h * kAttnChunks + c;
    if (tid < head_dim) {
        const int s4 = tid / 4, e = tid % 4;
        float r = 0.f;
        for (int g = 0; g < kThreads / 16; ++g) {
            const float4 pv = acc_part[g][s4];
            r += e == 0 ? pv.x : e == 1 ? pv.y : e == 2 ? pv.z : pv.w;
        }
        part.acc[slot * head_dim + tid] = r;
    }
    if (tid == 0) {
        double sum = red_d[0];
        for (int w = 1; w < kThreads / 64; ++w) sum += red_d[w];
        part.m[slot] = largest;
        part.l[slot] = sum;
    }
}

// ---- batched prefill ---------------------------------------------------------------------------
//
// The prompt's T positions pass each layer together: row LayerNorms, the four Linear products
// as GEMMs on the MFMA matmul path (weights in [in, out] copies made once so that both operands
// are row-major; prompts of up to 128 positions as split-K partial products on 64x64 tiles, longer
// ones on the backend's matmul path with rows padded to 128), epilogue kernels for the partial
// sums, the bias, residual, GELU and the K/V rows into the cache, and a causal attention kernel.
// Same arithmetic as the decode step; only the summation order of the dot products differs.

// The row LayerNorm H[t] = LayerNorm(X[t]) of a row that lane i of the workgroup has just
// computed at elements i, i + 256, ... (x[j], j < 4), as ln_load and ln_finish compute it from
// memory: the pivot x[0] passes through LDS.
// The weight and bias elements of lane i (i, i + 256, ...) are given already loaded.
__device__ __forceinline__ void ln_row_from_lanes(const float (&x)[4], int64_t d, const float (&w)[4],
                                                  const float (&b)[4], float* h) {
    __shared__ float pivot;
    LnIn r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        r.x[j] = i < d ? x[j] : 0.f;
        r.w[j] = i < d ? w[j] : 0.f;
        r.b[j] = i < d ? b[j] : 0.f;
    }
    if (threadIdx.x == 0) pivot = x[0];
    __syncthreads();
    r.c = pivot;
    ln_finish(r, d, h);
}

__device__ __forceinline__ void ln_row_from_lanes(const float (&x)[4], int64_t d, const float* w, const float* b,
                                                  float* h) {
    float wl[4], bl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        wl[j] = i < d ? w[i] : 0.f;
        bl[j] = i < d ? b[i] : 0.f;
    }
    ln_row_from_lanes(x, d, wl, bl, h);
}

// Split-K partial products whose loads a thread issues together: one memory round trip for up to
// this many splits (the prefill's products split K at most 16 ways on 256 CUs). The loads read
// clamped, always valid addresses, so that no branch separates them.
constexpr int kSplitBatch = 16;

// X[t] = wte[seq[t]] + wpe[t], and H[t] = LayerNorm(X[t]) with the first block's ln1; one
// workgroup per row.
__global__ __launch_bounds__(kThreads) void prefill_embed_kernel(const int64_t* seq, const float* wte, const float* wpe,
                                                                 float* X, const float* ln_w, const float* ln_b,
                                                                 float* H, int64_t d) {
    const int64_t t = blockIdx.x;
    const int64_t tok = seq[t];
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        x[j] = 0.f;
        if (i < d) {
            x[j] = __fadd_rn(wte[tok * d + i], wpe[t * d + i]);
            X[t * d + i] = x[j];
        }
    }
    ln_row_from_lanes(x, d, ln_w, ln_b, H + t * d);
}

// The residual epilogue of a d-wide product, one workgroup per row: X[t, n] += P[t, n] + bias[n]
// (P the sum of `splits` partials `split_stride` apart, added in split order), then, with ln_w,
// H[t] = LayerNorm(X[t]) for the next product (the following LayerNorm, computed in the same
// workgroup instead of a launch of its own).
__global__ __launch_bounds__(kThreads) void prefill_residual_kernel(const float* P, int64_t splits, int64_t split_stride,
                                                                    const float* bias, float* X, const float* ln_w,
                                                                    const float* ln_b, float* H, int64_t d) {
    const int64_t t = blockIdx.x;
    // every load first: the residual row, the bias, the next LayerNorm's parameters (the bias
    // again, unused, without one), the partials
    const float* lwp = ln_w != nullptr ? ln_w : bias;
    const float* lbp = ln_w != nullptr ? ln_b : bias;
    float xr[4], bs[4], lw[4], lb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = std::min<int64_t>(threadIdx.x + j * kThreads, d - 1);
        xr[j] = X[t * d + i];
        bs[j] = bias[i];
        lw[j] = lwp[i];
        lb[j] = lbp[i];
    }
    float p[4] = {0.f, 0.f, 0.f, 0.f};
    if (splits == 1) {  // one product (longer prompts)
#pragma unroll
        for (int j = 0; j < 4; ++j) p[j] = P[t * d + std::min<int64_t>(threadIdx.x + j * kThreads, d - 1)];
    }
    for (int64_t s0 = 0; s0 < splits && splits > 1; s0 += kSplitBatch) {
        float v[kSplitBatch][4];
#pragma unroll
        for (int q = 0; q < kSplitBatch; ++q) {
            const int64_t sq = std::min<int64_t>(s0 + q, splits - 1);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t i = std::min<int64_t>(threadIdx.x + j * kThreads, d - 1);
                v[q][j] = P[sq * split_stride + t * d + i];
            }
        }
#pragma unroll
        for (int q = 0; q < kSplitBatch; ++q)  // added in split order
            if (s0 + q < splits) {
#pragma unroll
                for (int j = 0; j < 4; ++j) p[j] = s0 + q == 0 ? v[q][j] : __fadd_rn(p[j], v[q][j]);
            }
    }
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t i = threadIdx.x + j * kThreads;
        x[j] = 0.f;
        if (i < d) {
            x[j] = __fadd_rn(xr[j], __fadd_rn(p[j], bs[j]));
            X[t * d + i] = x[j];
        }
    }
    if (ln_w != nullptr) ln_row_from_lanes(x, d, lw, lb, H + t * d);
}

// y = P[t, n] + bias[n] for the T x N product P (row stride N; with split K, P[t, n] is the sum
// of the `splits` partial products P + s * split_stride in split order), then by epilogue:
//   kQkv       query part -> Q[t, n]; key and value parts -> the cache rows of position t
//   kGelu*     F[t, n] = gelu(y)
// (the residual products take prefill_residual_kernel, which also computes the next LayerNorm).
template <int Epi, int Batch>
__global__ __launch_bounds__(kThreads) void prefill_epilogue_kernel(const float* P, int64_t splits, int64_t split_stride,
                                                                    const float* bias, float* out, int64_t T, int64_t N,
                                                                    int64_t d, int64_t head_dim, int64_t max_positions,
                                                                    float* kcache, float* vcache) {
    const int64_t total = T * N;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t t = e / N;
        const int64_t n = e - t * N;
        const float bn = bias[n];
        float p = splits == 1 ? P[e] : 0.f;  // one product (longer prompts) or split partials
        for (int64_t s0 = 0; s0 < splits && splits > 1; s0 += Batch) {
            float v[Batch];
#pragma unroll
            for (int q = 0; q < Batch; ++q) v[q] = P[std::min<int64_t>(s0 + q, splits - 1) * split_stride + e];
#pragma unroll
            for (int q = 0; q < Batch; ++q)  // added in split order
                if (s0 + q < splits) p = s0 + q == 0 ? v[q] : __fadd_rn(p, v[q]);
        }
        const float y = __fadd_rn(p, bn);
        if constexpr (Epi == kQkv) {
            const int64_t part = n / d;
            const int64_t within = n - part * d;
            if (part == 0) {
                out[t * d + within] = y;
            } else {
                const int64_t head = within / head_dim;
                const int64_t dim = within - head * head_dim;
                float* cache = part == 1 ? kcache : vcache;
                cache[(head * max_positions + t) * head_dim + dim] = y;
            }
        } else {
            static_assert(Epi == kGeluTanh || Epi == kGeluExact);
            out[e] = gelu_of<Epi>(y);
        }
    }
}

// Causal attention of query t of head h (workgroup (h, t)) over keys 0..t: scores q.k /
// sqrt(head_dim) by 16-lane groups, the row maximum, exponentials summed in double, the
// weighted sum of values divided by the float rounding of that sum.
__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(const float* __restrict__ Q,
                                                                     const float* __restrict__ kcache,
                                                                     const float* __restrict__ vcache, float* A,
                                                                     int64_t d, int64_t head_dim, int64_t max_positions,
                                                                     float divisor) {
    extern __shared__ float scores[];  // [t + 1]
    __shared__ float red_f[kThreads / 64];
    __shared__ double red_d[kThreads / 64];
    __shared__ float4 acc_part[kThreads / 16][16];
    const int64_t h = blockIdx.x;
    const int64_t t = blockIdx.y;
    const int64_t count = t + 1;
    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int sub = tid % 16, group = tid / 16;
    const bool dims_ok = 4 * sub < head_dim;
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (dims_ok) qv = *reinterpret_cast<const float4*>(Q + t * d + h * head_dim + 4 * sub);
    const float* K = kcache + h * max_positions * head_dim;
    const float* V = vcache + h * max_positions * head_dim;
    float local_max = -INFINITY;
    for (int64_t j = group; j < count; j += kThreads / 16) {
        float4 k = make_float4(0.f, 0.f, 0.f, 0.f);
        if (dims_ok) k = *reinterpret_cast<const float4*>(K + j * head_dim + 4 * sub);
        float sc = qv.x * k.x + qv.y * k.y + qv.z * k.z + qv.w * k.w;
        sc = row16_sum(sc);
        sc = __fdiv_rn(sc, divisor);
        if (sub == 0) scores[j] = sc;
        local_max = max_na(local_max, sc);
    }
    local_max = wave_max(local_max);
    if (lane == 0) red_f[wave] = local_max;
    __syncthreads();
    float largest = red_f[0];
    for (int w = 1; w < kThreads / 64; ++w) largest = max_na(largest, red_f[w]);
    double total = 0.0;
    for (int64_t j = tid; j < count; j += kThreads) {
        const float e = std::exp(__fsub_rn(scores[j], largest));
        scores[j] = e;
        total += static_cast<double>(e);
    }
    total = wave_sum(total);
    if (lane == 0) red_d[wave] = total;
    __syncthreads();
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (dims_ok) {
        for (int64_t j = group; j < count; j += kThreads / 16) {
            const float w = scores[j];
            const float4 v = *reinterpret_cast<const float4*>(V + j * head_dim + 4 * sub);
            acc.x += w * v.x;
            acc.y += w * v.y;
            acc.z += w * v.z;
            acc.w += w * v.w;
        }
    }
    acc_part[group][sub] = acc;
    __syncthreads();
    if (tid < head_dim) {
        double sum = red_d[0];
        for (int w = 1; w < kThreads / 64; ++w) sum += red_d[w];
        const int s4 = tid / 4, e = tid % 4;
        float r = 0.f;
        for (int g = 0; g < kThreads / 16; ++g) {
            const float4 pv = acc_part[g][s4];
            r += e == 0 ? pv.x : e == 1 ? pv.y : e == 2 ? pv.z : pv.w;
        }
        A[t * d + h * head_dim + tid] = __fdiv_rn(r, static_cast<float>(sum));
    }
}

// ---- engine ----------------------------------------------------------------------------------

struct Engine {
    kd_gpt_config cfg{};
    int64_t d = 0, hd = 0, ff = 0;
    hipStream_t stream = nullptr;
    float* params = nullptr;  // every parameter, kael names -> offsets
    std::unordered_map<std::string, std::pair<int64_t, int64_t>> offsets;  // name -> (offset, count)
    std::vector<bool> loaded;
    std::vector<std::string> names;
    std::unordered_map<std::string, std::vector<int64_t>> shape_of;  // name -> kael's shape
    float* kcache = nullptr;
    float* vcache = nullptr;
    float* x = nullptr;
    float* q = nullptr;
    AttnPartials partials{};
    float* f = nullptr;
    float* logits = nullptr;
    float* pv = nullptr;     // head argmax partials, one per workgroup
    int64_t* pi = nullptr;
    int64_t* seq = nullptr;
    Step* st = nullptr;
    Sampler* sp = nullptr;       // the pick's mode and draws (device)
    double* uniforms = nullptr;  // [max_positions + 1] draws for sampled picks
    int32_t* kept = nullptr;     // [vocab] sampling scratch
    float* kept_e = nullptr;     // [vocab]
    uint32_t* keys = nullptr;    // [65536] order keys of the sampled pick's x, zero past the vocabulary
    uint32_t* key_parts = nullptr;  // [2 * head workgroups] their largest and smallest keys
    Sampler host_sp{0.f, 0, 0, 0, 0};
    hipGraphExec_t graph = nullptr;
    int64_t host_pos = 0;     // mirror of st->pos: positions in the KV cache
    std::vector<int64_t> history;  // the whole sequence so far (prompt + generated), host copy
    int64_t host_forced = 0;
    // batched prefill (allocated at the first prefill): activations of up to pf_rows positions
    // (max_positions rounded up to whole 128-row tiles) and the weights as [in, out] copies
    int64_t pf_rows = 0;
    float* pf_x = nullptr;    // [pf_rows, d] residual stream
    float* pf_h = nullptr;    // [pf_rows, d] LayerNorm output
    float* pf_q = nullptr;    // [pf_rows, d] queries
    float* pf_a = nullptr;    // [pf_rows, d] attention output
    float* pf_f = nullptr;    // [pf_rows, ff] GELU output
    float* pf_p = nullptr;    // [pf_rows, max(3d, ff)] product before its epilogue
    float* pf_parts = nullptr;  // split-K partial products of prompts of at most 128 positions
    float* wt = nullptr;      // per layer: qkv^T [d, 3d], proj^T [d, d], fc1^T [d, ff], fc2^T [ff, d]
    bool wt_valid = false;    // cleared by every parameter upload

    const float* p(const std::string& name) const { return params + offsets.at(name).first; }

    GemvArgs base() const {
        GemvArgs a{};
        a.d = d;
        a.head_dim = hd;
        a.max_positions = cfg.max_positions;
        a.st = st;
        return a;
    }

    PickArgs pick_args() const {
        return PickArgs{st, seq, pv, pi, head_groups(), logits, cfg.vocab_size, sp, uniforms, kept, kept_e, keys, key_parts};
    }

    // Workgroups of head_kernel: 4 per CU, fewer when the vocabulary has fewer row pairs than
    // that grid has waves.
    int64_t head_groups() const {
        const int64_t waves = (cfg.vocab_size + 1) / 2;
        return std::max<int64_t>(1, std::min<int64_t>(4 * compute_units(), (waves + 3) / 4));
    }

    static dim3 rows_grid(int64_t n, bool split_k) {
        return dim3(static_cast<uint32_t>(split_k ? (n + 1) / 2 : (n + 7) / 8));
    }

    // Ln: the input is LayerNorm(a.x) with weight a.ln_w and bias a.ln_b (K = d).
    template <int Epi, int Pro> void gemv(hipStream_t s, const GemvArgs& a) const {
        // Long rows and few of them (fc2: K = 3072, N = 768): split K across the workgroup's waves
        // so that more workgroups stream weights. Rows of K <= 1024 take one wave per row pair:
        // measured 1.5 us faster per LayerNorm GEMV at K = 768 (fewer workgroups repeat the
        // LayerNorm and no cross-wave combine), 0.5 us without a prologue.
        const bool split = a.N <= 4096 && a.K > 1024;
        if (split) hipLaunchKernelGGL((gemv_kernel<Epi, 4, Pro>), rows_grid(a.N, true), dim3(kThreads), 0, s, a);
        else hipLaunchKernelGGL((gemv_kernel<Epi, 1, Pro>), rows_grid(a.N, false), dim3(kThreads), 0, s, a);
    }

    // One decode step: one kernel per phase, 63 launches per GPT-2-small token.
    int record_step(hipStream_t s) {
        const int64_t L = cfg.layers;
        hipLaunchKernelGGL(embed_kernel, dim3(static_cast<uint32_t>((d + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, st,
                           seq, p("token_embedding.weight"), p("position_embedding.weight"), x, d);
        const size_t attn_lds = static_cast<size_t>((cfg.max_positions + kAttnChunks - 1) / kAttnChunks) * sizeof(float);
        const float divisor = static_cast<float>(std::sqrt(static_cast<double>(hd)));
        for (int64_t l = 0; l < L; ++l) {
            const std::string b = "blocks." + std::to_string(l) + ".";
            float* kc = kcache + l * cfg.heads * cfg.max_positions * hd;
            float* vc = vcache + l * cfg.heads * cfg.max_positions * hd;
            GemvArgs qkv = base();
            qkv.W = p(b + "attn.qkv.weight");
            qkv.bias = p(b + "attn.qkv.bias");
            qkv.x = x;
            qkv.N = 3 * d;
            qkv.K = d;
            qkv.ln_w = p(b + "ln1.weight");
            qkv.ln_b = p(b + "ln1.bias");
            qkv.q = q;
            qkv.kcache = kc;
            qkv.vcache = vc;
            gemv<kQkv, kLn>(s, qkv);
            hipLaunchKernelGGL(attention_kernel, dim3(static_cast<uint32_t>(cfg.heads), kAttnChunks), dim3(kThreads), attn_lds,
                               s, st, q, kc, vc, partials, hd, cfg.max_positions, divisor);
            GemvArgs proj = base();
            proj.W = p(b + "attn.proj.weight");
            proj.bias = p(b + "attn.proj.bias");
            proj.x = nullptr;
            proj.attn = partials;
            proj.out = x;
            proj.N = d;
            proj.K = d;
            gemv<kResidual, kAttn>(s, proj);
            GemvArgs fc1 = base();
            fc1.W = p(b + "mlp.fc1.weight");
            fc1.bias = p(b + "mlp.fc1.bias");
            fc1.x = x;
            fc1.out = f;
            fc1.N = ff;
            fc1.K = d;
            fc1.ln_w = p(b + "ln2.weight");
            fc1.ln_b = p(b + "ln2.bias");
            if (cfg.tanh_gelu) gemv<kGeluTanh, kLn>(s, fc1);
            else gemv<kGeluExact, kLn>(s, fc1);
            GemvArgs fc2 = base();
            fc2.W = p(b + "mlp.fc2.weight");
            fc2.bias = p(b + "mlp.fc2.bias");
            fc2.x = f;
            fc2.out = x;
            fc2.N = d;
            fc2.K = ff;
            gemv<kResidual, kPlain>(s, fc2);
        }
        GemvArgs head = base();
        head.W = p("token_embedding.weight");
        head.x = x;
        head.ln_w = p("ln_final.weight");
        head.ln_b = p("ln_final.bias");
        head.N = cfg.vocab_size;
        head.K = d;
        head.out = logits;
        head.best_v = pv;
        head.best_i = pi;
        head.sp = sp;
        head.keys = keys;
        head.key_parts = key_parts;
        const int64_t parts = head_groups();
        hipLaunchKernelGGL(head_kernel, dim3(static_cast<uint32_t>(parts)), dim3(kThreads), 0, s, head);
        hipLaunchKernelGGL(pick_kernel, dim3(1), dim3(kPickThreads), 0, s, pick_args());
        return KD_OK;
    }

    int build_graph() {
        if (graph != nullptr || eager()) return KD_OK;
        hipGraph_t g;
        KD_HIP(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
        record_step(stream);
        KD_HIP(hipStreamEndCapture(stream, &g));
        KD_HIP(hipGraphInstantiate(&graph, g, nullptr, nullptr, 0));
        KD_HIP(hipGraphDestroy(g));
        return KD_OK;
    }

    int ready() {
        for (size_t i = 0; i < loaded.size(); ++i)
            if (!loaded[i]) return fail(KD_E_INVALID, "kd_gpt: parameter " + names[i] + " was never loaded");
        return build_graph();
    }

    int set_state(int64_t pos, int64_t forced) {
        Step s{pos, forced};
        KD_HIP(hipMemcpyAsync(st, &s, sizeof s, hipMemcpyHostToDevice, stream));
        KD_HIP(hipStreamSynchronize(stream));
        host_pos = pos;
        host_forced = forced;
        return KD_OK;
    }

    bool eager() const { return (cfg.flags & KD_GPT_EAGER) != 0; }

    int steps(int64_t count) {
        if (host_pos + count > cfg.max_positions)
            return fail(KD_E_INVALID, "kd_gpt: cached steps past max_positions");
        for (int64_t i = 0; i < count; ++i) {
            if (eager()) {
                record_step(stream);
                KD_LAUNCH_CHECK();
            } else {
                KD_HIP(hipGraphLaunch(graph, stream));
            }
        }
        host_pos += count;
        return KD_OK;
    }

    bool stepwise_prefill() const { return (cfg.flags & KD_GPT_STEPWISE_PREFILL) != 0; }

    int64_t layer_t_floats() const { return 12 * d * d; }
    float* wt_qkv(int64_t l) const { return wt + l * layer_t_floats(); }
    float* wt_proj(int64_t l) const { return wt_qkv(l) + 3 * d * d; }
    float* wt_fc1(int64_t l) const { return wt_proj(l) + d * d; }
    float* wt_fc2(int64_t l) const { return wt_fc1(l) + d * ff; }

    int ensure_prefill_buffers() {
        if (pf_x != nullptr) return KD_OK;
        pf_rows = (cfg.max_positions + 127) / 128 * 128;
        for (auto [ptr, cols] : {std::pair<float**, int64_t>{&pf_x, d}, {&pf_h, d}, {&pf_q, d}, {&pf_a, d}, {&pf_f, ff},
                                 {&pf_p, std::max(3 * d, ff)}}) {
            void* mem = nullptr;
            KD_HIP(hipMalloc(&mem, static_cast<size_t>(pf_rows * cols) * sizeof(float)));
            *ptr = static_cast<float*>(mem);
        }
        void* mem = nullptr;
        KD_HIP(hipMalloc(&mem, static_cast<size_t>(cfg.layers * layer_t_floats()) * sizeof(float)));
        wt = static_cast<float*>(mem);
        mem = nullptr;
        KD_HIP(hipMalloc(&mem, static_cast<size_t>(parts_floats()) * sizeof(float)));
        pf_parts = static_cast<float*>(mem);
        return KD_OK;
    }

    // Prompts of at most kShortPrompt positions: rows padded to 64 and the products split over K
    // into pf_parts (at most one 64x64-tile workgroup per CU, or one whole product), which the
    // epilogue adds in split order.
    static constexpr int64_t kShortPrompt = 128;
    int64_t parts_floats() const {
        return std::max<int64_t>(int64_t{compute_units()} * 64 * 64, kShortPrompt * std::max(3 * d, ff));
    }

    // A product ready for its epilogue: P (row stride N), or `splits` partials `stride` apart.
    struct Product {
        const float* P;
        int64_t splits;
        int64_t stride;
    };

    // dst [K, N] row-major = transpose of src [N, K] row-major (kael's Linear weight).
    static int transpose_into(float* dst, const float* src, int64_t N, int64_t K) {
        kd_element_layout l{};
        l.dims = 2;
        l.operands = 2;
        l.count = N * K;
        l.shape[0] = K;
        l.shape[1] = N;
        l.strides[0][0] = N * 4;
        l.strides[0][1] = 4;
        l.strides[1][0] = 4;
        l.strides[1][1] = K * 4;
        l.base[0] = dst;
        l.base[1] = const_cast<float*>(src);
        return kd_convert(KD_F32, KD_F32, &l);
    }

    int refresh_transposed() {
        if (wt_valid) return KD_OK;
        for (int64_t l = 0; l < cfg.layers; ++l) {
            const std::string b = "blocks." + std::to_string(l) + ".";
            if (int rc = transpose_into(wt_qkv(l), p(b + "attn.qkv.weight"), 3 * d, d)) return rc;
            if (int rc = transpose_into(wt_proj(l), p(b + "attn.proj.weight"), d, d)) return rc;
            if (int rc = transpose_into(wt_fc1(l), p(b + "mlp.fc1.weight"), ff, d)) return rc;
            if (int rc = transpose_into(wt_fc2(l), p(b + "mlp.fc2.weight"), d, ff)) return rc;
        }
        wt_valid = true;
        return KD_OK;
    }

    // A[T, K] . Wt[K, N] for the T positions of the prompt. Up to kShortPrompt positions with N a
    // multiple of 64 and K of 32: rows padded to 64, K split so that the 64x64-tile grid holds up to
    // one workgroup per CU (GPT-2 small at T = 64: qkv 36 tiles x 6, proj 12 x 12, fc1 48 x 4,
    // fc2 12 x 16; measured against two and four per CU and against a half and three quarters of
    // the CUs: 0.79 ms for the 64-token prefill against 0.87, 0.94, 0.89 and 0.80), the partials
    // left for the epilogue to add; each product reads its weights once. Otherwise the backend's matmul path on rows padded to 128. Padding rows hold leftovers
    // of earlier rows; their products are ignored.
    int product(const float* A, const float* Wt, int64_t T, int64_t K, int64_t N, Product* out) const {
        const auto aligned = [](const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
        if (T <= kShortPrompt && N % 64 == 0 && K % 32 == 0 && aligned(A) && aligned(Wt)) {
            const int64_t rows = (T + 63) / 64 * 64;
            const int64_t tiles = rows / 64 * (N / 64);
            const int64_t steps = K / 32;
            int64_t splits = 1;
            for (int64_t c = 1; c <= steps; ++c)
                if (steps % c == 0 && tiles * c <= compute_units()) splits = c;
            *out = Product{pf_parts, splits, rows * N};
            return kd::matmul_split_parts(A, Wt, pf_parts, rows, N, K, K, N, splits);
        }
        kd_matmul_sizes sz{1, (T + 127) / 128 * 128, K, N};
        *out = Product{pf_p, 1, 0};
        return kd_matmul(KD_F32, A, Wt, pf_p, &sz);
    }

    template <int Epi>
    void epilogue(const Product& pr, const float* bias, float* out, int64_t T, int64_t N, float* kc, float* vc) const {
        const int64_t total = T * N;
        const int64_t blocks = std::min<int64_t>((total + kThreads - 1) / kThreads, int64_t{compute_units()} * 16);
        // partial loads in flight per element: the fewest of 4, 8, 16 that cover the splits (each
        // load past the last split repeats it: measured 0.5 us slower per launch at 4 splits with 16)
        const dim3 grid(static_cast<uint32_t>(blocks));
        if (pr.splits <= 4)
            hipLaunchKernelGGL((prefill_epilogue_kernel<Epi, 4>), grid, dim3(kThreads), 0, kd::stream(), pr.P, pr.splits,
                               pr.stride, bias, out, T, N, d, hd, cfg.max_positions, kc, vc);
        else if (pr.splits <= 8)
            hipLaunchKernelGGL((prefill_epilogue_kernel<Epi, 8>), grid, dim3(kThreads), 0, kd::stream(), pr.P, pr.splits,
                               pr.stride, bias, out, T, N, d, hd, cfg.max_positions, kc, vc);
        else
            hipLaunchKernelGGL((prefill_epilogue_kernel<Epi, kSplitBatch>), grid, dim3(kThreads), 0, kd::stream(), pr.P,
                               pr.splits, pr.stride, bias, out, T, N, d, hd, cfg.max_positions, kc, vc);
    }

    // Positions 0..T-1 of seq (already on the device) through every layer at once; then the
    // head and the greedy pick on position T - 1, which write seq[T] and leave st->pos = T.
    int batched_prefill(int64_t T) {
        if (int rc = ensure_prefill_buffers()) return rc;
        if (int rc = refresh_transposed()) return rc;
        hipStream_t s = kd::stream();
        Product pr{};
        const float divisor = static_cast<float>(std::sqrt(static_cast<double>(hd)));
        hipLaunchKernelGGL(prefill_embed_kernel, dim3(static_cast<uint32_t>(T)), dim3(kThreads), 0, s, seq,
                           p("token_embedding.weight"), p("position_embedding.weight"), pf_x, p("blocks.0.ln1.weight"),
                           p("blocks.0.ln1.bias"), pf_h, d);
        KD_LAUNCH_CHECK();
        // X += P + bias per row, then H = the next LayerNorm of X (none after the last block: the
        // head kernel normalises the last row itself)
        const auto residual = [&](const float* bias, const float* ln_w, const float* ln_b) {
            hipLaunchKernelGGL(prefill_residual_kernel, dim3(static_cast<uint32_t>(T)), dim3(kThreads), 0, s, pr.P, pr.splits,
                               pr.stride, bias, pf_x, ln_w, ln_b, pf_h, d);
        };
        for (int64_t l = 0; l < cfg.layers; ++l) {
            const std::string b = "blocks." + std::to_string(l) + ".";
            const std::string next = "blocks." + std::to_string(l + 1) + ".";
            const bool last = l + 1 == cfg.layers;
            float* kc = kcache + l * cfg.heads * cfg.max_positions * hd;
            float* vc = vcache + l * cfg.heads * cfg.max_positions * hd;
            if (int rc = product(pf_h, wt_qkv(l), T, d, 3 * d, &pr)) return rc;
            epilogue<kQkv>(pr, p(b + "attn.qkv.bias"), pf_q, T, 3 * d, kc, vc);
            hipLaunchKernelGGL(prefill_attention_kernel, dim3(static_cast<uint32_t>(cfg.heads), static_cast<uint32_t>(T)),
                               dim3(kThreads), static_cast<size_t>(T) * sizeof(float), s, pf_q, kc, vc, pf_a, d, hd,
                               cfg.max_positions, divisor);
            if (int rc = product(pf_a, wt_proj(l), T, d, d, &pr)) return rc;
            residual(p(b + "attn.proj.bias"), p(b + "ln2.weight"), p(b + "ln2.bias"));
            if (int rc = product(pf_h, wt_fc1(l), T, d, ff, &pr)) return rc;
            if (cfg.tanh_gelu) epilogue<kGeluTanh>(pr, p(b + "mlp.fc1.bias"), pf_f, T, ff, nullptr, nullptr);
            else epilogue<kGeluExact>(pr, p(b + "mlp.fc1.bias"), pf_f, T, ff, nullptr, nullptr);
            if (int rc = product(pf_f, wt_fc2(l), T, ff, d, &pr)) return rc;
            residual(p(b + "mlp.fc2.bias"), last ? nullptr : p(next + "ln1.weight"), last ? nullptr : p(next + "ln1.bias"));
            KD_LAUNCH_CHECK();
        }
        GemvArgs head = base();
        head.W = p("token_embedding.weight");
        head.x = pf_x + (T - 1) * d;
        head.ln_w = p("ln_final.weight");
        head.ln_b = p("ln_final.bias");
        head.N = cfg.vocab_size;
        head.K = d;
        head.out = logits;
        head.best_v = pv;
        head.best_i = pi;
        head.sp = sp;
        head.keys = keys;
        head.key_parts = key_parts;
        const int64_t parts = head_groups();
        hipLaunchKernelGGL(head_kernel, dim3(static_cast<uint32_t>(parts)), dim3(kThreads), 0, s, head);
        hipLaunchKernelGGL(pick_kernel, dim3(1), dim3(kPickThreads), 0, s, pick_args());
        KD_LAUNCH_CHECK();
        KD_HIP(hipStreamSynchronize(s));
        host_pos = T;
        return KD_OK;
    }

    // Runs the last min(history, max_positions) tokens of the history from position 0 with an
    // empty cache and appends the greedy token they produce: the prompt, and kael's cache refill
    // once the sequence has outgrown the context (reference src/nn/transformer.cpp:270-284:
    // with a full cache every step clears it and reruns the window).
    int run_window() {
        const int64_t n = static_cast<int64_t>(history.size());
        const int64_t window = std::min(n, cfg.max_positions);
        KD_HIP(hipMemcpyAsync(seq, history.data() + (n - window), static_cast<size_t>(window) * sizeof(int64_t),
                              hipMemcpyHostToDevice, stream));
        if (stepwise_prefill()) {
            if (int rc = set_state(0, window)) return rc;
            if (int rc = steps(window)) return rc;
        } else {
            // the pick after the batched layers runs as the step of position window - 1
            if (int rc = set_state(window - 1, window)) return rc;
            if (int rc = batched_prefill(window)) return rc;
        }
        int64_t next = 0;
        KD_HIP(hipMemcpyAsync(&next, seq + window, sizeof next, hipMemcpyDeviceToHost, stream));
        KD_HIP(hipStreamSynchronize(stream));
        history.push_back(next);
        return KD_OK;
    }

    // After picks in sampling mode: the error a pick recorded, if any.
    int check_sampler() {
        if (host_sp.top_k == 0) return KD_OK;
        Sampler now{};
        KD_HIP(hipMemcpy(&now, sp, sizeof now, hipMemcpyDeviceToHost));
        if (now.error == 1) return fail(KD_E_INVALID, "kd_gpt: a sampled pick met a non-finite logit");
        if (now.error == 2)
            return fail(KD_E_INVALID, "kd_gpt: a sampled pick found no uniform draw left (kd_gpt_set_uniforms)");
        return KD_OK;
    }

    // `count` tokens (greedy, or sampled as set by kd_gpt_set_sampling): cached single-token
    // steps while the cache has room, then one window rerun per token.
    int generate(int64_t count) {
        int64_t produced = 0;
        while (produced < count) {
            if (host_pos < cfg.max_positions) {
                const int64_t n = std::min(count - produced, cfg.max_positions - host_pos);
                const int64_t first = host_pos + 1;  // index in seq of the first token these steps produce
                if (int rc = steps(n)) return rc;
                const size_t old = history.size();
                history.resize(old + static_cast<size_t>(n));
                KD_HIP(hipMemcpyAsync(history.data() + old, seq + first, static_cast<size_t>(n) * sizeof(int64_t),
                                      hipMemcpyDeviceToHost, stream));
                KD_HIP(hipStreamSynchronize(stream));
                produced += n;
            } else {
                if (int rc = run_window()) return rc;
                ++produced;
            }
        }
        return KD_OK;
    }

    ~Engine() {
        if (graph) (void)hipGraphExecDestroy(graph);
        for (void* ptr : {static_cast<void*>(pf_x), static_cast<void*>(pf_h), static_cast<void*>(pf_q),
                          static_cast<void*>(pf_a), static_cast<void*>(pf_f), static_cast<void*>(pf_p), static_cast<void*>(pf_parts),
                          static_cast<void*>(wt)})
            if (ptr) (void)hipFree(ptr);
        for (void* ptr : {static_cast<void*>(params), static_cast<void*>(kcache), static_cast<void*>(vcache),
                          static_cast<void*>(x), static_cast<void*>(q), static_cast<void*>(partials.m),
                          static_cast<void*>(partials.l), static_cast<void*>(partials.acc),
                          static_cast<void*>(f), static_cast<void*>(logits), static_cast<void*>(pv),
                          static_cast<void*>(pi), static_cast<void*>(seq), static_cast<void*>(st),
                          static_cast<void*>(sp), static_cast<void*>(uniforms), static_cast<void*>(kept),
                          static_cast<void*>(kept_e), static_cast<void*>(keys), static_cast<void*>(key_parts)})
            if (ptr) (void)hipFree(ptr);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

template <typename T> int alloc(T** out, int64_t count) {
    void* p = nullptr;
    KD_HIP(hipMalloc(&p, static_cast<size_t>(count) * sizeof(T)));
    *out = static_cast<T*>(p);
    return KD_OK;
}

// The shapes this engine's kernels handle (KD_OK) or the reason they do not.
int check_config(const kd_gpt_config& c) {
    if (c.vocab_size <= 0 || c.max_positions <= 0 || c.layers <= 0 || c.heads <= 0 || c.dimension <= 0)
        return fail(KD_E_INVALID, "kd_gpt: sizes must be positive");
    if (c.dimension % c.heads != 0) return fail(KD_E_INVALID, "kd_gpt: dimension must divide by heads");
    const int64_t hd = c.dimension / c.heads;
    if (hd > 64) return fail(KD_E_UNSUPPORTED, "kd_gpt: head_dim above 64 is not supported");
    if (c.dimension % 4 != 0) return fail(KD_E_UNSUPPORTED, "kd_gpt: dimension must be a multiple of 4");
    if (hd % 4 != 0) return fail(KD_E_UNSUPPORTED, "kd_gpt: head_dim must be a multiple of 4 (16-byte key rows)");
    if (4 * c.dimension > kMaxK) return fail(KD_E_UNSUPPORTED, "kd_gpt: 4 * dimension above 4096 is not supported");
    static_assert(kMaxK / 4 <= kMaxLnDim, "ln_load holds a row of at most kMaxLnDim elements");
    if (c.heads > kMaxHeads) return fail(KD_E_UNSUPPORTED, "kd_gpt: more than 64 heads is not supported");
    if (c.max_positions > 8192) return fail(KD_E_UNSUPPORTED, "kd_gpt: max_positions above 8192");
    if ((c.flags & ~(KD_GPT_EAGER | KD_GPT_STEPWISE_PREFILL)) != 0) return fail(KD_E_INVALID, "kd_gpt: unknown flags");
    return KD_OK;
}

int create(Engine& e, const kd_gpt_config& c) {
    if (int rc = check_config(c)) return rc;
    e.cfg = c;
    e.d = c.dimension;
    e.hd = c.dimension / c.heads;
    e.ff = 4 * c.dimension;
    // kael's parameter order and shapes (GPT::named_parameters; Linear weights [out, in])
    std::vector<std::pair<std::string, std::vector<int64_t>>> shapes;
    shapes.emplace_back("token_embedding.weight", std::vector<int64_t>{c.vocab_size, e.d});
    shapes.emplace_back("position_embedding.weight", std::vector<int64_t>{c.max_positions, e.d});
    for (int64_t l = 0; l < c.layers; ++l) {
        const std::string b = "blocks." + std::to_string(l) + ".";
        shapes.emplace_back(b + "ln1.weight", std::vector<int64_t>{e.d});
        shapes.emplace_back(b + "ln1.bias", std::vector<int64_t>{e.d});
        shapes.emplace_back(b + "attn.qkv.weight", std::vector<int64_t>{3 * e.d, e.d});
        shapes.emplace_back(b + "attn.qkv.bias", std::vector<int64_t>{3 * e.d});
        shapes.emplace_back(b + "attn.proj.weight", std::vector<int64_t>{e.d, e.d});
        shapes.emplace_back(b + "attn.proj.bias", std::vector<int64_t>{e.d});
        shapes.emplace_back(b + "ln2.weight", std::vector<int64_t>{e.d});
        shapes.emplace_back(b + "ln2.bias", std::vector<int64_t>{e.d});
        shapes.emplace_back(b + "mlp.fc1.weight", std::vector<int64_t>{e.ff, e.d});
        shapes.emplace_back(b + "mlp.fc1.bias", std::vector<int64_t>{e.ff});
        shapes.emplace_back(b + "mlp.fc2.weight", std::vector<int64_t>{e.d, e.ff});
        shapes.emplace_back(b + "mlp.fc2.bias", std::vector<int64_t>{e.d});
    }
    shapes.emplace_back("ln_final.weight", std::vector<int64_t>{e.d});
    shapes.emplace_back("ln_final.bias", std::vector<int64_t>{e.d});
    int64_t total = 0;
    for (const auto& [name, shape] : shapes) {
        int64_t count = 1;
        for (const int64_t s : shape) count *= s;
        e.offsets[name] = {total, count};
        e.shape_of[name] = shape;
        e.names.push_back(name);
        total += (count + 63) / 64 * 64;  // keep every parameter 256-byte aligned
    }
    e.loaded.assign(shapes.size(), false);
    KD_HIP(hipStreamCreateWithFlags(&e.stream, hipStreamNonBlocking));
    if (int rc = alloc(&e.params, total)) return rc;
    const int64_t cache = c.layers * c.heads * c.max_positions * e.hd;
    if (int rc = alloc(&e.kcache, cache)) return rc;
    if (int rc = alloc(&e.vcache, cache)) return rc;
    if (int rc = alloc(&e.x, e.d)) return rc;
    if (int rc = alloc(&e.q, e.d)) return rc;
    if (int rc = alloc(&e.partials.m, c.heads * kAttnChunks)) return rc;
    if (int rc = alloc(&e.partials.l, c.heads * kAttnChunks)) return rc;
    if (int rc = alloc(&e.partials.acc, c.heads * kAttnChunks * e.hd)) return rc;
    if (int rc = alloc(&e.f, e.ff)) return rc;
    if (int rc = alloc(&e.logits, c.vocab_size)) return rc;
    if (int rc = alloc(&e.pv, e.head_groups())) return rc;
    if (int rc = alloc(&e.pi, e.head_groups())) return rc;

    if (int rc = alloc(&e.seq, c.max_positions + 1)) return rc;
    if (int rc = alloc(&e.st, 1)) return rc;
    if (int rc = alloc(&e.sp, 1)) return rc;
    if (int rc = alloc(&e.uniforms, c.max_positions + 1)) return rc;
    if (int rc = alloc(&e.kept, c.vocab_size)) return rc;
    if (int rc = alloc(&e.kept_e, c.vocab_size)) return rc;
    if (int rc = alloc(&e.keys, int64_t{kPickSlots} * kPickThreads)) return rc;
    KD_HIP(hipMemset(e.keys, 0, size_t{kPickSlots} * kPickThreads * sizeof(uint32_t)));  // past the vocabulary: 0
    if (int rc = alloc(&e.key_parts, 2 * e.head_groups())) return rc;
    KD_HIP(hipMemcpy(e.sp, &e.host_sp, sizeof(Sampler), hipMemcpyHostToDevice));  // greedy
    return KD_OK;
}

// Copies one parameter into the engine from host or device memory.
int load_parameter(const char* what, void* handle, const char* name, const float* data, int64_t count, bool on_device) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || name == nullptr || data == nullptr) return fail(KD_E_INVALID, std::string(what) + ": null argument");
    const auto it = e->offsets.find(name);
    if (it == e->offsets.end()) return fail(KD_E_INVALID, std::string(what) + ": unknown parameter " + name);
    if (it->second.second != count) return fail(KD_E_INVALID, std::string(what) + ": wrong element count for " + name);
    const size_t bytes = static_cast<size_t>(count) * sizeof(float);
    if (on_device) {
        // Ordered after the work already queued on the backend stream (which produced `data`).
        KD_HIP(hipStreamSynchronize(kd::stream()));
        KD_HIP(hipMemcpyAsync(e->params + it->second.first, data, bytes, hipMemcpyDeviceToDevice, e->stream));
        KD_HIP(hipStreamSynchronize(e->stream));
    } else {
        KD_HIP(hipMemcpy(e->params + it->second.first, data, bytes, hipMemcpyHostToDevice));
    }
    for (size_t i = 0; i < e->names.size(); ++i)
        if (e->names[i] == name) e->loaded[i] = true;
    e->wt_valid = false;
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

extern "C" {

int kd_gpt_create(void** handle, const kd_gpt_config* config) {
    if (handle == nullptr || config == nullptr) return fail(KD_E_INVALID, "kd_gpt_create: null argument");
    *handle = nullptr;
    if (int rc = ensure_device()) return rc;
    auto* e = new Engine();
    if (int rc = create(*e, *config)) {
        delete e;
        return rc;
    }
    *handle = e;
    return KD_OK;
}

int kd_gpt_supported(const kd_gpt_config* config) {
    if (config == nullptr) return fail(KD_E_INVALID, "kd_gpt_supported: null argument");
    if (int rc = ensure_device()) return rc;
    return check_config(*config);
}

void kd_gpt_destroy(void* handle) { delete static_cast<Engine*>(handle); }

int kd_gpt_load_parameter(void* handle, const char* name, const float* data, int64_t count) {
    return load_parameter("kd_gpt_load_parameter", handle, name, data, count, false);
}

int kd_gpt_load_parameter_device(void* handle, const char* name, const float* data, int64_t count) {
    return load_parameter("kd_gpt_load_parameter_device", handle, name, data, count, true);
}

int kd_gpt_load_safetensors(void* handle, const char* path) {
    namespace st = kd::safetensors;
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || path == nullptr) return fail(KD_E_INVALID, "kd_gpt_load_safetensors: null argument");
    std::string error;
    bool unsupported = false;
    const auto file = st::File::open(path, &error, &unsupported);
    if (!file) return fail(unsupported ? KD_E_UNSUPPORTED : KD_E_INVALID, "kd_gpt_load_safetensors: " + error);
    // kael's name of each stored tensor; entries kael's GPT does not have are ignored, and of two
    // that translate to one name the first in name order is kept (load_gpt2_weights' emplace)
    std::unordered_map<std::string, const st::Entry*> found;
    for (const st::Entry& entry : file->entries()) {
        const std::string name = st::translated_gpt2_name(entry.name);
        if (e->offsets.count(name) != 0) found.emplace(name, &entry);
    }
    const auto shape_text = [](const std::vector<int64_t>& s) {
        std::string t = "[";
        for (size_t i = 0; i < s.size(); ++i) t += (i ? ", " : "") + std::to_string(s[i]);
        return t + "]";
    };
    // every parameter present with kael's shape before any is copied (Module::load_state_dict)
    for (const std::string& name : e->names) {
        const auto it = found.find(name);
        if (it == found.end()) return fail(KD_E_INVALID, "kd_gpt_load_safetensors: state dict is missing parameter " + name);
        std::vector<int64_t> shape = it->second->shape;
        if (st::stored_transposed(name) && shape.size() == 2) std::swap(shape[0], shape[1]);
        if (shape != e->shape_of.at(name))
            return fail(KD_E_INVALID, "kd_gpt_load_safetensors: parameter " + name + " has shape " +
                                          shape_text(e->shape_of.at(name)) + " but the state dict has " + shape_text(shape));
    }
    std::vector<float> values;
    for (const std::string& name : e->names) {
        const st::Entry& entry = *found.at(name);
        values.resize(static_cast<size_t>(entry.numel()));
        file->to_f32(entry, values.data(), st::stored_transposed(name) && entry.shape.size() == 2);
        if (int rc = load_parameter("kd_gpt_load_safetensors", handle, name.c_str(), values.data(), entry.numel(), false))
            return rc;
    }
    return KD_OK;
}

int kd_safetensors_tensor(const char* path, const char* name, float* out, int64_t capacity, int64_t* shape,
                          int32_t* dims) {
    namespace st = kd::safetensors;
    if (path == nullptr || name == nullptr || dims == nullptr) return fail(KD_E_INVALID, "kd_safetensors_tensor: null argument");
    std::string error;
    bool unsupported = false;
    const auto file = st::File::open(path, &error, &unsupported);
    if (!file) return fail(unsupported ? KD_E_UNSUPPORTED : KD_E_INVALID, "kd_safetensors_tensor: " + error);
    const st::Entry* entry = file->find(name);
    if (entry == nullptr) return fail(KD_E_INVALID, std::string("kd_safetensors_tensor: no tensor named ") + name);
    if (entry->shape.size() > KD_MAX_DIMS) return fail(KD_E_UNSUPPORTED, "kd_safetensors_tensor: more than 8 dims");
    *dims = static_cast<int32_t>(entry->shape.size());
    if (shape != nullptr)
        for (size_t i = 0; i < entry->shape.size(); ++i) shape[i] = entry->shape[i];
    if (out == nullptr) return KD_OK;  // size query
    if (capacity < entry->numel()) return fail(KD_E_INVALID, "kd_safetensors_tensor: output holds fewer elements than the tensor");
    file->to_f32(*entry, out, false);
    return KD_OK;
}

int kd_gpt_prefill(void* handle, const int64_t* prompt, int64_t length) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || prompt == nullptr || length <= 0) return fail(KD_E_INVALID, "kd_gpt_prefill: bad arguments");
    for (int64_t i = 0; i < length; ++i)
        if (prompt[i] < 0 || prompt[i] >= e->cfg.vocab_size) return fail(KD_E_INVALID, "kd_gpt_prefill: token id out of range");
    if (int rc = e->ready()) return rc;
    e->history.assign(prompt, prompt + length);
    if (int rc = e->run_window()) return rc;
    return e->check_sampler();
}

int kd_gpt_decode(void* handle, int64_t count, int64_t* tokens) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || count < 0) return fail(KD_E_INVALID, "kd_gpt_decode: bad arguments");
    if (e->history.empty()) return fail(KD_E_INVALID, "kd_gpt_decode: call kd_gpt_prefill first");
    if (int rc = e->generate(count)) return rc;
    if (int rc = e->check_sampler()) return rc;
    if (tokens != nullptr && count > 0)
        std::memcpy(tokens, e->history.data() + e->history.size() - count, static_cast<size_t>(count) * sizeof(int64_t));
    return KD_OK;
}

int kd_gpt_forward_logits(void* handle, const int64_t* tokens, int64_t count, float* logits) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || tokens == nullptr || logits == nullptr || count <= 0)
        return fail(KD_E_INVALID, "kd_gpt_forward_logits: bad arguments");
    if (count > e->cfg.max_positions) return fail(KD_E_INVALID, "kd_gpt_forward_logits: more tokens than max_positions");
    if (e->host_sp.top_k > 0) return fail(KD_E_INVALID, "kd_gpt_forward_logits: needs the greedy pick (temperature 0)");
    for (int64_t i = 0; i < count; ++i)
        if (tokens[i] < 0 || tokens[i] >= e->cfg.vocab_size) return fail(KD_E_INVALID, "kd_gpt_forward_logits: token id out of range");
    if (int rc = e->ready()) return rc;
    KD_HIP(hipMemcpyAsync(e->seq, tokens, static_cast<size_t>(count) * sizeof(int64_t), hipMemcpyHostToDevice, e->stream));
    if (int rc = e->set_state(0, count)) return rc;
    const int64_t v = e->cfg.vocab_size;
    for (int64_t t = 0; t < count; ++t) {
        if (int rc = e->steps(1)) return rc;
        KD_HIP(hipMemcpyAsync(logits + t * v, e->logits, static_cast<size_t>(v) * sizeof(float), hipMemcpyDeviceToHost, e->stream));
    }
    // the tokens, then the greedy token the last position produced
    e->history.assign(tokens, tokens + count);
    e->history.push_back(0);
    KD_HIP(hipMemcpyAsync(&e->history.back(), e->seq + count, sizeof(int64_t), hipMemcpyDeviceToHost, e->stream));
    KD_HIP(hipStreamSynchronize(e->stream));
    return KD_OK;
}

int kd_gpt_sequence(void* handle, int64_t* ids, int64_t capacity, int64_t* length) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || length == nullptr) return fail(KD_E_INVALID, "kd_gpt_sequence: bad arguments");
    const int64_t n = static_cast<int64_t>(e->history.size());
    *length = n;
    if (ids != nullptr && capacity > 0 && n > 0)
        std::memcpy(ids, e->history.data(), static_cast<size_t>(std::min(n, capacity)) * sizeof(int64_t));
    return KD_OK;
}

int kd_gpt_set_sampling(void* handle, double temperature, int64_t top_k) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || !(temperature >= 0.0) || top_k < 0)
        return fail(KD_E_INVALID, "kd_gpt_set_sampling: needs a temperature >= 0 and top_k >= 0");
    if (temperature > 0.0 && e->cfg.vocab_size > KD_GPT_SAMPLE_MAX_VOCAB)
        return fail(KD_E_UNSUPPORTED, "kd_gpt_set_sampling: sampling on the device takes vocabularies of at most "
                                      "KD_GPT_SAMPLE_MAX_VOCAB (65536) entries");
    const float t = static_cast<float>(temperature);
    if (temperature > 0.0 && !(t > 0.f && std::isfinite(t)))
        return fail(KD_E_INVALID, "kd_gpt_set_sampling: the temperature does not round to a positive finite float");
    KD_HIP(hipStreamSynchronize(e->stream));
    KD_HIP(hipStreamSynchronize(kd::stream()));
    // top_k 0 or >= the vocabulary: kael masks nothing, which keeping all vocab_size entries restates
    const int64_t keep = top_k == 0 || top_k >= e->cfg.vocab_size ? e->cfg.vocab_size : top_k;
    e->host_sp = Sampler{t, 0, temperature > 0.0 ? keep : 0, 0, 0};
    KD_HIP(hipMemcpy(e->sp, &e->host_sp, sizeof(Sampler), hipMemcpyHostToDevice));
    return KD_OK;
}

int kd_gpt_set_uniforms(void* handle, const double* uniforms, int64_t count) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || count < 0 || (count > 0 && uniforms == nullptr))
        return fail(KD_E_INVALID, "kd_gpt_set_uniforms: bad arguments");
    if (count > e->cfg.max_positions + 1)
        return fail(KD_E_INVALID, "kd_gpt_set_uniforms: more draws than max_positions + 1 at once");
    for (int64_t i = 0; i < count; ++i)
        if (!(uniforms[i] >= 0.0 && uniforms[i] < 1.0))
            return fail(KD_E_INVALID, "kd_gpt_set_uniforms: every draw must lie in [0, 1)");
    KD_HIP(hipStreamSynchronize(e->stream));
    KD_HIP(hipStreamSynchronize(kd::stream()));
    if (count > 0)
        KD_HIP(hipMemcpy(e->uniforms, uniforms, static_cast<size_t>(count) * sizeof(double), hipMemcpyHostToDevice));
    e->host_sp.draw = 0;
    e->host_sp.draws = count;
    e->host_sp.error = 0;
    KD_HIP(hipMemcpy(e->sp, &e->host_sp, sizeof(Sampler), hipMemcpyHostToDevice));
    return KD_OK;
}

int kd_gpt_draws_used(void* handle, int64_t* used) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || used == nullptr) return fail(KD_E_INVALID, "kd_gpt_draws_used: bad arguments");
    KD_HIP(hipStreamSynchronize(e->stream));
    KD_HIP(hipStreamSynchronize(kd::stream()));
    Sampler now{};
    KD_HIP(hipMemcpy(&now, e->sp, sizeof now, hipMemcpyDeviceToHost));
    *used = now.draw;
    return KD_OK;
}

int kd_gpt_logits(void* handle, float* logits) {
    auto* e = static_cast<Engine*>(handle);
    if (e == nullptr || logits == nullptr) return fail(KD_E_INVALID, "kd_gpt_logits: bad arguments");
    if (e->history.empty()) return fail(KD_E_INVALID, "kd_gpt_logits: no position has been run");
    KD_HIP(hipStreamSynchronize(e->stream));
    KD_HIP(hipMemcpy(logits, e->logits, static_cast<size_t>(e->cfg.vocab_size) * sizeof(float), hipMemcpyDeviceToHost));
    return KD_OK;
}

} // extern "C"
