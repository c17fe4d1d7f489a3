// kd_random.hip - kael's bernoulli masks and dropout drawn on the device from kael's generator.
//
// Reference: kael::bernoulli (src/random.cpp:106-110) is (rand(shape, F64) < p).to(dtype), where
// rand draws one std::uniform_real_distribution<double>(0, 1) value per element from the global
// std::mt19937_64 (src/random.cpp:66-84); kael::nn::functional::dropout (src/nn/functional.cpp:32-39)
// is input * bernoulli(shape, keep, dtype) / keep, each op rounded to the element type, the scalar
// `keep` converted to it. kael draws the mask on the host and copies it over; here the draws, the
// compare and the two element ops run in one launch, and the generator state comes back advanced
// by exactly `count` draws, so the caller's later draws continue kael's stream.
//
// The state is passed as libstdc++ streams a mersenne_twister_engine (operator<<): the 312 state
// words, then the index of the next word to temper (0..312).
//
// MT19937-64 (Matsumoto and Nishimura; the C++ standard's mt19937_64 parameters). The state is
// regenerated 312 words at a time (a twist): new word k mixes old words k and k + 1 into
// y = (upper bit of old[k]) | (lower 31 bits of old[k + 1]) and is
// old[k + 156] ^ (y >> 1) ^ (y odd ? A : 0) for k < 156, and new[k - 156] ^ ... for k >= 156 (word
// 311 takes new word 0 as its second input), so a twist is two parallel phases of 156 words. A
// draw is the tempered next word x; libstdc++'s generate_canonical<double, 53> over a 64-bit engine
// uses one word and returns double(x) / 2^64 (the conversion rounded to nearest), or the largest
// double below 1 when that rounds up to 1; uniform_real_distribution(0, 1) returns it unchanged.
//
// Device layout: draw e is element e. The draws split into blocks that follow the twists: block 0
// is what is left of the current state (words pos..311), block j >= 1 the 312 words of the j-th
// twist. Every workgroup runs the twist chain in LDS (two barriers per 312 draws) and handles the
// blocks j with j % gridDim.x == blockIdx.x: it tempers their words, compares, and loads and
// stores their elements, the input of its next block loaded one block ahead. The memory traffic is
// spread over the chip; only the cheap chain is serial. The workgroup of the last block writes the
// final state to a second buffer (others may still be reading the first).
#include "kd_internal.h"

namespace kd {

namespace {

constexpr int kWords = 312;
constexpr int kShift = 156;
constexpr uint64_t kMatrixA = 0xB5026F5AA96619E9ull;
constexpr uint64_t kUpperMask = 0xFFFFFFFF80000000ull;  // the top 33 bits
constexpr uint64_t kLowerMask = 0x000000007FFFFFFFull;  // the low 31 bits
constexpr int kRngThreads = 320;                         // 312 words, rounded up to whole waves

__host__ __device__ __forceinline__ uint64_t twist_word(uint64_t first, uint64_t second, uint64_t far) {
    const uint64_t y = (first & kUpperMask) | (second & kLowerMask);
    return far ^ (y >> 1) ^ ((y & 1) ? kMatrixA : 0);
}

__device__ __forceinline__ uint64_t temper(uint64_t x) {
    x ^= (x >> 29) & 0x5555555555555555ull;
    x ^= (x << 17) & 0x71D67FFFEDA60000ull;
    x ^= (x << 37) & 0xFFF7EEE000000000ull;
    x ^= x >> 43;
    return x;
}

// generate_canonical<double, 53>: one 64-bit word, double(x) * 2^-64, kept below 1.
__device__ __forceinline__ double canonical(uint64_t x) {
    const double u = static_cast<double>(x) * 0x1p-64;
    return u >= 1.0 ? 0x1.fffffffffffffp-1 : u;
}

template <typename T> __device__ __forceinline__ T dropped(T x, bool keep, T keep_t);
template <> __device__ __forceinline__ float dropped<float>(float x, bool keep, float keep_t) {
    return __fdiv_rn(__fmul_rn(x, keep ? 1.0f : 0.0f), keep_t);
}
template <> __device__ __forceinline__ double dropped<double>(double x, bool keep, double keep_t) {
    return __ddiv_rn(__dmul_rn(x, keep ? 1.0 : 0.0), keep_t);
}

struct RngArgs {
    void* out;
    void* mask;          // dropout: the mask as T(1) / T(0) too, or nullptr
    const void* in;      // dropout input (nullptr for a mask)
    const uint64_t* state;  // device copy: 312 words, then the position
    uint64_t* next;         // the state after the draws, same layout
    int64_t count;
    int64_t blocks;      // blocks of draws (block 0: the rest of the current state)
    int64_t first;       // draws in block 0
    double p;            // the compare threshold (keep for dropout)
};

// Dropout = true: out = in * (u < p) / T(p) (and mask = T(u < p) when asked for). Dropout = false:
// out = T(u < p).
template <typename T, bool Dropout>
__global__ __launch_bounds__(kRngThreads) void mt_kernel(RngArgs a, T keep_t) {
    __shared__ uint64_t mt[2][kWords];
    const int t = threadIdx.x;
    if (t < kWords) mt[0][t] = a.state[t];
    const int64_t pos = static_cast<int64_t>(a.state[kWords]);
    int cur = 0;
    const int64_t G = gridDim.x;
    const int64_t mine = static_cast<int64_t>(blockIdx.x);
    // element range of block j
    auto start = [&](int64_t j) { return j == 0 ? int64_t{0} : a.first + (j - 1) * kWords; };
    auto size = [&](int64_t j) {
        return j == 0 ? a.first : std::min<int64_t>(kWords, a.count - start(j));
    };
    const T* in = static_cast<const T*>(a.in);
    T* out = static_cast<T*>(a.out);
    T* mask = static_cast<T*>(a.mask);
    // the input of this workgroup's next block, loaded a block ahead
    T x = T(0);
    if constexpr (Dropout) {
        if (mine < a.blocks && t < size(mine)) x = in[start(mine) + t];
    }
    const int64_t last = a.blocks - 1;
    const int64_t own_last = mine <= last ? last - (last - mine) % G : -1;  // this workgroup's last block
    __syncthreads();
    for (int64_t j = 0; j <= own_last; ++j) {
        if (j > 0) {
            const uint64_t* old = mt[cur];
            uint64_t* nw = mt[cur ^ 1];
            if (t < kShift) nw[t] = twist_word(old[t], old[t + 1], old[t + kShift]);
            __syncthreads();
            if (t >= kShift && t < kWords) {
                const uint64_t second = t + 1 < kWords ? old[t + 1] : nw[0];
                nw[t] = twist_word(old[t], second, nw[t - kShift]);
            }
            __syncthreads();
            cur ^= 1;
        }
        if (j % G == mine) {
            const int64_t n = size(j);
            const int64_t word = j == 0 ? pos : 0;
            const int64_t e = start(j) + t;
            T xn = T(0);
            if constexpr (Dropout) {
                const int64_t next = j + G;
                if (next <= last && t < size(next)) xn = in[start(next) + t];
            }
            if (t < n) {
                const bool hit = canonical(temper(mt[cur][word + t])) < a.p;
                if constexpr (Dropout) {
                    out[e] = dropped<T>(x, hit, keep_t);
                    if (mask != nullptr) mask[e] = hit ? T(1) : T(0);
                } else {
                    out[e] = hit ? T(1) : T(0);
                }
            }
            x = xn;
        }
    }
    if (mine == last % G) {
        // state after the last draw: the current words and the index past the last one used
        if (t < kWords) a.next[t] = mt[cur][t];
        if (t == 0) a.next[kWords] = static_cast<uint64_t>(last == 0 ? pos + a.first : size(last));
    }
}

template <typename T, bool Dropout>
int run_rng(void* out, void* mask, const void* in, int64_t count, double p, uint64_t* host_state) {
    const int64_t pos = static_cast<int64_t>(host_state[kWords]);
    RngArgs a{};
    a.out = out;
    a.mask = mask;
    a.in = in;
    a.count = count;
    a.first = std::min<int64_t>(kWords - pos, count);
    a.blocks = 1 + (count - a.first + kWords - 1) / kWords;
    a.p = p;
    Workspace lease;
    if (int rc = workspace(lease, 2 * (kWords + 1) * sizeof(uint64_t))) return rc;
    uint64_t* dev_state = static_cast<uint64_t*>(lease.ptr);
    a.state = dev_state;
    a.next = dev_state + kWords + 1;
    hipStream_t s = stream();
    KD_HIP(hipMemcpyAsync(dev_state, host_state, (kWords + 1) * sizeof(uint64_t), hipMemcpyHostToDevice, s));
    // Enough workgroups that each handles a few blocks, at most two per CU.
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(a.blocks, 2 * int64_t{compute_units()}));
    hipLaunchKernelGGL((mt_kernel<T, Dropout>), dim3(static_cast<uint32_t>(grid)), dim3(kRngThreads), 0, s, a,
                       static_cast<T>(p));
    KD_LAUNCH_CHECK();
    KD_HIP(hipMemcpyAsync(host_state, a.next, (kWords + 1) * sizeof(uint64_t), hipMemcpyDeviceToHost, s));
    KD_HIP(hipStreamSynchronize(s));
    return KD_OK;
}

int check_state(const uint64_t* state, const char* what) {
    if (state == nullptr) return fail(KD_E_INVALID, std::string(what) + ": null generator state");
    if (state[kWords] > kWords)
        return fail(KD_E_INVALID, std::string(what) + ": generator position " + std::to_string(state[kWords]) +
                                      " outside [0, 312]");
    return KD_OK;
}

} // namespace

} // namespace kd

using namespace kd;

extern "C" void kd_mt19937_64_seed(uint64_t* state, uint64_t seed) {
    // std::mt19937_64(seed): x0 = seed, x_i = f * (x_{i-1} ^ (x_{i-1} >> 62)) + i, position 312 (the
    // first draw twists).
    state[0] = seed;
    for (int i = 1; i < kWords; ++i)
        state[i] = 6364136223846793005ull * (state[i - 1] ^ (state[i - 1] >> 62)) + static_cast<uint64_t>(i);
    state[kWords] = kWords;
}

extern "C" int kd_bernoulli(int dtype, void* out, int64_t count, double probability, uint64_t* state) {
    if (count < 0) return fail(KD_E_INVALID, "kd_bernoulli: negative count");
    if (!(probability >= 0.0 && probability <= 1.0))
        return fail(KD_E_INVALID, "kd_bernoulli: probability must be in [0, 1]");
    if (dtype_size(dtype) == 0) return fail(KD_E_INVALID, "kd_bernoulli: unknown dtype");
    if (int rc = check_state(state, "kd_bernoulli")) return rc;
    if (count == 0) return KD_OK;
    if (out == nullptr) return fail(KD_E_INVALID, "kd_bernoulli: null output");
    if (int rc = ensure_device()) return rc;
    switch (dtype) {
    case KD_F32: return run_rng<float, false>(out, nullptr, nullptr, count, probability, state);
    case KD_F64: return run_rng<double, false>(out, nullptr, nullptr, count, probability, state);
    case KD_I64: return run_rng<int64_t, false>(out, nullptr, nullptr, count, probability, state);
    default: return run_rng<uint8_t, false>(out, nullptr, nullptr, count, probability, state);
    }
}

extern "C" int kd_dropout(int dtype, void* out, void* mask, const void* in, int64_t count, double keep,
                          uint64_t* state) {
    if (count < 0) return fail(KD_E_INVALID, "kd_dropout: negative count");
    if (!(keep > 0.0 && keep <= 1.0)) return fail(KD_E_INVALID, "kd_dropout: keep probability must be in (0, 1]");
    if (dtype != KD_F32 && dtype != KD_F64) return fail(KD_E_INVALID, "kd_dropout: dtype must be f32 or f64");
    if (int rc = check_state(state, "kd_dropout")) return rc;
    if (count == 0) return KD_OK;
    if (out == nullptr || in == nullptr) return fail(KD_E_INVALID, "kd_dropout: null operand");
    if (int rc = ensure_device()) return rc;
    return dtype == KD_F32 ? run_rng<float, true>(out, mask, in, count, keep, state)
                           : run_rng<double, true>(out, mask, in, count, keep, state);
}
