// kd_kael_init.cpp - the parameters of kael's GPT as its constructor initialises them, on the host.
//
// Reference: kael::manual_seed(seed) (src/random.cpp:62-65), then GPT::GPT
// (src/nn/transformer.cpp:167-184) and GPT::initialize_weights (:186-207). kael draws everything
// from one std::mt19937_64, in module construction order:
//   - each Embedding constructor fills its table with randn (src/nn/layers.cpp:70-73);
//   - each Linear constructor fills its weight with kaiming_uniform_(sqrt 5) and its bias with a
//     fan-in uniform (src/nn/layers.cpp:17-40; src/nn/init.cpp:30-33, 61-64), one rand draw per
//     element; LayerNorm, GELU and Dropout draw nothing;
//   - initialize_weights redraws both tables and every block weight as randn * std (std 0.02, or
//     0.02 / sqrt(2 layers) for attn.proj and mlp.fc2), sets block biases to zero and keeps the
//     LayerNorm ones and zeros.
// kael::randn (src/random.cpp:86-88) uses a fresh std::normal_distribution<double>(0, 1) per
// tensor (a pair left over at its end is dropped) and kael::rand a fresh
// std::uniform_real_distribution<double>(0, 1); this file draws through the same standard library
// types in the same order (the constructor's draws that initialize_weights overwrites included, so
// the stream stays aligned), hence kael's values wherever both use the same standard library.
// normal_ rounds as kael's f32 tensor ops do: (float)draw * (float)std, then + (float)0.
#include <cmath>
#include <cstring>
#include <random>
#include <string>

#include "kd_api.h"

namespace kd {
int fail(int status, const std::string& message);
}

namespace {

void draw_normal(std::mt19937_64& engine, float* out, int64_t count, double std) {
#pragma clang fp contract(off)
    std::normal_distribution<double> normal(0.0, 1.0);
    const float scale = static_cast<float>(std);
    const float mean = 0.0f;
    for (int64_t i = 0; i < count; ++i) {
        const float product = static_cast<float>(normal(engine)) * scale;
        if (out != nullptr) out[i] = product + mean;
    }
}

void draw_uniform(std::mt19937_64& engine, int64_t count) {
    std::uniform_real_distribution<double> uniform(0.0, 1.0);
    for (int64_t i = 0; i < count; ++i) (void)uniform(engine);
}

void fill(float* out, int64_t count, float value) {
    for (int64_t i = 0; i < count; ++i) out[i] = value;
}

} // namespace

extern "C" int kd_gpt_kael_init(const kd_gpt_config* config, uint64_t seed, float* params, int64_t capacity,
                                int64_t* count) {
    using kd::fail;
    if (config == nullptr || count == nullptr) return fail(KD_E_INVALID, "kd_gpt_kael_init: null argument");
    const kd_gpt_config& c = *config;
    if (c.vocab_size <= 0 || c.max_positions <= 0 || c.layers <= 0 || c.heads <= 0 || c.dimension <= 0 ||
        c.dimension % c.heads != 0)
        return fail(KD_E_INVALID, "kd_gpt_kael_init: sizes must be positive and dimension divisible by heads");
    const int64_t d = c.dimension, ff = 4 * c.dimension, V = c.vocab_size, P = c.max_positions, L = c.layers;
    const int64_t block = 2 * d + 3 * d * d + 3 * d + d * d + d + 2 * d + ff * d + ff + d * ff + d;
    const int64_t total = V * d + P * d + L * block + 2 * d;
    *count = total;
    if (params == nullptr) return KD_OK;
    if (capacity < total) return fail(KD_E_INVALID, "kd_gpt_kael_init: capacity below the parameter count");

    std::mt19937_64 engine(seed);
    // GPT::GPT: the two Embedding tables, then each block's Linear layers (qkv, proj, fc1, fc2:
    // weight, then bias).
    draw_normal(engine, nullptr, V * d, 1.0);
    draw_normal(engine, nullptr, P * d, 1.0);
    for (int64_t l = 0; l < L; ++l) {
        for (const auto& [in, out] : {std::pair{d, 3 * d}, {d, d}, {d, ff}, {ff, d}}) {
            draw_uniform(engine, out * in);
            draw_uniform(engine, out);
        }
    }
    // initialize_weights, writing GPT::named_parameters() order.
    const double std = 0.02;
    const double residual_std = std / std::sqrt(2.0 * static_cast<double>(L));
    float* p = params;
    draw_normal(engine, p, V * d, std);  // token_embedding.weight
    p += V * d;
    draw_normal(engine, p, P * d, std);  // position_embedding.weight
    p += P * d;
    for (int64_t l = 0; l < L; ++l) {
        fill(p, d, 1.0f);  // ln1.weight
        fill(p + d, d, 0.0f);
        p += 2 * d;
        draw_normal(engine, p, 3 * d * d, std);  // attn.qkv
        fill(p + 3 * d * d, 3 * d, 0.0f);
        p += 3 * d * d + 3 * d;
        draw_normal(engine, p, d * d, residual_std);  // attn.proj
        fill(p + d * d, d, 0.0f);
        p += d * d + d;
        fill(p, d, 1.0f);  // ln2
        fill(p + d, d, 0.0f);
        p += 2 * d;
        draw_normal(engine, p, ff * d, std);  // mlp.fc1
        fill(p + ff * d, ff, 0.0f);
        p += ff * d + ff;
        draw_normal(engine, p, d * ff, residual_std);  // mlp.fc2
        fill(p + d * ff, d, 0.0f);
        p += d * ff + d;
    }
    fill(p, d, 1.0f);  // ln_final
    fill(p + d, d, 0.0f);
    return KD_OK;
}
