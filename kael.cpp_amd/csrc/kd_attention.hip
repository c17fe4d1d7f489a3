// kd_attention.hip - kael's causal self-attention (reference src/nn/transformer.cpp:103-138: the
// fused projection's output viewed [B, T, 3, H, D], q / k / v selected and transposed per head,
// softmax(mask(q . k^T / sqrt(D))) . v, the heads merged back to [B, T, H * D]) as one kernel
// forward and one backward, for f32 and D = 64, without a KV cache or dropout.
//
// Forward: one workgroup of four waves per (batch, head, block of 32 queries); wave w walks key
// blocks w, w + 4, ... up to the diagonal: S^T = K_J . Q_I^T on v_mfma_f32_32x32x2f32 (each lane then holds 16 scores
// of one query: lane (li, lh), register r is key 8 (r / 4) + 4 lh + r % 4 of query li), the
// scale and the causal mask, an online softmax per query (running max and sum, the output
// rescaled when the max grows), and O^T += V_J^T . P^T, whose B operand is the score register
// itself. The waves' (max, sum, output) meet in LDS and merge as the online softmax would; the
// output is written in the merged-head layout and the row's log-sum-exp m + log(l) is kept for
// the backward.
//
// Backward (the gradient of every op of kael's chain: the products, the scale, the mask and
// softmax backward y (g - sum(g y))): with delta_i = sum_d dO[i][d] O[i][d] (= sum_j P dP over
// the row) and P recomputed from the log-sum-exp, dS = P (dP - delta) / sqrt(D), one launch of two
// kinds of workgroup:
//   dQ groups, one per (batch, head, query block): delta, then for each key block S^T,
//     dP^T = V_J . dO_I^T, dS^T, and dQ += dS . K_J;
//   dK / dV groups, one per (batch, head, key block): for each query block at or after it delta,
//     S, dP = dO_I . V_J^T, dS, dV += P^T . dO_I and dK += dS^T . Q_I;
//   the four waves split the blocks they walk and add their partial sums in wave order.
// Every MFMA sums over 64 features (or 32 keys / queries) with the operands' features split as
// k-pairs (s, 32 + s), which is a reordering of the same sum. The softmax exponentials use the
// hardware exp2 (__expf: a few ulp), well inside the device tolerance kael's tests apply.
#include <algorithm>
#include <cmath>

#include "kd_internal.h"

namespace kd {

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kD = 64;      // head dim
constexpr int kBlock = 32;  // queries / keys per block

__device__ __forceinline__ v16f mfma(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v16f zero16() {
    v16f z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.f;
    return z;
}

// Row of block position 8 (s / 4) + 4 lh + s % 4: the k index of MFMA step s in the products
// whose k runs over a block of 32 (the score registers' layout).
__device__ __forceinline__ int block_row(int s, int lh) { return 8 * (s / 4) + 4 * lh + (s % 4); }

struct AttentionShape {
    int batch, length, heads;
    int64_t row;  // qkv elements per token: 3 * heads * D
    int64_t out_row;  // merged-head elements per token: heads * D
    float inv_scale;  // 1 / sqrt(D) = 1 / 8: kael divides by sqrt(D) = 8, and x * 0.125 equals x / 8 exactly
};

// ---- work split and LDS tiles --------------------------------------------------------------
//
// A workgroup is 4 waves on one block of 32 rows: the forward and dQ groups on a query block,
// wave w taking key blocks w, w + 4, ... up to the diagonal; a dK / dV group on a key block, wave w
// taking query blocks kb + w, kb + w + 4, ... Workgroups run longest first (the last query blocks,
// the first key blocks), with all (batch, head) pairs interleaved so that every XCD gets its share of
// each length.
//
// Every global load reads whole rows, 16 bytes per lane and four 256-byte rows per instruction:
// a lane-per-row operand loaded directly would touch 64 cache lines per instruction, and those
// loads made up the largest part of a wave's time. The block all four waves share (the query rows,
// or a dK / dV group's key rows) is loaded a quarter per wave into a shared LDS tile behind one
// workgroup barrier; the blocks a wave walks pass through an LDS tile of its own (rows padded to 68
// floats), so the waves never wait for each other inside the loop: a wave issues every global load
// of its first block at once, keeps the next block's loads in flight in registers while it computes
// the current one, and orders its own LDS writes and reads with wave-level fences only. At the end
// the waves' partial results meet in LDS behind one workgroup barrier and are combined in wave
// order: the forward's (max, sum, output) triples as an online-softmax merge, the gradients as sums.

constexpr int kWaves = 4;
constexpr int kLd = kD + 4;           // padded LDS row
constexpr int kTile = kBlock * kLd;   // one 32-row tile
constexpr int kTileVec = kBlock * kD / 4 / 64;  // 16-byte pieces of a tile per lane

// Orders a wave's LDS accesses across its lanes: a wave's LDS operations execute in issue order,
// so it only has to keep the compiler from moving them across this point.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Floats 4 c4 .. 4 c4 + 3 of row `row` of a [T, D] head matrix (row stride ld), zeros for a row past
// the last: the load reads the last row instead, so no load needs a branch.
__device__ __forceinline__ v4f row_piece(const float* __restrict__ base, int row, int length, int64_t ld, int c4) {
    const v4f x = *reinterpret_cast<const v4f*>(base + static_cast<int64_t>(min(row, length - 1)) * ld + 4 * c4);
    return row < length ? x : v4f{0.f, 0.f, 0.f, 0.f};
}

// Rows t0 .. t0 + 31 of a [T, D] head matrix (row stride ld) into registers, 16 bytes per load,
// zeros past the last row; tile_store writes them to a wave's LDS tile.
__device__ __forceinline__ void tile_load(v4f (&reg)[kTileVec], const float* __restrict__ base, int t0, int length,
                                          int64_t ld, int lane) {
#pragma unroll
    for (int q = 0; q < kTileVec; ++q) {
        const int idx = lane + 64 * q;
        const int row = idx / (kD / 4), c4 = idx % (kD / 4);
        reg[q] = row_piece(base, t0 + row, length, ld, c4);
    }
}

__device__ __forceinline__ void tile_store(float* __restrict__ tile, const v4f (&reg)[kTileVec], int lane) {
#pragma unroll
    for (int q = 0; q < kTileVec; ++q) {
        const int idx = lane + 64 * q;
        const int row = idx / (kD / 4), c4 = idx % (kD / 4);
        *reinterpret_cast<v4f*>(tile + row * kLd + 4 * c4) = reg[q];
    }
}

// Row `row` (features 32 * lh .. 32 * lh + 31) of a wave's LDS tile.
__device__ __forceinline__ void lds_half_row(float (&reg)[32], const float* __restrict__ tile, int row, int lh) {
    const v4f* src = reinterpret_cast<const v4f*>(tile + row * kLd + 32 * lh);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const v4f v = src[q];
        reg[4 * q] = v[0];
        reg[4 * q + 1] = v[1];
        reg[4 * q + 2] = v[2];
        reg[4 * q + 3] = v[3];
    }
}

// A 32 x 64 accumulator pair acc[dt][r] = X[block_row(r, lh)][32 dt + li] into an LDS tile.
__device__ __forceinline__ void spill_pair(float* __restrict__ tile, const v16f (&acc)[2], int li, int lh) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        tile[block_row(r, lh) * kLd + li] = acc[0][r];
        tile[block_row(r, lh) * kLd + 32 + li] = acc[1][r];
    }
}

// Rows 8 w .. 8 w + 7 of the sum of the 4 waves' tiles (in wave order) stored to dst rows r0 + row
// (row stride ld) below `length`: each lane 8 consecutive elements of one row.
__device__ __forceinline__ void store_tile_sum(float* __restrict__ dst, const float* __restrict__ tiles, int r0,
                                               int length, int64_t ld, int wave, int lane) {
    const int row = 8 * wave + lane / 8, c0 = 8 * (lane % 8);
    if (r0 + row >= length) return;
    float acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = tiles[row * kLd + c0 + c];
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[c] += tiles[w * kTile + row * kLd + c0 + c];
    float* out = dst + static_cast<int64_t>(r0 + row) * ld + c0;
    *reinterpret_cast<v4f*>(out) = v4f{acc[0], acc[1], acc[2], acc[3]};
    *reinterpret_cast<v4f*>(out + 4) = v4f{acc[4], acc[5], acc[6], acc[7]};
}

// A wave's quarter (rows 8 wave .. 8 wave + 7) of rows t0 .. t0 + 31 of a [T, D] head matrix, 16
// bytes per load and 4 whole rows per instruction, zeros past the last row: the four waves load a
// block that all of them read together, and part_store puts it in a workgroup-shared tile.
constexpr int kPartVec = kTileVec / kWaves;

__device__ __forceinline__ void part_load(v4f (&reg)[kPartVec], const float* __restrict__ base, int t0, int length,
                                          int64_t ld, int wave, int lane) {
#pragma unroll
    for (int q = 0; q < kPartVec; ++q) {
        const int row = 8 * wave + 4 * q + lane / (kD / 4), c4 = lane % (kD / 4);
        reg[q] = row_piece(base, t0 + row, length, ld, c4);
    }
}

__device__ __forceinline__ void part_store(float* __restrict__ tile, const v4f (&reg)[kPartVec], int wave, int lane) {
#pragma unroll
    for (int q = 0; q < kPartVec; ++q) {
        const int row = 8 * wave + 4 * q + lane / (kD / 4), c4 = lane % (kD / 4);
        *reinterpret_cast<v4f*>(tile + row * kLd + 4 * c4) = reg[q];
    }
}

// x of this lane and of lane ^ 32, in some order: v_permlane32_swap exchanges lanes 0-31 of one copy
// with lanes 32-63 of the other, so every lane holds its own value in one result and its partner's in
// the other. Their max or sum is the same in both halves (either order gives the same float).
__device__ __forceinline__ void both_halves(float x, float& a, float& b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    a = __uint_as_float(p[0]);
    b = __uint_as_float(p[1]);
}

__device__ __forceinline__ float halves_max(float x) {
    float a, b;
    both_halves(x, a, b);
    return fmaxf(a, b);
}

__device__ __forceinline__ float halves_sum(float x) {
    float a, b;
    both_halves(x, a, b);
    return a + b;
}

// X^T . Y^T over 64 features in two independent MFMA chains (even and odd k-pairs), added at the
// end: a[t] / b[t] hold features t and 32 + t of the lane's row (half lh).
__device__ __forceinline__ v16f dot_rows(const float (&a)[32], const float (&b)[32]) {
    v16f s0 = zero16(), s1 = zero16();
#pragma unroll
    for (int t = 0; t < 32; t += 2) {
        s0 = mfma(a[t], b[t], s0);
        s1 = mfma(a[t + 1], b[t + 1], s1);
    }
    return s0 + s1;
}

// ---- forward -----------------------------------------------------------------------------

__global__ __launch_bounds__(kWaves * 64, 2) void attention_forward_kernel(float* __restrict__ out, float* __restrict__ lse,
                                                                           const float* __restrict__ qkv,
                                                                           AttentionShape sh) {
    __shared__ float tiles[kWaves * kTile];  // each wave's K, then V, tile of its current key block
    __shared__ float qtile[kTile];           // the query block
    __shared__ float ms[kWaves][kBlock], ls[kWaves][kBlock];
    const int blocks = (sh.length + kBlock - 1) / kBlock;
    const int units = sh.batch * sh.heads;
    const int bh = static_cast<int>(blockIdx.x % units);
    const int qb = blocks - 1 - static_cast<int>(blockIdx.x / units);  // longest rows first, all heads interleaved
    const int b = bh / sh.heads, h = bh % sh.heads;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, li = lane % 32, lh = lane / 32;
    const float* q = qkv + static_cast<int64_t>(b) * sh.length * sh.row + h * kD;
    const float* k = q + sh.heads * kD;
    const float* v = k + sh.heads * kD;
    float* tile = tiles + wave * kTile;
    const int query = qb * kBlock + li;

    // every load in flight together: the wave's quarter of the query block, its first K and V tiles
    v4f qpart[kPartVec], kload[kTileVec], vload[kTileVec];
    part_load(qpart, q, qb * kBlock, sh.length, sh.row, wave, lane);
    if (wave <= qb) {
        tile_load(kload, k, wave * kBlock, sh.length, sh.row, lane);
        tile_load(vload, v, wave * kBlock, sh.length, sh.row, lane);
    }
    part_store(qtile, qpart, wave, lane);
    __syncthreads();
    float qreg[32];
    lds_half_row(qreg, qtile, li, lh);
    v16f o[2] = {zero16(), zero16()};
    float m = -INFINITY, l = 0.f;
    for (int kb = wave; kb <= qb; kb += kWaves) {
        const int j0 = kb * kBlock;
        float kreg[32];
        tile_store(tile, kload, lane);  // K of this block (the previous block's reads are done)
        wave_sync();
        lds_half_row(kreg, tile, li, lh);
        wave_sync();
        tile_store(tile, vload, lane);  // then V in its place: a wave's LDS operations run in issue order
        wave_sync();
        const bool more = kb + kWaves <= qb;
        if (more) {  // the next block's loads run while this block computes
            tile_load(kload, k, j0 + kWaves * kBlock, sh.length, sh.row, lane);
            tile_load(vload, v, j0 + kWaves * kBlock, sh.length, sh.row, lane);
        }
        v16f s = dot_rows(kreg, qreg);
        // scale, mask, block max of this query's scores (16 here, 16 in lane li + 32)
        float bmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = j0 + block_row(r, lh);
            const float x = (key > query || key >= sh.length) ? -INFINITY : s[r] * sh.inv_scale;
            s[r] = x;
            bmax = fmaxf(bmax, x);
        }
        bmax = halves_max(bmax);
        const float mnew = fmaxf(m, bmax);
        const float alpha = mnew == -INFINITY ? 1.f : __expf(m - mnew);
        float bsum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float p = s[r] == -INFINITY ? 0.f : __expf(s[r] - mnew);
            s[r] = p;
            bsum += p;
        }
        bsum = halves_sum(bsum);
        l = l * alpha + bsum;
        m = mnew;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        }
        // O^T[d][i] += sum_j V[j][d] P[i][j]: A = V^T (lane li: feature 32 dt + li), B = P^T
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float* vr = tile + block_row(t, lh) * kLd + li;
            o[0] = mfma(vr[0], s[t], o[0]);
            o[1] = mfma(vr[32], s[t], o[1]);
        }
        wave_sync();
    }
    // merge: o[dt][r] = O^T[32 dt + block_row(r, lh)][query li] of this wave's key blocks
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        tile[li * kLd + 32 * 0 + block_row(r, lh)] = o[0][r];
        tile[li * kLd + 32 * 1 + block_row(r, lh)] = o[1][r];
    }
    if (lh == 0) {
        ms[wave][li] = m;
        ls[wave][li] = l;
    }
    __syncthreads();
    // wave w finishes queries 8 w .. 8 w + 7, each lane 8 features of one of them
    const int row = 8 * wave + lane / 8, c0 = 8 * (lane % 8);
    const int t = qb * kBlock + row;
    if (t < sh.length) {
        float mx = ms[0][row];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, ms[w][row]);
        float total = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float f = ms[w][row] == -INFINITY ? 0.f : __expf(ms[w][row] - mx);
            total += f * ls[w][row];
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] += f * tiles[w * kTile + row * kLd + c0 + c];
        }
        const float inv = 1.f / total;
        float* dst = out + (static_cast<int64_t>(b) * sh.length + t) * sh.out_row + h * kD + c0;
        *reinterpret_cast<v4f*>(dst) = v4f{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
        *reinterpret_cast<v4f*>(dst + 4) = v4f{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
        if (lane % 8 == 0) lse[static_cast<int64_t>(bh) * sh.length + t] = mx + logf(total);
    }
}

// ---- backward ----------------------------------------------------------------------------
//
// One launch holds both kinds of workgroup: first the dK / dV groups (a key block each, the longer
// ones), then the dQ groups (a query block each). Each computes the delta of the query rows it
// needs, with the same expression, so neither waits for the other.

// delta of one query row, sum_d dO[d] O[d]: each half's 32 products summed in order, then the halves.
__device__ __forceinline__ float row_delta(const float (&g)[32], const float (&o)[32]) {
    float part = 0.f;
#pragma unroll
    for (int t = 0; t < 32; ++t) part += g[t] * o[t];
    return halves_sum(part);
}

// The dQ group `group`: lds holds 7 tiles.
__device__ __forceinline__ void dq_group(int group, float* __restrict__ lds, float* __restrict__ dqkv,
                                         const float* __restrict__ dout, const float* __restrict__ qkv,
                                         const float* __restrict__ out, const float* __restrict__ lse,
                                         const AttentionShape& sh) {
    float* tiles = lds;                   // each wave's V, then K, tile of its current key block
    float* rows[3] = {lds + kWaves * kTile, lds + (kWaves + 1) * kTile, lds + (kWaves + 2) * kTile};  // Q, dO, O
    const int blocks = (sh.length + kBlock - 1) / kBlock;
    const int units = sh.batch * sh.heads;
    const int bh = group % units;
    const int qb = blocks - 1 - group / units;
    const int b = bh / sh.heads, h = bh % sh.heads;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, li = lane % 32, lh = lane / 32;
    const int64_t tok0 = static_cast<int64_t>(b) * sh.length;
    const float* q = qkv + tok0 * sh.row + h * kD;
    const float* k = q + sh.heads * kD;
    const float* v = k + sh.heads * kD;
    const float* go = dout + tok0 * sh.out_row + h * kD;
    const float* o = out + tok0 * sh.out_row + h * kD;
    float* tile = tiles + wave * kTile;
    const int i0 = qb * kBlock;
    const int query = i0 + li;

    // every load in flight together: the wave's quarter of the query block's Q, dO and O, its first
    // K and V tiles
    v4f qpart[kPartVec], gpart[kPartVec], opart[kPartVec], kload[kTileVec], vload[kTileVec];
    part_load(qpart, q, i0, sh.length, sh.row, wave, lane);
    part_load(gpart, go, i0, sh.length, sh.out_row, wave, lane);
    part_load(opart, o, i0, sh.length, sh.out_row, wave, lane);
    const float row_lse = query < sh.length ? lse[static_cast<int64_t>(bh) * sh.length + query] : 0.f;
    if (wave <= qb) {
        tile_load(kload, k, wave * kBlock, sh.length, sh.row, lane);
        tile_load(vload, v, wave * kBlock, sh.length, sh.row, lane);
    }
    part_store(rows[0], qpart, wave, lane);
    part_store(rows[1], gpart, wave, lane);
    part_store(rows[2], opart, wave, lane);
    __syncthreads();
    float qreg[32], doreg[32];
    lds_half_row(qreg, rows[0], li, lh);
    lds_half_row(doreg, rows[1], li, lh);
    float dl;
    {
        float oreg[32];
        lds_half_row(oreg, rows[2], li, lh);
        dl = row_delta(doreg, oreg);
    }

    v16f dq[2] = {zero16(), zero16()};
    for (int kb = wave; kb <= qb; kb += kWaves) {
        const int j0 = kb * kBlock;
        v16f dp, s;
        {
            float vreg[32];
            tile_store(tile, vload, lane);  // V of this block (the previous block's reads are done)
            wave_sync();
            lds_half_row(vreg, tile, li, lh);
            wave_sync();
            tile_store(tile, kload, lane);  // then K in its place: a wave's LDS operations run in issue order
            wave_sync();
            dp = dot_rows(vreg, doreg);
        }
        {
            float kreg[32];
            lds_half_row(kreg, tile, li, lh);
            s = dot_rows(kreg, qreg);  // the forward's product, term for term
        }
        if (kb + kWaves <= qb) {  // the next block's loads run while this block finishes
            tile_load(kload, k, j0 + kWaves * kBlock, sh.length, sh.row, lane);
            tile_load(vload, v, j0 + kWaves * kBlock, sh.length, sh.row, lane);
        }
        // s[r] = S[query][key], dp[r] = dP[query][key] for key j0 + block_row(r, lh)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = j0 + block_row(r, lh);
            const bool live = key <= query && key < sh.length && query < sh.length;
            const float p = live ? __expf(s[r] * sh.inv_scale - row_lse) : 0.f;
            s[r] = p * (dp[r] - dl) * sh.inv_scale;
        }
        // dQ[i][d] += sum_j dS[i][j] K[j][d]: A = dS (lane li: query li), B = K (feature 32 dt + li)
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float* kr = tile + block_row(t, lh) * kLd + li;
            dq[0] = mfma(s[t], kr[0], dq[0]);
            dq[1] = mfma(s[t], kr[32], dq[1]);
        }
        wave_sync();
    }
    // dq[dt][r] = dQ[i0 + block_row(r, lh)][32 dt + li]: the waves' partial sums, added in wave order
    spill_pair(tile, dq, li, lh);
    __syncthreads();
    store_tile_sum(dqkv + tok0 * sh.row + h * kD, tiles, i0, sh.length, sh.row, wave, lane);
}

// The dK / dV group `group`: lds holds 9 tiles and 2 x 4 rows of 32.
__device__ __forceinline__ void dkv_group(int group, float* __restrict__ lds, float* __restrict__ dqkv,
                                          const float* __restrict__ dout, const float* __restrict__ qkv,
                                          const float* __restrict__ out, const float* __restrict__ lse,
                                          const AttentionShape& sh) {
    float* tiles = lds;                        // each wave's Q (O first) and dO tiles; the first holds K at the start
    float* vtile = lds + 2 * kWaves * kTile;   // the key block's V
    float (*lses)[kBlock] = reinterpret_cast<float (*)[kBlock]>(vtile + kTile);
    float (*deltas)[kBlock] = lses + kWaves;
    const int blocks = (sh.length + kBlock - 1) / kBlock;
    const int units = sh.batch * sh.heads;
    const int bh = group % units;
    const int kb = group / units;  // key block 0 has the most query blocks: first
    const int b = bh / sh.heads, h = bh % sh.heads;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, li = lane % 32, lh = lane / 32;
    const int64_t tok0 = static_cast<int64_t>(b) * sh.length;
    const float* q = qkv + tok0 * sh.row + h * kD;
    const float* k = q + sh.heads * kD;
    const float* v = k + sh.heads * kD;
    const float* go = dout + tok0 * sh.out_row + h * kD;
    const float* o = out + tok0 * sh.out_row + h * kD;
    const float* row_lse = lse + static_cast<int64_t>(bh) * sh.length;
    float* qtile = tiles + wave * kTile;
    float* gtile = tiles + (kWaves + wave) * kTile;
    const int j0 = kb * kBlock;
    const int key = j0 + li;

    v4f kpart[kPartVec], vpart[kPartVec], qload[kTileVec], gload[kTileVec], oload[kTileVec];
    float lload = 0.f;
    // every load in flight together: the wave's quarter of the key block's K and V, and the wave's
    // first query block (Q, dO, O and log-sum-exp rows)
    part_load(kpart, k, j0, sh.length, sh.row, wave, lane);
    part_load(vpart, v, j0, sh.length, sh.row, wave, lane);
    const auto load_query_block = [&](int i0) {
        tile_load(qload, q, i0, sh.length, sh.row, lane);
        tile_load(gload, go, i0, sh.length, sh.out_row, lane);
        tile_load(oload, o, i0, sh.length, sh.out_row, lane);
        if (lane < kBlock) lload = i0 + lane < sh.length ? row_lse[i0 + lane] : 0.f;
    };
    if (kb + wave < blocks) load_query_block((kb + wave) * kBlock);
    // K passes through the first tile, which wave 0 reuses only after the second barrier; V stays in
    // LDS (read again for every query block, which leaves the registers to the products)
    part_store(tiles, kpart, wave, lane);
    part_store(vtile, vpart, wave, lane);
    __syncthreads();
    float kreg[32];
    lds_half_row(kreg, tiles, li, lh);
    __syncthreads();

    v16f dk[2] = {zero16(), zero16()}, dv[2] = {zero16(), zero16()};
    const auto block_products = [&](int i0) {
        tile_store(qtile, oload, lane);  // O first, for the rows' delta (the previous block's reads are done)
        tile_store(gtile, gload, lane);
        if (lane < kBlock) lses[wave][lane] = lload;
        wave_sync();
        {
            float greg[32], oreg[32];
            lds_half_row(greg, gtile, li, lh);
            lds_half_row(oreg, qtile, li, lh);
            const float dl = row_delta(greg, oreg);
            if (lh == 0) deltas[wave][li] = dl;
        }
        wave_sync();
        tile_store(qtile, qload, lane);  // then Q in its place: a wave's LDS operations run in issue order
        wave_sync();
        v16f s, dp;
        {
            float qreg[32];
            lds_half_row(qreg, qtile, li, lh);
            s = dot_rows(qreg, kreg);
        }
        {
            float doreg[32], vreg[32];
            lds_half_row(doreg, gtile, li, lh);
            lds_half_row(vreg, vtile, li, lh);
            dp = dot_rows(doreg, vreg);
        }
        // s[r] = S[query][key], dp[r] = dP[query][key] for query i0 + block_row(r, lh), key li
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int local = block_row(r, lh);
            const int query = i0 + local;
            const bool live = key <= query && query < sh.length && key < sh.length;
            p[r] = live ? __expf(s[r] * sh.inv_scale - lses[wave][local]) : 0.f;
            s[r] = p[r] * (dp[r] - deltas[wave][local]) * sh.inv_scale;
        }
        // dV[j][d] += sum_i P[i][j] dO[i][d], dK[j][d] += sum_i dS[i][j] Q[i][d]:
        // A = P^T / dS^T (lane li: key li), B = dO / Q (feature 32 dt + li)
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int off = block_row(t, lh) * kLd + li;
            dv[0] = mfma(p[t], gtile[off], dv[0]);
            dv[1] = mfma(p[t], gtile[off + 32], dv[1]);
            dk[0] = mfma(s[t], qtile[off], dk[0]);
            dk[1] = mfma(s[t], qtile[off + 32], dk[1]);
        }
        wave_sync();
    };
    // the first query block's loads were issued before the barriers; each later one's just before use
    // (loads kept in flight across a block would need registers the products use)
    if (kb + wave < blocks) {
        block_products((kb + wave) * kBlock);
        for (int qb = kb + wave + kWaves; qb < blocks; qb += kWaves) {
            load_query_block(qb * kBlock);
            block_products(qb * kBlock);
        }
    }
    // dk / dv[dt][r] = dK / dV[j0 + block_row(r, lh)][32 dt + li]: partial sums added in wave order
    spill_pair(qtile, dk, li, lh);
    spill_pair(gtile, dv, li, lh);
    __syncthreads();
    float* dstk = dqkv + tok0 * sh.row + sh.heads * kD + h * kD;
    store_tile_sum(dstk, tiles, j0, sh.length, sh.row, wave, lane);
    store_tile_sum(dstk + sh.heads * kD, tiles + kWaves * kTile, j0, sh.length, sh.row, wave, lane);
}

constexpr int kBackwardLds = (2 * kWaves + 1) * kTile + 2 * kWaves * kBlock;  // the dK / dV group's, the larger

__global__ __launch_bounds__(kWaves * 64, 2) void attention_backward_kernel(float* __restrict__ dqkv,
                                                                            const float* __restrict__ dout,
                                                                            const float* __restrict__ qkv,
                                                                            const float* __restrict__ out,
                                                                            const float* __restrict__ lse,
                                                                            AttentionShape sh) {
    __shared__ float lds[kBackwardLds];
    const int groups = sh.batch * sh.heads * ((sh.length + kBlock - 1) / kBlock);
    const int i = static_cast<int>(blockIdx.x);
    if (i < groups)
        dkv_group(i, lds, dqkv, dout, qkv, out, lse, sh);
    else
        dq_group(i - groups, lds, dqkv, dout, qkv, out, lse, sh);
}

// ---- attention of new queries against a KV cache -------------------------------------------------
//
// kael's CausalSelfAttention::forward with a cache (generation): `length` new queries at positions
// past .. past + length - 1 against the keys and values of positions 0 .. keys - 1 (past = keys -
// length), query t seeing keys 0 .. past + t. The operands are read in place through their strides
// (kael's per-head views of the fused projection and its concatenated cache tensors), features
// contiguous. A workgroup per (batch, head, query); wave w walks key groups w, w + waves, ... of 32
// keys. A lane holds one feature: every key row is one coalesced 256-byte load, and the 32 lanes'
// products of a group reduce in a butterfly (5 halving exchanges, then one add) that leaves key
// (lane / 2)'s score in lanes 2j and 2j + 1. The online softmax runs per group (running max and
// sum, the output rescaled when the max grows), each lane accumulating its feature of the output
// over the group's keys in key order; the waves' (max, sum, output) merge in LDS in wave order.
// Decode has few (batch, head) rows, so a workgroup then takes 16 waves.

struct CachedShape {
    int batch, heads, length, keys;
    int64_t qs[3], ks[3], vs[3];  // strides (batch, head, position) in elements
};

constexpr int kCachedGroup = 32;
constexpr int kCachedMaxWaves = 16;

// The 2N values x of every lane summed pairwise with lane ^ D's: a lane whose bit D is set keeps
// the upper N sums, the other the lower N.
template <int N, int D>
__device__ __forceinline__ void butterfly_step(const float (&x)[2 * N], float (&y)[N], int lane) {
    const bool upper = (lane & D) != 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float send = upper ? x[i] : x[N + i];
        const float keep = upper ? x[N + i] : x[i];
        y[i] = keep + __shfl_xor(send, D);
    }
}

__global__ __launch_bounds__(kCachedMaxWaves * 64) void cached_attention_kernel(float* __restrict__ out,
                                                                                const float* __restrict__ q,
                                                                                const float* __restrict__ k,
                                                                                const float* __restrict__ v,
                                                                                CachedShape sh) {
    __shared__ float ms[kCachedMaxWaves], ls[kCachedMaxWaves];
    __shared__ float os[kCachedMaxWaves][kD];
    const int waves = static_cast<int>(blockDim.x) / 64;
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int row = static_cast<int>(blockIdx.x);
    const int t = row % sh.length, h = (row / sh.length) % sh.heads, b = row / (sh.length * sh.heads);
    const int limit = sh.keys - sh.length + t + 1;  // keys 0 .. limit - 1 are visible
    const float qd = q[b * sh.qs[0] + h * sh.qs[1] + t * sh.qs[2] + lane];
    const float* kb = k + b * sh.ks[0] + h * sh.ks[1] + lane;
    const float* vb = v + b * sh.vs[0] + h * sh.vs[1] + lane;
    const int groups = (limit + kCachedGroup - 1) / kCachedGroup;
    float m = -INFINITY, l = 0.f, o = 0.f;
    for (int g = wave; g < groups; g += waves) {
        const int j0 = g * kCachedGroup;
        float x[32], vr[32];
#pragma unroll
        for (int jj = 0; jj < 32; ++jj) {
            const int64_t j = min(j0 + jj, limit - 1);  // a key past the limit reads the last visible row, masked below
            x[jj] = kb[j * sh.ks[2]];
            vr[jj] = vb[j * sh.vs[2]];
        }
#pragma unroll
        for (int jj = 0; jj < 32; ++jj) x[jj] *= qd;
        float y16[16], y8[8], y4[4], y2[2], y1[1];
        butterfly_step<16, 32>(x, y16, lane);
        butterfly_step<8, 16>(y16, y8, lane);
        butterfly_step<4, 8>(y8, y4, lane);
        butterfly_step<2, 4>(y4, y2, lane);
        butterfly_step<1, 2>(y2, y1, lane);
        // lanes 2j and 2j + 1 hold the two halves of key j0 + j's sum: every lane now has the score
        float s = y1[0] + __shfl_xor(y1[0], 1);
        s = j0 + lane / 2 < limit ? s * 0.125f : -INFINITY;  // 1 / sqrt(64), exact
        float gmax = s;
#pragma unroll
        for (int d = 2; d < 64; d *= 2) gmax = fmaxf(gmax, __shfl_xor(gmax, d));
        const float mnew = fmaxf(m, gmax);
        const float alpha = mnew == -INFINITY ? 1.f : __expf(m - mnew);
        const float p = s == -INFINITY ? 0.f : __expf(s - mnew);
        float gsum = p;  // each key once: the lanes that differ in bits 1-5
#pragma unroll
        for (int d = 2; d < 64; d *= 2) gsum += __shfl_xor(gsum, d);
        l = l * alpha + gsum;
        o *= alpha;
#pragma unroll
        for (int jj = 0; jj < 32; ++jj)
            o += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 2 * jj)) * vr[jj];
        m = mnew;
    }
    if (lane == 0) {
        ms[wave] = m;
        ls[wave] = l;
    }
    os[wave][lane] = o;
    __syncthreads();
    if (wave == 0) {
        float mx = -INFINITY;
        for (int w = 0; w < waves; ++w) mx = fmaxf(mx, ms[w]);
        float total = 0.f, acc = 0.f;
        for (int w = 0; w < waves; ++w) {
            const float f = ms[w] == -INFINITY ? 0.f : __expf(ms[w] - mx);
            total += f * ls[w];
            acc += f * os[w][lane];
        }
        out[((static_cast<int64_t>(b) * sh.length + t) * sh.heads + h) * kD + lane] = acc / total;
    }
}

int check_shape(int dtype, int64_t batch, int64_t length, int64_t heads, int64_t head_dim, AttentionShape& sh,
                const char* what) {
    if (dtype != KD_F32) return fail(KD_E_UNSUPPORTED, std::string(what) + ": dtype must be f32");
    if (head_dim != kD) return fail(KD_E_UNSUPPORTED, std::string(what) + ": head dim must be 64");
    if (batch < 1 || length < 1 || heads < 1) return fail(KD_E_INVALID, std::string(what) + ": empty shape");
    const int64_t blocks = (length + kBlock - 1) / kBlock;
    const int64_t row = 3 * heads * kD;
    if (2 * batch * heads * blocks >= (int64_t{1} << 31) || length * row >= (int64_t{1} << 31) || batch > INT32_MAX)
        return fail(KD_E_INVALID, std::string(what) + ": shape too large");
    sh.batch = static_cast<int>(batch);
    sh.length = static_cast<int>(length);
    sh.heads = static_cast<int>(heads);
    sh.row = row;
    sh.out_row = heads * kD;
    sh.inv_scale = 0.125f;  // D = 64: a power of two, so the product is the division's exact result
    return KD_OK;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

} // namespace

} // namespace kd

using namespace kd;

extern "C" int kd_causal_attention(int dtype, void* out, void* lse, const void* qkv, int64_t batch, int64_t length,
                                   int64_t heads, int64_t head_dim) {
    AttentionShape sh;
    if (int rc = check_shape(dtype, batch, length, heads, head_dim, sh, "kd_causal_attention")) return rc;
    if (out == nullptr || qkv == nullptr || lse == nullptr || !aligned16(out) || !aligned16(qkv))
        return fail(KD_E_INVALID, "kd_causal_attention: out, lse and qkv must be given, out and qkv 16-byte aligned");
    if (int rc = ensure_device()) return rc;
    const int64_t blocks = (length + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(attention_forward_kernel, dim3(static_cast<uint32_t>(batch * heads * blocks)), dim3(kWaves * 64), 0,
                       stream(), static_cast<float*>(out), static_cast<float*>(lse), static_cast<const float*>(qkv), sh);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

extern "C" int kd_causal_attention_backward(int dtype, void* dqkv, const void* dout, const void* qkv, const void* out,
                                            const void* lse, int64_t batch, int64_t length, int64_t heads,
                                            int64_t head_dim) {
    AttentionShape sh;
    if (int rc = check_shape(dtype, batch, length, heads, head_dim, sh, "kd_causal_attention_backward")) return rc;
    if (dqkv == nullptr || dout == nullptr || qkv == nullptr || out == nullptr || lse == nullptr || !aligned16(dqkv) ||
        !aligned16(dout) || !aligned16(qkv) || !aligned16(out))
        return fail(KD_E_INVALID, "kd_causal_attention_backward: every operand must be given, 16-byte aligned");
    if (int rc = ensure_device()) return rc;
    const int64_t blocks = (length + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(attention_backward_kernel, dim3(static_cast<uint32_t>(2 * batch * heads * blocks)),
                       dim3(kWaves * 64), 0, stream(), static_cast<float*>(dqkv), static_cast<const float*>(dout),
                       static_cast<const float*>(qkv), static_cast<const float*>(out), static_cast<const float*>(lse),
                       sh);
    KD_LAUNCH_CHECK();
    return KD_OK;
}

extern "C" int kd_cached_attention(int dtype, void* out, const void* q, const int64_t* q_strides, const void* k,
                                   const int64_t* k_strides, const void* v, const int64_t* v_strides, int64_t batch,
                                   int64_t heads, int64_t length, int64_t keys, int64_t head_dim) {
    const char* what = "kd_cached_attention";
    if (dtype != KD_F32) return fail(KD_E_UNSUPPORTED, std::string(what) + ": dtype must be f32");
    if (head_dim != kD) return fail(KD_E_UNSUPPORTED, std::string(what) + ": head dim must be 64");
    if (batch < 1 || heads < 1 || length < 1 || keys < length)
        return fail(KD_E_INVALID, std::string(what) + ": needs batch, heads, length >= 1 and keys >= length");
    if (out == nullptr || q == nullptr || k == nullptr || v == nullptr || q_strides == nullptr ||
        k_strides == nullptr || v_strides == nullptr)
        return fail(KD_E_INVALID, std::string(what) + ": every operand and stride array must be given");
    CachedShape sh;
    // every element the kernel reads lies at or below the last row's last feature of each operand
    const int64_t dims[3][3] = {{batch, heads, length}, {batch, heads, keys}, {batch, heads, keys}};
    const int64_t* strides[3] = {q_strides, k_strides, v_strides};
    int64_t* dst[3] = {sh.qs, sh.ks, sh.vs};
    for (int o = 0; o < 3; ++o) {
        int64_t last = kD - 1;
        for (int d = 0; d < 3; ++d) {
            if (strides[o][d] < 0) return fail(KD_E_INVALID, std::string(what) + ": negative stride");
            last += (dims[o][d] - 1) * strides[o][d];
            dst[o][d] = strides[o][d];
        }
        if (last >= (int64_t{1} << 40)) return fail(KD_E_INVALID, std::string(what) + ": operand too large");
    }
    const int64_t rows = batch * heads * length;
    if (rows >= (int64_t{1} << 31) || keys >= (int64_t{1} << 31))
        return fail(KD_E_INVALID, std::string(what) + ": shape too large");
    sh.batch = static_cast<int>(batch);
    sh.heads = static_cast<int>(heads);
    sh.length = static_cast<int>(length);
    sh.keys = static_cast<int>(keys);
    if (int rc = ensure_device()) return rc;
    // few rows (decode): 16 waves share each row's keys; otherwise 4 waves and more workgroups
    const int waves = rows < 2 * compute_units() ? kCachedMaxWaves : 4;
    hipLaunchKernelGGL(cached_attention_kernel, dim3(static_cast<uint32_t>(rows)), dim3(waves * 64), 0, stream(),
                       static_cast<float*>(out), static_cast<const float*>(q), static_cast<const float*>(k),
                       static_cast<const float*>(v), sh);
    KD_LAUNCH_CHECK();
    return KD_OK;
}
