// Layout shared by the span-schedule attention kernel and the merge that completes
// its cut tasks: the tile sequence's worker ranges and the edge-state records.
#pragma once

#include "common.h"

namespace sgd {
namespace span {

constexpr int kTile = 16;   // tokens per tile
constexpr int kHeads = 4;   // query heads per kv head (padded group)
constexpr int kD = 128;     // head_dim
// One edge record: unnormalized P.V acc[kHeads][kD], then the running max m[kHeads]
// (log2 domain) and the denominator den[kHeads].
constexpr int kPieceFloats = kHeads * kD + 2 * kHeads;
constexpr int kPieceM = kHeads * kD, kPieceDen = kHeads * kD + kHeads;

constexpr int kWaves = 8;   // waves per workgroup: one workgroup per CU
constexpr int kRecord = 16; // ints per wave record of the plan's span table

// floor(n / d) for 0 <= n < 2^53, 0 < d, quotient < 2^31: a double quotient (n and d
// are exact in double) corrected by one step either way with integer products -- the
// GPU has no integer divider, and a 64-bit division is a long instruction sequence.
__host__ __device__ __forceinline__ int32_t floor_div(int64_t n, int64_t d) {
    int64_t q = (int64_t)((double)n / (double)d);
    if (q * d > n) --q;
    else if ((q + 1) * d <= n) ++q;
    return (int32_t)q;
}

// First tile of wave u of U: floor(u * T / U).
__device__ __forceinline__ int64_t wave_start(int64_t u, int64_t T, int32_t U) { return floor_div(u * T, U); }

// The wave whose range holds tile x (0 <= x < T): the largest u with wave_start(u) <= x.
__device__ __forceinline__ int32_t wave_of(int64_t x, int64_t T, int32_t U) { return floor_div((x + 1) * U - 1, T); }

// Workgroup w holds waves [w * kWaves, (w + 1) * kWaves).
__device__ __forceinline__ int64_t worker_start(int64_t w, int64_t T, int32_t U) {
    return wave_start(w * kWaves, T, U);
}
__device__ __forceinline__ int32_t worker_of(int64_t x, int64_t T, int32_t U) { return wave_of(x, T, U) / kWaves; }

}  // namespace span
}  // namespace sgd
