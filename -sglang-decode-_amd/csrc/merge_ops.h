// Row-merge building blocks shared by the split merge (merge.hip) and the upstream
// two-stage comparator (upstream.hip): one wave's LSE-weighted sum over a range of a
// (request, head) row's split slots, with each block of up to kRowsInFlight rows and
// their LSEs in flight together, and the merged row's store.
#pragma once

#include "common.h"

namespace sgd {
namespace mergeops {

constexpr int kRowsInFlight = 16;  // split rows per round trip
constexpr float kLog2e = 1.4426950408889634f;

template <int DPL>
__device__ __forceinline__ void load_row(const float *src, float (&v)[DPL]) {
    if constexpr (DPL == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(src);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else if constexpr (DPL == 2) {
        const float2 t = *reinterpret_cast<const float2 *>(src);
        v[0] = t.x; v[1] = t.y;
    } else {
        v[0] = src[0];
    }
}

// One wave's LSE-weighted sum over splits [s0, s1) of the (request, head) row `row`:
// its running max m (log2 domain), denominator and unnormalized sum acc (this lane's
// DPL dims), built in blocks of kRowsInFlight split rows -- each block's rows and
// LSEs in flight together -- combined online from block to block.  An empty range
// leaves (-inf, 0, 0).
template <int DPL>
__device__ __forceinline__ void merge_part(const float *__restrict__ partial, const float *__restrict__ lse,
                                           int64_t row, int32_t smax, int32_t s0, int32_t s1, int lane,
                                           float &m, float &den, float (&acc)[DPL]) {
    constexpr int D = DPL * 64;
    const float *lrow = lse + row * smax;
    const float *prow = partial + row * smax * D + lane * DPL;
    m = -INFINITY;
    den = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    for (int b = s0; b < s1; b += kRowsInFlight) {
        float v[kRowsInFlight][DPL];
#pragma unroll
        for (int s = 0; s < kRowsInFlight; ++s) {
            if (b + s < s1) load_row<DPL>(prow + (int64_t)(b + s) * D, v[s]);
            else
#pragma unroll
                for (int i = 0; i < DPL; ++i) v[s][i] = 0.f;
        }
        // lane l < kRowsInFlight holds split b + l's LSE
        const bool mine = lane < kRowsInFlight && b + lane < s1;
        const float l2 = mine ? lrow[b + lane] * kLog2e : -INFINITY;
        const float mb = fmaxf(m, wave_max(l2));
        const float so = __builtin_amdgcn_exp2f(m - mb);  // 0 for the first block (m = -inf)
        const float w = mine ? __builtin_amdgcn_exp2f(l2 - mb) : 0.f;
        den = den * so + wave_sum(w);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] *= so;
#pragma unroll
        for (int s = 0; s < kRowsInFlight; ++s) {
            if (b + s < s1) {
                const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s));
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[i] += v[s][i] * ws;
            }
        }
        m = mb;
    }
}

// The merged row out = acc / den (0 for a row without splits, NaN on a plan error).
template <int DT, int DPL>
__device__ __forceinline__ void store_row(uint16_t *__restrict__ out, int64_t row, float den,
                                          const float (&acc)[DPL], bool bad, int lane) {
    const float inv = 1.0f / fmaxf(den, 1.0e-30f);
    uint16_t *dst = out + row * (DPL * 64) + lane * DPL;
#pragma unroll
    for (int i = 0; i < DPL; ++i) dst[i] = (uint16_t)from_f32<DT>(bad ? __builtin_nanf("") : acc[i] * inv);
}

// The merge of one (request, head) row by one wave: n splits of partial/lse rows.
template <int DT, int DPL>  // DPL = dims per lane
__device__ __forceinline__ void merge_row(const float *__restrict__ partial, const float *__restrict__ lse,
                                          int32_t n, bool bad, uint16_t *__restrict__ out, int64_t row,
                                          int32_t smax, int lane) {
    float m, den, acc[DPL];
    merge_part<DPL>(partial, lse, row, smax, 0, n, lane, m, den, acc);
    store_row<DT, DPL>(out, row, den, acc, bad, lane);
}

}  // namespace mergeops
}  // namespace sgd
