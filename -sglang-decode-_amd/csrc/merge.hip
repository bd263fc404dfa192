// Split merge: per (request, query head), LSE-weighted combination of the
// normalized partial outputs of its splits (kernels/merge.py:7-30).
//
// One wave per (request, head).  The merge is latency-bound (a few KB per row),
// so the dependent chain is two memory round trips: the split count, then the
// split LSEs (one per lane) together with up to kRowsInFlight partial rows
// (each a coalesced 256-1024 B burst, lanes owning head_dim/64 consecutive dims),
// all issued before any is used.  The global max and the weights exp(lse_s - max)
// come from wave reductions.  This is the two-pass form of the reference's
// running-max merge (same value up to rounding).  Rows with no split produce
// exact zeros (0 / max(den, 1e-30)); a plan error produces NaN.
#include "common.h"

namespace sgd {
namespace {

constexpr int kMergeWaves = 4;
constexpr int kRowsInFlight = 16;  // divides 64: a block of rows never straddles two LSE blocks
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

template <int DT, int DPL>  // DPL = dims per lane
__global__ __launch_bounds__(64 * kMergeWaves) void k_merge(const float *__restrict__ partial,
                                                            const float *__restrict__ lse,
                                                            const int32_t *__restrict__ counts,
                                                            const int32_t *__restrict__ error,
                                                            uint16_t *__restrict__ out, int32_t hq,
                                                            int32_t smax) {
    constexpr int D = DPL * 64;
    const int lane = threadIdx.x & 63;
    const int head = blockIdx.y * kMergeWaves + (threadIdx.x >> 6);
    const int r = blockIdx.x;
    if (head >= hq) return;
    const int32_t n = __builtin_amdgcn_readfirstlane(counts[r]);
    const int64_t row = (int64_t)r * hq + head;
    const float *lrow = lse + row * smax;
    const float *prow = partial + row * smax * D + lane * DPL;
    float den = 0.f, acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    float mx = -INFINITY;
    if (n > 64) {  // more splits than lanes: the max first, over all of them
        for (int b = 0; b < n; b += 64)
            mx = fmaxf(mx, wave_max(b + lane < n ? lrow[b + lane] * kLog2e : -INFINITY));
    }
    for (int b = 0; b < n; b += kRowsInFlight) {
        // rows b .. b+kRowsInFlight-1 and (per 64 rows) their LSEs, all in flight at once
        float v[kRowsInFlight][DPL];
#pragma unroll
        for (int s = 0; s < kRowsInFlight; ++s) {
            if (b + s < n) load_row<DPL>(prow + (int64_t)(b + s) * D, v[s]);
            else
#pragma unroll
                for (int i = 0; i < DPL; ++i) v[s][i] = 0.f;
        }
        const int lb = b & ~63;  // LSE block holding rows b..: lane l has split lb + l
        const float l2 = lb + lane < n ? lrow[lb + lane] * kLog2e : -INFINITY;
        if (n <= 64 && b == 0) mx = wave_max(l2);
        const float w = lb + lane < n ? __builtin_amdgcn_exp2f(l2 - mx) : 0.f;
        if ((b & 63) == 0) den += wave_sum(w);
#pragma unroll
        for (int s = 0; s < kRowsInFlight; ++s) {
            if (b + s < n) {
                const float ws = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), (b + s - lb)));
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[i] += v[s][i] * ws;
            }
        }
    }
    const bool bad = *error != 0;
    const float inv = 1.0f / fmaxf(den, 1.0e-30f);
    uint16_t *dst = out + row * D + lane * DPL;
#pragma unroll
    for (int i = 0; i < DPL; ++i) dst[i] = (uint16_t)from_f32<DT>(bad ? __builtin_nanf("") : acc[i] * inv);
}

template <int DT>
int launch_merge(const float *partial, const float *lse, const int32_t *counts, const int32_t *error, void *out,
                 int32_t bcap, int32_t hq, int32_t d, int32_t smax, hipStream_t stream) {
    const dim3 grid(bcap, (hq + kMergeWaves - 1) / kMergeWaves);
    const dim3 block(64 * kMergeWaves);
    auto *o = static_cast<uint16_t *>(out);
    switch (d) {
        case 64: hipLaunchKernelGGL((k_merge<DT, 1>), grid, block, 0, stream, partial, lse, counts, error, o, hq, smax); break;
        case 128: hipLaunchKernelGGL((k_merge<DT, 2>), grid, block, 0, stream, partial, lse, counts, error, o, hq, smax); break;
        case 256: hipLaunchKernelGGL((k_merge<DT, 4>), grid, block, 0, stream, partial, lse, counts, error, o, hq, smax); break;
        default: return einval("merge_splits: head_dim %d not in {64,128,256}", d);
    }
    return launch_status("merge_splits");
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_merge_splits(const float *partial, const float *lse, const int32_t *counts,
                                const int32_t *active, const int32_t *error, void *out, int32_t bcap,
                                int32_t query_heads, int32_t head_dim, int32_t max_splits, int32_t dtype,
                                void *stream) {
    (void)active;  // every row r < bcap is written; inactive rows have counts[r] == 0
    if (bcap <= 0 || query_heads <= 0 || max_splits <= 0) return einval("merge_splits: bad geometry");
    if ((reinterpret_cast<uintptr_t>(partial) & 15) != 0) return einval("merge_splits: partial not 16B aligned");
    clear_stale_error();
    if (dtype == SGD_BF16)
        return launch_merge<SGD_BF16>(partial, lse, counts, error, out, bcap, query_heads, head_dim, max_splits,
                                      (hipStream_t)stream);
    if (dtype == SGD_FP16)
        return launch_merge<SGD_FP16>(partial, lse, counts, error, out, bcap, query_heads, head_dim, max_splits,
                                      (hipStream_t)stream);
    return einval("merge_splits: dtype %d", dtype);
}
