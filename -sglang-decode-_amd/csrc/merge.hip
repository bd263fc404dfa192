// Split merge: per (request, query head), LSE-weighted combination of the
// normalized partial outputs of its splits, in split order (kernels/merge.py:7-30).
//
// One wave per (request, head); each lane owns head_dim/64 consecutive dims, so
// every partial row is read as one coalesced 256-1024 B burst.  Rows with no
// split produce exact zeros (acc 0 / max(den, 1e-30)); a plan error produces NaN.
#include "common.h"

namespace sgd {
namespace {

constexpr int kMergeWaves = 4;

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
    const int32_t n = counts[r];
    const int64_t row = (int64_t)r * hq + head;
    float m = -INFINITY, den = 0.f, acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    for (int s = 0; s < n; ++s) {
        const int64_t slot = row * smax + s;
        const float l = lse[slot];
        const float *src = partial + slot * D + lane * DPL;
        float v[DPL];
        if constexpr (DPL == 4) {
            const float4 t = *reinterpret_cast<const float4 *>(src);
            v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
        } else if constexpr (DPL == 2) {
            const float2 t = *reinterpret_cast<const float2 *>(src);
            v[0] = t.x; v[1] = t.y;
        } else {
            v[0] = src[0];
        }
        const float nm = fmaxf(m, l);
        const float ow = __expf(m - nm), w = __expf(l - nm);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] = acc[i] * ow + v[i] * w;
        den = den * ow + w;
        m = nm;
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
