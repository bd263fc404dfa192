// Split merge: per (request, query head), LSE-weighted combination of the
// normalized partial outputs of its splits (kernels/merge.py:7-30).
//
// The merge is latency-bound (a few KB per row): the split count, then the split
// LSEs together with up to kRowsInFlight partial rows (each a coalesced 256-1024 B
// burst, lanes owning head_dim/64 consecutive dims), all issued before any is used.
// A row with more splits is cut over the workgroup's waves (k_merge).  The max and
// the weights exp(lse_s - max) come from wave reductions, combined online from block
// to block and wave to wave in a fixed order: the value of the reference's running-max
// merge up to rounding.  Rows with no split produce exact zeros (0 / max(den, 1e-30));
// a plan error produces NaN.
#include "merge_ops.h"

namespace sgd {
namespace {

using namespace mergeops;

// One workgroup of kSplitWaves waves per (request, head).  A row with at most
// kRowsInFlight splits is merged by wave 0 alone (one round trip for its data); a
// longer one is cut into kSplitWaves contiguous split ranges, merged by the waves side
// by side and combined in wave order through LDS -- so a 64-split row costs a block's
// round trip, not four.
constexpr int kSplitWaves = 4;

template <int DT, int DPL>
__global__ __launch_bounds__(64 * kSplitWaves) void k_merge(const float *__restrict__ partial,
                                                            const float *__restrict__ lse,
                                                            const int32_t *__restrict__ counts,
                                                            const int32_t *__restrict__ error,
                                                            uint16_t *__restrict__ out, int32_t hq,
                                                            int32_t smax) {
    __shared__ float sm[kSplitWaves], sd[kSplitWaves], sacc[kSplitWaves][DPL * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x, head = blockIdx.y;
    const int32_t n = __builtin_amdgcn_readfirstlane(counts[r]);
    const bool bad = *error != 0;
    const int64_t row = (int64_t)r * hq + head;
    if (n <= kRowsInFlight) {
        if (wave == 0) merge_row<DT, DPL>(partial, lse, n, bad, out, row, smax, lane);
        return;  // n is the workgroup's: no wave waits below
    }
    const int32_t q = (n + kSplitWaves - 1) / kSplitWaves;
    float m, den, acc[DPL];
    merge_part<DPL>(partial, lse, row, smax, min(wave * q, n), min((wave + 1) * q, n), lane, m, den, acc);
    if (lane == 0) {
        sm[wave] = m;
        sd[wave] = den;
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i) sacc[wave][lane * DPL + i] = acc[i];
    lds_barrier();
    if (wave != 0) return;
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kSplitWaves; ++k) M = fmaxf(M, sm[k]);
    float D = 0.f, X[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) X[i] = 0.f;
#pragma unroll
    for (int k = 0; k < kSplitWaves; ++k) {
        if (sd[k] == 0.f) continue;  // an empty range
        const float sc = __builtin_amdgcn_exp2f(sm[k] - M);
        D += sd[k] * sc;
#pragma unroll
        for (int i = 0; i < DPL; ++i) X[i] += sacc[k][lane * DPL + i] * sc;
    }
    store_row<DT, DPL>(out, row, D, X, bad, lane);
}

template <int DT>
int launch_merge(const float *partial, const float *lse, const int32_t *counts, const int32_t *error, void *out,
                 int32_t bcap, int32_t hq, int32_t d, int32_t smax, hipStream_t stream) {
    const dim3 grid(bcap, hq), block(64 * kSplitWaves);
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
