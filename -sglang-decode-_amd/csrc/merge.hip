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

// Rows the full merge (k_merge: one 4-wave workgroup per row, 60 VGPRs, so 8 per CU)
// keeps resident at once; beyond them its workgroups queue in rounds.  Read once per
// process from the first device used (a node's GPUs are alike); it only chooses between
// two correct merge orders and sizes a strided grid, so any value is safe.
int merge_rows_resident() {
    static int rows = [] {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        return 8 * cus;
    }();
    return rows;
}

namespace {

using namespace mergeops;

// One workgroup of kSplitWaves waves per (request, head) row.  A row with at most
// kRowsInFlight splits is merged by wave 0 alone (one round trip for its data); a longer
// one is cut into kSplitWaves contiguous split ranges, merged by the waves side by side
// and combined in wave order through LDS -- so a 64-split row costs a block's round trip,
// not four.
constexpr int kSplitWaves = 4;

template <int DT, int DPL>
__device__ __forceinline__ void merge_one(const float *__restrict__ partial, const float *__restrict__ lse,
                                          int32_t n, bool bad, uint16_t *__restrict__ out, int64_t row,
                                          int32_t smax, float (&sm)[kSplitWaves], float (&sd)[kSplitWaves],
                                          float (&sacc)[kSplitWaves][DPL * 64], int lane, int wave) {
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

// Every row: a (request, head) grid, one row per workgroup.
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
    merge_one<DT, DPL>(partial, lse, n, bad, out, (int64_t)r * hq + head, smax, sm, sd, sacc, lane, wave);
}

// The rows of requests with no split or at least min_splits of them (all rows on a plan
// error): at most one residency round of workgroups (the occupancy API's count per CU),
// striding over the rows in (request, head) order.  A row of 1 <= n < min_splits splits (written by the attention) costs its
// workgroup only the split count, which is requested a row ahead.
template <int DT, int DPL>
__global__ __launch_bounds__(64 * kSplitWaves) void k_merge_rows(const float *__restrict__ partial,
                                                                 const float *__restrict__ lse,
                                                                 const int32_t *__restrict__ counts,
                                                                 const int32_t *__restrict__ error,
                                                                 uint16_t *__restrict__ out, int32_t hq,
                                                                 int32_t smax, int32_t rows, int32_t min_splits) {
    __shared__ float sm[kSplitWaves], sd[kSplitWaves], sacc[kSplitWaves][DPL * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool bad = *error != 0;
    int32_t row = blockIdx.x;
    int32_t n = row < rows ? __builtin_amdgcn_readfirstlane(counts[row / hq]) : 0;
    while (row < rows) {  // uniform over the workgroup
        const int32_t next = row + gridDim.x;
        const int32_t n_next = next < rows ? __builtin_amdgcn_readfirstlane(counts[next / hq]) : 0;
        if (bad || n == 0 || n >= min_splits) {
            merge_one<DT, DPL>(partial, lse, n, bad, out, row, smax, sm, sd, sacc, lane, wave);
            if (next < rows) lds_barrier();  // the LDS combine of this row is read before the next one's
        }
        row = next;
        n = n_next;
    }
}

template <int DT, int DPL>
void launch_merge_d(const float *partial, const float *lse, const int32_t *counts, const int32_t *error,
                    uint16_t *out, int32_t bcap, int32_t hq, int32_t smax, int32_t min_splits, hipStream_t stream) {
    const dim3 block(64 * kSplitWaves);
    if (min_splits <= 1) {
        hipLaunchKernelGGL((k_merge<DT, DPL>), dim3(bcap, hq), block, 0, stream, partial, lse, counts, error, out, hq,
                           smax);
        return;
    }
    static int resident = [] {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_merge_rows<DT, DPL>, 64 * kSplitWaves, 0) !=
                hipSuccess ||
            per_cu <= 0)
            per_cu = 4;
        return per_cu * cus;
    }();
    const int32_t rows = bcap * hq;
    hipLaunchKernelGGL((k_merge_rows<DT, DPL>), dim3(rows < resident ? rows : resident), block, 0, stream, partial,
                       lse, counts, error, out, hq, smax, rows, min_splits);
}

template <int DT>
int launch_merge(const float *partial, const float *lse, const int32_t *counts, const int32_t *error, void *out,
                 int32_t bcap, int32_t hq, int32_t d, int32_t smax, int32_t min_splits, hipStream_t stream) {
    auto *o = static_cast<uint16_t *>(out);
    switch (d) {
        case 64: launch_merge_d<DT, 1>(partial, lse, counts, error, o, bcap, hq, smax, min_splits, stream); break;
        case 128: launch_merge_d<DT, 2>(partial, lse, counts, error, o, bcap, hq, smax, min_splits, stream); break;
        case 256: launch_merge_d<DT, 4>(partial, lse, counts, error, o, bcap, hq, smax, min_splits, stream); break;
        default: return einval("merge_splits: head_dim %d not in {64,128,256}", d);
    }
    return launch_status("merge_splits");
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_merge_splits_min(const float *partial, const float *lse, const int32_t *counts,
                                    const int32_t *active, const int32_t *error, void *out, int32_t bcap,
                                    int32_t query_heads, int32_t head_dim, int32_t max_splits, int32_t min_splits,
                                    int32_t dtype, void *stream) {
    (void)active;  // every row r < bcap is written; inactive rows have counts[r] == 0
    if (bcap <= 0 || query_heads <= 0 || max_splits <= 0) return einval("merge_splits: bad geometry");
    if ((int64_t)bcap * query_heads > INT32_MAX) return einval("merge_splits: too many rows");
    if ((reinterpret_cast<uintptr_t>(partial) & 15) != 0) return einval("merge_splits: partial not 16B aligned");
    clear_stale_error();
    if (dtype == SGD_BF16)
        return launch_merge<SGD_BF16>(partial, lse, counts, error, out, bcap, query_heads, head_dim, max_splits,
                                      min_splits, (hipStream_t)stream);
    if (dtype == SGD_FP16)
        return launch_merge<SGD_FP16>(partial, lse, counts, error, out, bcap, query_heads, head_dim, max_splits,
                                      min_splits, (hipStream_t)stream);
    return einval("merge_splits: dtype %d", dtype);
}

extern "C" int sgd_merge_splits(const float *partial, const float *lse, const int32_t *counts,
                                const int32_t *active, const int32_t *error, void *out, int32_t bcap,
                                int32_t query_heads, int32_t head_dim, int32_t max_splits, int32_t dtype,
                                void *stream) {
    return sgd_merge_splits_min(partial, lse, counts, active, error, out, bcap, query_heads, head_dim, max_splits,
                                1, dtype, stream);
}
