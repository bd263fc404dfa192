// The decode step's CSR metadata from the request pool, in one launch: the inputs the
// reference adapter consumes (integrations/sglang_backend.py:98-107 reads
// forward_metadata.kv_indptr, kv_indices and num_kv_splits), produced upstream by
// SGLang's triton backend (v0.4.6.post5, triton_backend.py init_forward_metadata for
// decode: kv_indptr[1:] = cumsum(seq_lens), then create_flashinfer_kv_indices_triton
// copying req_to_token[req_pool_indices[i], 0:seq_lens[i]] to kv_indices[kv_indptr[i]:],
// then its split heuristic).  Split counts here follow the reference harness rule
// (benchmarks/workloads.py:20-21): chunk = max(1, ceil(max L / S_max)), S_r =
// clamp(ceil(L_r / chunk), 1, S_max).  Optionally the plan's lengths / splits / active
// are written too, so the plan build needs no copy of its own.
//
// kRowParts workgroups per request row.  Each computes the row's offset (the sum of
// the lengths before it) and the batch's longest length with a workgroup reduction over
// the batch's lengths (batch <= 4096 ints, served from cache), then copies its share of
// the row's token slots (4 bytes read and 4 written per token, 64 consecutive slots per
// wave instruction).  The parts put a whole row's loads in flight at once: a row of a
// few thousand tokens is one round trip, not one per 256 tokens.  Part 0 writes the
// row's kv_indptr entry, split count and plan inputs.
//
// A row is invalid when its length is negative or longer than a req_to_token row, or
// its pool index lies outside the table: it then counts as length 0 everywhere (no slot
// is read or written for it) and *error is set.  When the valid rows' total exceeds
// indices_capacity, every row counts as length 0 (kv_indptr all zero, one split each)
// and *error is set.  Nothing is accessed out of bounds either way.
#include "common.h"

namespace sgd {
namespace {

constexpr int kMetaThreads = 256;
constexpr int kRowParts = 8;

struct MetaArgs {
    const void *seq_lens;          // [batch], int32 or int64
    const void *req_pool_indices;  // [batch], int32 or int64
    const int32_t *req_to_token;   // [rows, row_stride]
    int64_t row_stride, rows;
    int32_t cols;                  // usable tokens per req_to_token row
    int32_t *kv_indptr;            // [batch + 1]
    int32_t *kv_indices;           // [indices_capacity]
    int64_t indices_capacity;
    int32_t *num_kv_splits;        // [batch] or null
    int32_t *plan_lengths, *plan_splits, *plan_active;  // [batch], [batch], [1]; or null
    int32_t *error;                // [1] or null (set to 1 on an invalid row, never cleared here)
    int32_t batch, max_splits, lens64, pool64;
};

__device__ __forceinline__ int64_t load_int(const void *p, int32_t i, int32_t is64) {
    return is64 ? static_cast<const int64_t *>(p)[i] : static_cast<const int32_t *>(p)[i];
}

// Length of row i as counted (0 for an invalid row; the capacity rule applies to the
// batch's total and is taken by the caller).
__device__ __forceinline__ int64_t row_length(const MetaArgs &a, int32_t i) {
    const int64_t L = load_int(a.seq_lens, i, a.lens64);
    const int64_t pool = load_int(a.req_pool_indices, i, a.pool64);
    return (L < 0 || L > a.cols || pool < 0 || pool >= a.rows) ? 0 : L;
}

__global__ __launch_bounds__(kMetaThreads) void k_csr_metadata(MetaArgs a) {
    __shared__ int64_t red_sum[kMetaThreads / 64], red_total[kMetaThreads / 64], red_max[kMetaThreads / 64];
    const int32_t r = blockIdx.x, part = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (r >= a.batch) {  // the launch of an empty batch: kv_indptr = [0], active = 0
        if (tid == 0 && part == 0) {
            a.kv_indptr[0] = 0;
            if (a.plan_active) *a.plan_active = 0;
        }
        return;
    }
    int64_t before = 0, total = 0, longest = 0;
    for (int32_t i = tid; i < a.batch; i += kMetaThreads) {
        const int64_t L = row_length(a, i);
        if (i < r) before += L;
        total += L;
        longest = max(longest, L);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        before += __shfl_xor(before, o, 64);
        total += __shfl_xor(total, o, 64);
        longest = max(longest, __shfl_xor(longest, o, 64));
    }
    if (lane == 0) {
        red_sum[wave] = before;
        red_total[wave] = total;
        red_max[wave] = longest;
    }
    __syncthreads();
    int64_t offset = 0, all = 0, maxlen = 0;
#pragma unroll
    for (int w = 0; w < kMetaThreads / 64; ++w) {
        offset += red_sum[w];
        all += red_total[w];
        maxlen = max(maxlen, red_max[w]);
    }
    const bool overflow = all > a.indices_capacity;
    const int64_t raw = load_int(a.seq_lens, r, a.lens64);
    const int64_t pool = load_int(a.req_pool_indices, r, a.pool64);
    const int64_t L = overflow ? 0 : row_length(a, r);
    const bool bad = overflow || (L == 0 && raw != 0);
    if (overflow) offset = maxlen = 0;
    if (tid == 0 && part == 0) {
        a.kv_indptr[r + 1] = (int32_t)(offset + L);
        if (r == 0) a.kv_indptr[0] = 0;
        const int64_t chunk = max<int64_t>(1, (maxlen + a.max_splits - 1) / a.max_splits);
        const int32_t s = (int32_t)min<int64_t>(a.max_splits, max<int64_t>(1, (L + chunk - 1) / chunk));
        if (a.num_kv_splits) a.num_kv_splits[r] = s;
        if (a.plan_lengths) a.plan_lengths[r] = (int32_t)L;
        if (a.plan_splits) a.plan_splits[r] = s;
        if (a.plan_active && r == 0) *a.plan_active = a.batch;
        if (bad && a.error) *a.error = 1;
    }
    const int32_t *src = a.req_to_token + (L > 0 ? pool * a.row_stride : 0);
    int32_t *dst = a.kv_indices + offset;
    for (int64_t j = part * kMetaThreads + tid; j < L; j += kRowParts * kMetaThreads) dst[j] = src[j];
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_csr_metadata(const void *seq_lens, int32_t seq_lens_is_int64, const void *req_pool_indices,
                                int32_t pool_indices_is_int64, const int32_t *req_to_token, int64_t rows,
                                int64_t row_stride, int32_t cols, int32_t batch, int32_t max_splits,
                                int32_t *kv_indptr, int32_t *kv_indices, int64_t indices_capacity,
                                int32_t *num_kv_splits, int32_t *plan_lengths, int32_t *plan_splits,
                                int32_t *plan_active, int32_t *error, void *stream) {
    if (batch < 0 || batch > 4096) return einval("csr_metadata: batch %d outside [0, 4096]", batch);
    if (max_splits <= 0) return einval("csr_metadata: max_splits %d", max_splits);
    if (!kv_indptr) return einval("csr_metadata: kv_indptr is required");
    if (batch > 0 && (!seq_lens || !req_pool_indices || !req_to_token || rows <= 0 || cols < 0 ||
                      row_stride < cols || indices_capacity < 0 || (indices_capacity > 0 && !kv_indices)))
        return einval("csr_metadata: seq_lens, req_pool_indices, req_to_token [rows >= 1, stride >= cols] "
                      "and kv_indices are required");
    if (indices_capacity >= (1ll << 31)) return einval("csr_metadata: kv_indices capacity beyond int32 offsets");
    if ((plan_lengths != nullptr) != (plan_splits != nullptr))
        return einval("csr_metadata: plan lengths and splits go together");
    MetaArgs a{};
    a.seq_lens = seq_lens;
    a.req_pool_indices = req_pool_indices;
    a.req_to_token = req_to_token;
    a.row_stride = row_stride;
    a.rows = rows;
    a.cols = cols;
    a.kv_indptr = kv_indptr;
    a.kv_indices = kv_indices;
    a.indices_capacity = indices_capacity;
    a.num_kv_splits = num_kv_splits;
    a.plan_lengths = plan_lengths;
    a.plan_splits = plan_splits;
    a.plan_active = plan_active;
    a.error = error;
    a.batch = batch;
    a.max_splits = max_splits;
    a.lens64 = seq_lens_is_int64 != 0;
    a.pool64 = pool_indices_is_int64 != 0;
    clear_stale_error();
    // an empty batch still launches one workgroup: it writes kv_indptr[0] (and active)
    hipLaunchKernelGGL(k_csr_metadata, dim3(batch > 0 ? batch : 1, kRowParts), dim3(kMetaThreads), 0,
                       (hipStream_t)stream, a);
    return launch_status("csr_metadata");
}
