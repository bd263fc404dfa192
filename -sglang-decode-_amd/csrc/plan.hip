// Device plan construction for the persistent decode: count/scan, SoA records,
// mode selection + bucket order + packs, and the STATIC (LPT) lists.
//
// Every stage runs in ONE 1024-thread workgroup: the batch (<= 4096 rows) and the
// record table (<= 16384 records) are small, and keeping the whole plan in one
// workgroup lets the fused entry run all stages in a single launch with only
// workgroup barriers between them (the reference launches four kernels,
// planning/builder.py:6-28).  Results are identical to the reference stages:
//   count_scan           kernels/plan.py:7-27
//   emit_records         kernels/plan.py:30-45
//   make_order_and_packs kernels/plan.py:48-100
//   greedy_lists         kernels/plan.py:103-135 (same lists as planning/reference.py:57-67)
// Integer arithmetic is int32 with wrap-around, like the reference's lanes.
#include "common.h"

namespace sgd {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kMaxBuckets = 16;
constexpr int kLdsRules = 32;  // policy rules the fused kernel copies to LDS (more stay in global memory)

__device__ __forceinline__ int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
__device__ __forceinline__ int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
__device__ __forceinline__ int32_t cdiv(int32_t a, int32_t b) { return wadd(wadd(a, b), -1) / b; }

struct PlanShared {
    int32_t scan_tmp[16];
    uint64_t scan_tmp64[16];
    int32_t bucket_size[kMaxBuckets];
    int32_t bucket_record_base[kMaxBuckets];
    int32_t bucket_pack_base[kMaxBuckets];
    int32_t bucket_pack_count[kMaxBuckets];
    int32_t bucket_width[kMaxBuckets];
    int32_t bucket_packed_packs[kMaxBuckets];
    int32_t bucket_packed_tasks[kMaxBuckets];
    int32_t mode;
    int32_t record_count;
    int32_t num_packs;
    int32_t max_w, min_w;
    int32_t red_max[16], red_min[16], red_or[16];
    int32_t rules[5 * kLdsRules];   // the fused kernel's copy of the policy rules
    int32_t hist[16][kMaxBuckets];  // per-wave bucket counts of one partition pass
    int32_t carry[kMaxBuckets];     // bucket counts of the earlier passes
};

// ---------------------------------------------------------------- count/scan
// Optional LDS copies of the per-row values for the fused kernel's later stages.
struct RowMirror {
    int32_t *lengths, *counts, *offsets, *chunk;  // LDS, [bcap] ([bcap + 1] for offsets); counts may be null
};

constexpr int kMaxRowsPerThread = 4;  // bcap <= 4096 = 4 x kPlanThreads

// The plan's inputs taken from the CSR metadata of the step instead of the plan's own
// lengths/splits/active buffers: rows r < batch get length kv_indptr[r+1] - kv_indptr[r]
// and split count num_kv_splits[r], active = batch -- the values the reference adapter
// copies into the plan before every build (integrations/sglang_backend.py:98-99) -- and
// those values are also stored to the plan's buffers (the attention reads them).
struct CsrRows {
    const int32_t *indptr, *splits;
    int32_t batch;
    int32_t *lengths_out, *splits_out, *active_out;
};

__device__ void stage_count_scan(const int32_t *lengths, const int32_t *splits, const int32_t *active_p,
                                 int32_t *counts, int32_t *offsets, int32_t *chunk, int32_t *record_count,
                                 int32_t *error, int32_t bcap, int32_t smax, int32_t max_context,
                                 PlanShared &sh, const RowMirror *mirror = nullptr, const CsrRows *csr = nullptr) {
    const int tid = threadIdx.x;
    const int per = (bcap + kPlanThreads - 1) / kPlanThreads;  // rows per thread (contiguous)
    const int32_t active = csr ? csr->batch : *active_p;
    if (csr && tid == 0) *csr->active_out = active;
    const int r0 = tid * per;
    int invalid_any = 0;
    int32_t local = 0, nrow[kMaxRowsPerThread];
    // pass 1: validity, chunk, n
#pragma unroll
    for (int i = 0; i < kMaxRowsPerThread; ++i) {
        nrow[i] = 0;
        const int r = r0 + i;
        if (i >= per || r >= bcap) continue;
        const bool live = r < active;
        int32_t raw_length, raw_split;  // issued with the load of active
        if (csr) {
            raw_length = live ? wadd(csr->indptr[r + 1], -csr->indptr[r]) : 0;
            raw_split = live ? csr->splits[r] : 1;
            if (live) {
                csr->lengths_out[r] = raw_length;
                csr->splits_out[r] = raw_split;
            }
        } else {
            raw_length = lengths[r];
            raw_split = splits[r];
        }
        const int32_t length = live ? raw_length : 0;
        const int32_t s = live ? raw_split : 1;
        const bool invalid = live && (length < 0 || length > max_context || s < 1 || s > smax);
        invalid_any |= invalid;
        const int32_t c = wmul(cdiv(cdiv(max(length, 0), max(s, 1)), 32), 32);
        chunk[r] = c;
        nrow[i] = (live && !invalid) ? cdiv(length, max(c, 1)) : 0;
        local = wadd(local, nrow[i]);
        if (mirror) {
            mirror->lengths[r] = length;
            mirror->chunk[r] = c;
        }
    }
    // workgroup OR of the validity flags through LDS (outputs stay in flight)
    const bool wave_invalid = __ballot(invalid_any) != 0;
    if ((tid & 63) == 0) sh.red_or[tid >> 6] = wave_invalid;
    lds_barrier();
    bool any_invalid = false;
#pragma unroll
    for (int w = 0; w < kPlanThreads / 64; ++w) any_invalid |= sh.red_or[w] != 0;
    const bool err = (active < 0) || (active > bcap) || any_invalid;
    if (err) local = 0;
    int32_t total;
    int32_t running = block_exclusive_scan<int32_t>(local, sh.scan_tmp, &total);
#pragma unroll
    for (int i = 0; i < kMaxRowsPerThread; ++i) {
        const int r = r0 + i;
        if (i >= per || r >= bcap) continue;
        const int32_t n = err ? 0 : nrow[i];
        counts[r] = n;
        offsets[r] = running;
        if (mirror) {
            if (mirror->counts) mirror->counts[r] = n;
            mirror->offsets[r] = running;
        }
        running = wadd(running, n);
    }
    if (tid == 0) {
        offsets[bcap] = total;
        *record_count = total;
        *error = err ? 1 : 0;
        sh.record_count = total;
        if (mirror) mirror->offsets[bcap] = total;
    }
}

// ---------------------------------------------------------------- records
// lengths/counts/offsets/chunk are read through the given pointers (global memory for
// the single-stage kernel, the LDS copies in the fused one); weight_mirror, when set, is
// an LDS copy of the weights for the later stages.
__device__ void stage_emit_records(const int32_t *lengths, const int32_t *counts, const int32_t *offsets,
                                   const int32_t *chunk, int32_t *request, int32_t *split, int32_t *begin,
                                   int32_t *end, int32_t *weight, int32_t bcap, int32_t smax,
                                   int32_t block_kv, int32_t *weight_mirror = nullptr) {
    const int64_t pairs = (int64_t)bcap * smax;
    for (int64_t p = threadIdx.x; p < pairs; p += kPlanThreads) {
        const int r = (int)(p / smax), s = (int)(p % smax);
        const int32_t n = counts ? counts[r] : wadd(offsets[r + 1], -offsets[r]);
        if (s >= n) continue;
        const int32_t idx = wadd(offsets[r], s);
        const int32_t c = chunk[r];
        const int32_t b = wmul(s, c);
        const int32_t e = min(wadd(b, c), lengths[r]);
        request[idx] = r;
        split[idx] = s;
        begin[idx] = b;
        end[idx] = e;
        const int32_t w = cdiv(wadd(e, -b), block_kv);
        weight[idx] = w;
        if (weight_mirror) weight_mirror[idx] = w;
    }
}

// The request of record rec: the upper bound of rec in offsets[1 .. bcap] (records of a
// request are contiguous; empty requests are skipped).
__device__ __forceinline__ int32_t request_of(const int32_t *offsets, int32_t bcap, int32_t rec) {
    int32_t lo = 0, hi = bcap;  // upper bound of rec in offsets[1 .. bcap]
    while (lo < hi) {
        const int32_t mid = (lo + hi) >> 1;
        if (rec >= offsets[mid + 1]) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// The fused kernel's emission, one record per thread (work grows with the records, not
// with bcap x smax): the request of record idx comes from the LDS offsets, the fields
// are those of stage_emit_records.
__device__ void stage_emit_by_record(const RowMirror &rows, int32_t total, int32_t bcap, int32_t *request,
                                     int32_t *split, int32_t *begin, int32_t *end, int32_t *weight,
                                     int32_t block_kv, int32_t *weight_mirror) {
    for (int32_t idx = threadIdx.x; idx < total; idx += kPlanThreads) {
        const int32_t r = request_of(rows.offsets, bcap, idx);
        const int32_t s = wadd(idx, -rows.offsets[r]);
        const int32_t c = rows.chunk[r];
        const int32_t b = wmul(s, c);
        const int32_t e = min(wadd(b, c), rows.lengths[r]);
        request[idx] = r;
        split[idx] = s;
        begin[idx] = b;
        end[idx] = e;
        const int32_t w = cdiv(wadd(e, -b), block_kv);
        weight[idx] = w;
        weight_mirror[idx] = w;
    }
}

__device__ __forceinline__ int bucket_of(int32_t w, int buckets) {
    int b = 0;
    for (int k = 1; k < buckets; ++k) b += w > (1 << (k - 1));
    return b;
}

// ---------------------------------------------------------------- bucket tables
struct BucketOf {
    int32_t rbase, pbase, width, pp, pt;
};

// The bucket holding sorted record position j (buckets are laid out heaviest first),
// read from the LDS tables at uniform addresses.  The callers loop over tasks, so the
// lanes past the last task are switched off: a per-lane register copy of the tables read
// back with v_readlane would read those lanes' stale registers (the compiler loads the
// copy inside the loop), while an LDS broadcast gives every active lane the table.
__device__ __forceinline__ BucketOf bucket_at(const PlanShared &sh, int32_t j, int buckets) {
    BucketOf o{0, 0, 1, 0, 0};
    for (int q = buckets - 1; q >= 0; --q) {
        const int32_t lo = sh.bucket_record_base[q], n = sh.bucket_size[q];
        if (j >= lo && j < lo + n) {
            o.rbase = lo;
            o.pbase = sh.bucket_pack_base[q];
            o.width = sh.bucket_width[q];
            o.pp = sh.bucket_packed_packs[q];
            o.pt = sh.bucket_packed_tasks[q];
        }
    }
    return o;
}

// The pack that task `task` starts (its index, and its task count in `count`), or -1
// when the task is inside a pack.  Within a bucket the first packed_tasks tasks form
// packs of `width`, the rest are singletons (make_order_and_packs, kernels/plan.py:48-100).
__device__ __forceinline__ int32_t pack_of(const BucketOf &o, int32_t task, int32_t hkv, int32_t &count) {
    const int32_t p = task - o.rbase * hkv;
    if (p < o.pt) {
        count = o.width;
        return p % o.width == 0 ? o.pbase + p / o.width : -1;
    }
    count = 1;
    return o.pbase + o.pp + (p - o.pt);
}

// ---------------------------------------------------------------- mode, order, packs
// weight is read through the given pointer (global, or the fused kernel's LDS copy);
// total = record count.  Leaves the selected mode in sh.mode.
__device__ void stage_order_and_packs(const int32_t *weight, int32_t total, int32_t *order,
                                      int32_t *pack_first, int32_t *pack_count, int32_t *num_packs,
                                      int32_t *mode_out, const int32_t *rules, int32_t rule_count,
                                      int32_t force, int32_t hkv, int32_t workers, int32_t buckets,
                                      int32_t record_capacity, PlanShared &sh,
                                      int16_t *order_mirror = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int per = (record_capacity + kPlanThreads - 1) / kPlanThreads;
    const int i0 = tid * per;
    // max/min weight over valid records (max starts at 1, min at INT32_MAX as plan.py:57-58)
    int32_t mx = 1, mn = INT32_MAX;
    for (int k = 0; k < per; ++k) {
        const int i = i0 + k;
        if (i >= total) break;
        const int32_t w = weight[i];
        mx = max(mx, w);
        mn = min(mn, w);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mx = max(mx, __shfl_xor(mx, o, 64));
        mn = min(mn, __shfl_xor(mn, o, 64));
    }
    if (lane == 0) { sh.red_max[wid] = mx; sh.red_min[wid] = mn; }
    lds_barrier();
    if (tid == 0) {
        int32_t a = 1, b = INT32_MAX;
        for (int w = 0; w < kPlanThreads / 64; ++w) { a = max(a, sh.red_max[w]); b = min(b, sh.red_min[w]); }
        const int32_t ratio = wmul(a, 100) / max(b, 1);
        const int32_t tasks = wmul(total, hkv);
        int32_t mode = 1;
        for (int row = 0; row < rule_count; ++row) {
            const int32_t *r = rules + 5 * row;
            if (tasks >= r[0] && tasks <= r[1] && ratio >= r[2] && ratio <= r[3]) mode = r[4];
        }
        if (a == b) mode = 1;
        if (force >= 0) mode = force;
        sh.mode = mode;
        sh.max_w = a;
        *mode_out = mode;
    }
    lds_barrier();
    const int32_t mode = sh.mode, max_w = sh.max_w;
    if (mode == 0 || mode == 1) {
        for (int i = tid; i < total; i += kPlanThreads) order[i] = i;
        if (tid == 0) {
            *num_packs = 0;
            sh.num_packs = 0;
        }
        return;
    }
    // Stable partition by bucket, heaviest first, in passes of kPlanThreads records
    // (record i = pass base + thread): each wave ranks its lanes within their bucket by
    // ballot, and the waves' counts meet in LDS.  First the bucket sizes ...
    if (tid < kMaxBuckets) {
        sh.bucket_size[tid] = 0;
        sh.carry[tid] = 0;
    }
    lds_barrier();
    for (int p0 = 0; p0 < total; p0 += kPlanThreads) {
        const int i = p0 + tid;
        const int b = i < total ? bucket_of(weight[i], buckets) : -1;
        for (int q = 0; q < buckets; ++q) {
            const uint64_t m = __ballot(b == q);
            if (lane == q && m) atomicAdd(&sh.bucket_size[q], (int32_t)__popcll(m));
        }
    }
    lds_barrier();
    // ... then the bucket tables, lane b of wave 0 for bucket b (bases run over the
    // heavier buckets b' > b) ...
    if (wid == 0) {
        const int b = lane;
        const bool live = b < buckets;
        const int32_t size = live ? sh.bucket_size[b] : 0;
        const int32_t tasks = size * hkv;
        const int32_t width = (live && mode == 4) ? min(4, max(1, max_w / (1 << b))) : 1;
        const int32_t packed_tasks = max(0, tasks - workers) / width * width;
        const int32_t packed_packs = packed_tasks / width;
        const int32_t count = live ? packed_packs + tasks - packed_tasks : 0;
        int32_t rec_base = 0, pack_base = 0, packs = 0;
        for (int q = 0; q < kMaxBuckets; ++q) {
            const int32_t sq = __builtin_amdgcn_readlane(size, q), cq = __builtin_amdgcn_readlane(count, q);
            if (q > b) {
                rec_base += sq;
                pack_base += cq;
            }
            packs += cq;
        }
        if (b < kMaxBuckets) {
            sh.bucket_record_base[b] = rec_base;
            sh.bucket_pack_base[b] = pack_base;
            sh.bucket_pack_count[b] = count;
            sh.bucket_width[b] = width;
            sh.bucket_packed_packs[b] = packed_packs;
            sh.bucket_packed_tasks[b] = packed_tasks;
        }
        if (lane == 0) {
            *num_packs = packs;
            sh.num_packs = packs;
        }
    }
    lds_barrier();
    // ... then each record's rank: earlier passes, earlier waves, earlier lanes.
    for (int p0 = 0; p0 < total; p0 += kPlanThreads) {
        const int i = p0 + tid;
        const int b = i < total ? bucket_of(weight[i], buckets) : -1;
        uint64_t same = 0;
        int32_t lane_count = 0;
        for (int q = 0; q < buckets; ++q) {
            const uint64_t m = __ballot(b == q);
            if (b == q) same = m;
            if (lane == q) lane_count = (int32_t)__popcll(m);
        }
        if (lane < kMaxBuckets) sh.hist[wid][lane] = lane_count;
        lds_barrier();
        if (b >= 0) {
            int32_t r = sh.carry[b] + (int32_t)__popcll(same & ((1ull << lane) - 1));
            for (int w = 0; w < wid; ++w) r += sh.hist[w][b];
            const int32_t pos = sh.bucket_record_base[b] + r;
            order[pos] = i;
            if (order_mirror) order_mirror[pos] = (int16_t)i;
        }
        lds_barrier();
        if (tid < kMaxBuckets) {
            int32_t n = 0;
            for (int w = 0; w < kPlanThreads / 64; ++w) n += sh.hist[w][tid];
            sh.carry[tid] += n;
        }
        lds_barrier();
    }
    // Pack tables, one task per thread (consecutive threads, consecutive tasks: the
    // stores of a wave land on neighbouring pack entries, not one record's Hkv tasks
    // per lane): a task that starts a pack writes it.
    const int32_t ntasks = wmul(total, hkv);
    for (int32_t task = tid; task < ntasks; task += kPlanThreads) {
        const BucketOf o = bucket_at(sh, task / hkv, buckets);
        int32_t count;
        const int32_t unit = pack_of(o, task, hkv, count);
        if (unit >= 0) {
            pack_first[unit] = task;
            pack_count[unit] = count;
        }
    }
}

// ---------------------------------------------------------------- STATIC lists
// Longest-processing-time assignment (kernels/plan.py:103-135, planning/reference.py:
// 57-67): tasks in (-weight, task) order, each to the worker with the least (load,
// worker).  The records are sorted once (bitonic, in LDS); the assignment runs in
// rounds that are provably the sequential choice:
//
// Keep the workers sorted by key (load << 32 | worker).  Within a run of tasks of equal
// weight w, with S the sorted keys and T = S[0] + (w << 32) (the first worker's key
// after it takes a task), let k = #{i : S[i] < T}.  Sequentially, the next k tasks go
// to S[0], S[1], ..., S[k-1] in that order: when S[i] (i < k) is due, every worker
// already given a task this round has key S[j] + (w << 32) >= T > S[i] (S[j] <= S[i]),
// and every other worker has a key >= S[i]; after S[k-1] the least key is T, S[0]'s.
// So a round assigns min(k, tasks left in the run) tasks at once, then merges the
// raised keys S[0..m) + (w << 32) (still sorted) with the untouched S[m..) (sorted)
// by binary-search placement.  Keys are distinct (distinct workers), so the merge has
// no ties.  A balanced plan takes about tasks / workers rounds; any plan at most one
// round per task.  Each list is written as it grows: a worker's first task to
// static_head, each later one to static_next of its previous task, and a final pass
// terminates the lists (every entry is written once, so no ordering between the
// rounds' global stores is needed).
constexpr int kGreedyMaxRecords = 16384;
constexpr int kGreedyMaxWorkers = 4096;

struct LptLds {
    uint64_t key[2][kGreedyMaxWorkers];  // sorted worker keys, double-buffered across rounds
    int32_t tail[kGreedyMaxWorkers];     // each worker's last task, -1 before its first
};

struct GreedyShared {
    uint32_t keys[kGreedyMaxRecords];  // (0xffff - weight) << 16 | record, sorted ascending
    LptLds lpt;
};

// First index i in [lo, hi) with a[i] >= x (a ascending), by binary search.
__device__ __forceinline__ int32_t lower_bound_u64(const uint64_t *a, int32_t lo, int32_t hi, uint64_t x) {
    while (lo < hi) {
        const int32_t mid = (lo + hi) >> 1;
        if (a[mid] < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// keys: LDS array of kGreedyMaxRecords entries; weight may alias it (the fused kernel's
// LDS weights become the keys in place: each index is read and then written by the same
// thread).
__device__ void stage_greedy_lists(const int32_t *weight, int32_t total, int32_t mode, int32_t *static_head,
                                   int32_t *static_next, int32_t hkv, int32_t workers, uint32_t *keys,
                                   LptLds &g) {
    if (mode != 2) return;
    const int tid = threadIdx.x;
    int n2 = 1;
    while (n2 < total) n2 <<= 1;
    for (int i = tid; i < n2; i += kPlanThreads)
        keys[i] = i < total ? ((uint32_t)(0xffff - weight[i]) << 16) | (uint32_t)i : 0xffffffffu;
    for (int w = tid; w < workers; w += kPlanThreads) {
        g.key[0][w] = (uint64_t)(uint32_t)w;  // load 0: sorted by worker
        g.tail[w] = -1;
    }
    lds_barrier();
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < n2; i += kPlanThreads) {
                const int p = i ^ j;
                if (p > i) {
                    const uint32_t a = keys[i], b = keys[p];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) { keys[i] = b; keys[p] = a; }
                }
            }
            lds_barrier();
        }
    }
    const int64_t ntasks = (int64_t)total * hkv;
    int cur = 0;
    for (int64_t q = 0; q < ntasks;) {
        // the run of records with the weight of sorted record q / hkv
        const uint32_t hi = keys[q / hkv] >> 16;
        const int32_t w = 0xffff - (int32_t)hi;
        int32_t lo_r = (int32_t)(q / hkv) + 1, hi_r = total;  // first sorted record of another weight
        while (lo_r < hi_r) {
            const int32_t mid = (lo_r + hi_r) >> 1;
            if ((keys[mid] >> 16) == hi) lo_r = mid + 1;
            else hi_r = mid;
        }
        const int64_t run_end = (int64_t)lo_r * hkv;
        while (q < run_end) {
            const uint64_t *S = g.key[cur];
            uint64_t *out = g.key[cur ^ 1];
            const uint64_t raise = (uint64_t)(uint32_t)w << 32;
            const int32_t k = lower_bound_u64(S, 1, workers, S[0] + raise);
            const int32_t m = (int32_t)min((int64_t)k, run_end - q);
            for (int i = tid; i < workers; i += kPlanThreads) {
                const uint64_t s = S[i];
                if (i < m) {
                    // task q + i of the sorted stream goes to worker S[i]
                    const int64_t qi = q + i;
                    const int32_t rec = (int32_t)(keys[qi / hkv] & 0xffff);
                    const int32_t task = rec * hkv + (int32_t)(qi % hkv);
                    const int32_t worker = (int32_t)(uint32_t)s;
                    const int32_t prev = g.tail[worker];
                    if (prev < 0) static_head[worker] = task;
                    else static_next[prev] = task;
                    g.tail[worker] = task;
                    const uint64_t up = s + raise;
                    out[i + lower_bound_u64(S, m, workers, up) - m] = up;
                } else {
                    // untouched key: behind the raised keys below it
                    int32_t lo = 0, hi2 = m;
                    while (lo < hi2) {
                        const int32_t mid = (lo + hi2) >> 1;
                        if (S[mid] + raise < s) lo = mid + 1;
                        else hi2 = mid;
                    }
                    out[(i - m) + lo] = s;
                }
            }
            lds_barrier();
            cur ^= 1;
            q += m;
        }
    }
    for (int w = tid; w < workers; w += kPlanThreads) {
        const int32_t last = g.tail[w];
        if (last < 0) static_head[w] = -1;
        else static_next[last] = -1;
    }
}

// ---------------------------------------------------------------- dispatch table
// One entry per dispatch unit with its record resolved, so an attention launch goes
// from a unit straight to its rows: {first task, tasks in the unit, request, split,
// begin, end, kv group, kind}.  Units follow the mode the plan chose: tasks for R1
// and STATIC (kind 1, task t is record t / Hkv: STATIC reads records directly and
// R1's order is the identity, kernels/attention.py:41-47), packs for D1/D4 (kind 2,
// pack u located in the bucket tables exactly as stage_order_and_packs lays the packs
// out, its first record through the order).  Nothing is written for R0.  Everything
// comes from LDS: record rec is (request_of(rec), rec - offsets[r]), with begin and end
// computed as stage_emit_records computes them.
__device__ void stage_dispatch_table(int32_t *table, int32_t capacity, const int16_t *order_mirror,
                                     const RowMirror &rows, int32_t bcap, int32_t total, int32_t hkv,
                                     int32_t buckets, const PlanShared &sh) {
    const int32_t mode = sh.mode;
    if (mode == 0) return;
    // one task per thread, so a wave writes neighbouring entries (the Hkv lanes of a
    // record find its request together: their LDS reads are broadcasts)
    const int32_t ntasks = wmul(total, hkv);
    for (int32_t task = threadIdx.x; task < ntasks; task += kPlanThreads) {
        const int32_t j = task / hkv, g = task - j * hkv;
        const int32_t rec = mode >= 3 ? (int32_t)order_mirror[j] : j;
        const int32_t r = request_of(rows.offsets, bcap, rec);
        const int32_t s = wadd(rec, -rows.offsets[r]);
        const int32_t c = rows.chunk[r];
        const int32_t b = wmul(s, c);
        const int32_t e = min(wadd(b, c), rows.lengths[r]);
        int32_t count = 1, unit = task;
        if (mode >= 3) unit = pack_of(bucket_at(sh, j, buckets), task, hkv, count);
        if (unit < 0 || unit >= capacity) continue;
        int32_t *ent = table + 8 * (int64_t)unit;
        *reinterpret_cast<int4 *>(ent) = make_int4(task, count, r, s);
        *reinterpret_cast<int4 *>(ent + 4) = make_int4(b, e, g, mode >= 3 ? 2 : 1);
    }
}

// ---------------------------------------------------------------- kernels
__global__ __launch_bounds__(kPlanThreads) void k_count_scan(const int32_t *lengths, const int32_t *splits,
                                                             const int32_t *active, int32_t *counts,
                                                             int32_t *offsets, int32_t *chunk,
                                                             int32_t *record_count, int32_t *error,
                                                             int32_t bcap, int32_t smax, int32_t max_context) {
    __shared__ PlanShared sh;
    stage_count_scan(lengths, splits, active, counts, offsets, chunk, record_count, error, bcap, smax,
                     max_context, sh);
}

__global__ __launch_bounds__(kPlanThreads) void k_emit_records(const int32_t *lengths, const int32_t *counts,
                                                               const int32_t *offsets, const int32_t *chunk,
                                                               int32_t *request, int32_t *split, int32_t *begin,
                                                               int32_t *end, int32_t *weight, int32_t bcap,
                                                               int32_t smax, int32_t block_kv) {
    stage_emit_records(lengths, counts, offsets, chunk, request, split, begin, end, weight, bcap, smax,
                       block_kv);
}

__global__ __launch_bounds__(kPlanThreads) void k_order_and_packs(
    const int32_t *weight, const int32_t *record_count, int32_t *order, int32_t *pack_first,
    int32_t *pack_count, int32_t *num_packs, int32_t *mode, const int32_t *rules, int32_t rule_count,
    int32_t force, int32_t hkv, int32_t workers, int32_t buckets, int32_t record_capacity) {
    __shared__ PlanShared sh;
    stage_order_and_packs(weight, *record_count, order, pack_first, pack_count, num_packs, mode, rules,
                          rule_count, force, hkv, workers, buckets, record_capacity, sh);
}

__global__ __launch_bounds__(kPlanThreads) void k_greedy_lists(const int32_t *weight, const int32_t *record_count,
                                                               const int32_t *mode, int32_t *static_head,
                                                               int32_t *static_next, int32_t hkv,
                                                               int32_t workers) {
    extern __shared__ char dyn[];
    GreedyShared &g = *reinterpret_cast<GreedyShared *>(dyn);
    stage_greedy_lists(weight, *record_count, *mode, static_head, static_next, hkv, workers, g.keys, g.lpt);
}

// Dynamic LDS of the fused kernel.  Region A holds the per-row values (lengths,
// offsets, chunks) from count/scan through the dispatch table, with the order mirror
// (int16: records < 16384) that the dispatch table reads; the LPT's worker keys and
// tails take it over afterwards.  Region B holds the record weights between emission,
// ordering and the LPT, where they become the sort keys.
struct FusedLds {
    union {
        struct {
            struct {
                int32_t lengths[4096], offsets[4097], chunk[4096];
            } rows;
            int16_t order[kGreedyMaxRecords];
        } pre;
        LptLds lpt;
    } a;
    union {
        int32_t weight[kGreedyMaxRecords];
        uint32_t keys[kGreedyMaxRecords];
    } b;
};
static_assert(sizeof(FusedLds) <= 160 * 1024, "fused plan LDS");

// All stages in one launch; every intermediate that a later stage reads stays in LDS,
// so the stages wait on no global round trip of their own outputs.
__global__ __launch_bounds__(kPlanThreads) void k_build_plan(sgd_plan_buffers p, int32_t force, int32_t run_greedy,
                                                             int32_t *zero_counters, int32_t num_counters,
                                                             const int32_t *csr_indptr, const int32_t *csr_splits,
                                                             int32_t csr_batch) {
    __shared__ PlanShared sh;
    extern __shared__ __align__(16) char dyn[];
    FusedLds &L = *reinterpret_cast<FusedLds *>(dyn);
    for (int i = threadIdx.x; i < num_counters; i += kPlanThreads) zero_counters[i] = 0;
    // The policy rules go to LDS: loaded (one int per thread, index clamped into the
    // buffer, which holds at least one row) together with count/scan's loads, stored
    // after it, published by the barrier that follows.
    static_assert(5 * kLdsRules <= kPlanThreads, "one rule int per thread");
    const bool rules_lds = p.rule_count <= kLdsRules;
    const int32_t rule_v = p.rules[min((int)threadIdx.x, 5 * max(p.rule_count, 1) - 1)];
    const RowMirror mirror{L.a.pre.rows.lengths, nullptr, L.a.pre.rows.offsets, L.a.pre.rows.chunk};
    const CsrRows csr{csr_indptr, csr_splits, csr_batch, p.lengths, p.splits, p.active};
    stage_count_scan(p.lengths, p.splits, p.active, p.counts, p.offsets, p.chunk, p.record_count, p.error,
                     p.batch_capacity, p.max_splits, p.max_context, sh, &mirror, csr_indptr ? &csr : nullptr);
    if (rules_lds && (int)threadIdx.x < 5 * p.rule_count) sh.rules[threadIdx.x] = rule_v;
    if (force == 0) {  // forced R0: counts/offsets only (planning/builder.py:11-14)
        if (threadIdx.x == 0) { *p.mode = 0; *p.num_packs = 0; }
        return;
    }
    lds_barrier();
    const int32_t total = sh.record_count;
    stage_emit_by_record(mirror, total, p.batch_capacity, p.request, p.split, p.begin, p.end, p.weight, p.block_kv,
                         L.b.weight);
    lds_barrier();
    stage_order_and_packs(L.b.weight, total, p.order, p.pack_first, p.pack_count, p.num_packs, p.mode,
                          rules_lds ? sh.rules : p.rules,
                          p.rule_count, force, p.kv_heads, p.workers, p.buckets, p.batch_capacity * p.max_splits,
                          sh, L.a.pre.order);
    if (p.dispatch) {
        lds_barrier();
        stage_dispatch_table(p.dispatch, p.batch_capacity * p.max_splits * p.kv_heads, L.a.pre.order, mirror,
                             p.batch_capacity, total, p.kv_heads, p.buckets, sh);
    }
    if (run_greedy) {
        lds_barrier();
        // the LPT's worker keys and tails take region A (free by now), its keys replace the weights
        stage_greedy_lists(L.b.weight, total, sh.mode, p.static_head, p.static_next, p.kv_heads, p.workers,
                           L.b.keys, L.a.lpt);
    }
}

bool greedy_attr[kOnceDevices] = {}, build_attr[kOnceDevices] = {};

int prepare_plan_launch() {
    if (int rc = set_dynamic_lds((const void *)k_greedy_lists, (int)sizeof(GreedyShared), greedy_attr, "greedy_lists"))
        return rc;
    return set_dynamic_lds((const void *)k_build_plan, (int)sizeof(FusedLds), build_attr, "build_plan");
}

int check_plan_geometry(int32_t bcap, int32_t smax, int32_t hkv, int32_t workers, int32_t buckets) {
    if (bcap <= 0 || bcap > 4096) return einval("batch_capacity %d outside [1, 4096]", bcap);
    if (smax <= 0 || (int64_t)bcap * smax > kGreedyMaxRecords)
        return einval("record capacity %lld outside [1, %d]", (long long)bcap * smax, kGreedyMaxRecords);
    if (hkv <= 0 || (int64_t)bcap * smax * hkv >= (1ll << 31)) return einval("task capacity overflow");
    if (workers <= 0 || workers > kGreedyMaxWorkers) return einval("workers %d outside [1, %d]", workers,
                                                                     kGreedyMaxWorkers);
    if (buckets <= 0 || buckets > kMaxBuckets) return einval("buckets %d outside [1, %d]", buckets, kMaxBuckets);
    return 0;
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_count_scan(const int32_t *lengths, const int32_t *splits, const int32_t *active,
                              int32_t *counts, int32_t *offsets, int32_t *chunk, int32_t *record_count,
                              int32_t *error, int32_t bcap, int32_t smax, int32_t max_context, void *stream) {
    if (bcap <= 0 || bcap > 4096 || smax <= 0) return einval("count_scan: bcap %d / smax %d", bcap, smax);
    clear_stale_error();
    hipLaunchKernelGGL(k_count_scan, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, lengths, splits,
                       active, counts, offsets, chunk, record_count, error, bcap, smax, max_context);
    return launch_status("count_scan");
}

extern "C" int sgd_emit_records(const int32_t *lengths, const int32_t *counts, const int32_t *offsets,
                                const int32_t *chunk, int32_t *request, int32_t *split, int32_t *begin,
                                int32_t *end, int32_t *weight, int32_t bcap, int32_t smax, int32_t block_kv,
                                void *stream) {
    if (bcap <= 0 || smax <= 0 || block_kv <= 0) return einval("emit_records: bad geometry");
    clear_stale_error();
    hipLaunchKernelGGL(k_emit_records, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, lengths, counts,
                       offsets, chunk, request, split, begin, end, weight, bcap, smax, block_kv);
    return launch_status("emit_records");
}

extern "C" int sgd_order_and_packs(const int32_t *weight, const int32_t *record_count, int32_t *order,
                                   int32_t *pack_first, int32_t *pack_count, int32_t *num_packs, int32_t *mode,
                                   const int32_t *rules, int32_t rule_count, int32_t force_mode,
                                   int32_t kv_heads, int32_t workers, int32_t buckets,
                                   int32_t record_capacity, void *stream) {
    if (record_capacity <= 0 || record_capacity > kGreedyMaxRecords || kv_heads <= 0 || workers <= 0 ||
        buckets <= 0 || buckets > kMaxBuckets || rule_count < 0)
        return einval("order_and_packs: bad geometry");
    if (force_mode < -1 || force_mode > 4) return einval("order_and_packs: force_mode %d outside [-1, 4]", force_mode);
    clear_stale_error();
    hipLaunchKernelGGL(k_order_and_packs, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, weight,
                       record_count, order, pack_first, pack_count, num_packs, mode, rules, rule_count,
                       force_mode, kv_heads, workers, buckets, record_capacity);
    return launch_status("order_and_packs");
}

extern "C" int sgd_greedy_lists(const int32_t *weight, const int32_t *record_count, const int32_t *mode,
                                int32_t *static_head, int32_t *static_next, int32_t kv_heads, int32_t workers,
                                int32_t record_capacity, void *stream) {
    if (record_capacity <= 0 || record_capacity > kGreedyMaxRecords || kv_heads <= 0 || workers <= 0 ||
        workers > kGreedyMaxWorkers)
        return einval("greedy_lists: bad geometry");
    if (int rc = prepare_plan_launch()) return rc;
    clear_stale_error();
    hipLaunchKernelGGL(k_greedy_lists, dim3(1), dim3(kPlanThreads), sizeof(GreedyShared), (hipStream_t)stream,
                       weight, record_count, mode, static_head, static_next, kv_heads, workers);
    return launch_status("greedy_lists");
}

namespace {

int launch_build_plan(const sgd_plan_buffers *plan, int32_t force_mode, int32_t run_greedy, int32_t *zero_counters,
                      int32_t num_counters, const int32_t *kv_indptr, const int32_t *num_kv_splits, int32_t batch,
                      void *stream) {
    if (!plan) return einval("build_plan: null plan");
    if (force_mode < -1 || force_mode > 4) return einval("build_plan: force_mode %d outside [-1, 4]", force_mode);
    if (int rc = check_plan_geometry(plan->batch_capacity, plan->max_splits, plan->kv_heads, plan->workers,
                                     plan->buckets))
        return rc;
    if (plan->rule_count < 0) return einval("build_plan: negative rule_count");
    if (num_counters < 0 || (num_counters > 0 && !zero_counters)) return einval("build_plan: counters");
    if (int rc = prepare_plan_launch()) return rc;
    clear_stale_error();
    hipLaunchKernelGGL(k_build_plan, dim3(1), dim3(kPlanThreads), sizeof(FusedLds), (hipStream_t)stream, *plan,
                       force_mode, run_greedy, zero_counters, num_counters, kv_indptr, num_kv_splits, batch);
    return launch_status("build_plan");
}

}  // namespace

extern "C" int sgd_build_plan(const sgd_plan_buffers *plan, int32_t force_mode, int32_t run_greedy,
                              int32_t *zero_counters, int32_t num_counters, void *stream) {
    return launch_build_plan(plan, force_mode, run_greedy, zero_counters, num_counters, nullptr, nullptr, 0, stream);
}

extern "C" int sgd_build_plan_csr(const sgd_plan_buffers *plan, const int32_t *kv_indptr,
                                  const int32_t *num_kv_splits, int32_t batch, int32_t force_mode,
                                  int32_t run_greedy, int32_t *zero_counters, int32_t num_counters, void *stream) {
    if (!kv_indptr || !num_kv_splits) return einval("build_plan_csr: kv_indptr and num_kv_splits are required");
    if (plan && (batch < 0 || batch > plan->batch_capacity))
        return einval("build_plan_csr: batch %d outside [0, %d]", batch, plan->batch_capacity);
    return launch_build_plan(plan, force_mode, run_greedy, zero_counters, num_counters, kv_indptr, num_kv_splits,
                             batch, stream);
}
