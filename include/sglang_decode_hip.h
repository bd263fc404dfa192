/*
 * sglang_decode_hip.h -- C ABI of the MI355X (gfx950) persistent paged GQA
 * decode-attention path.
 *
 * One entry per stage of the reference's launch sequence.  Each entry replaces
 * a Triton `kernel[grid](...)` call of the reference (cited per entry, paths
 * relative to the reference repository root) and is what its Python runtime
 * binds through ctypes.
 *
 * Conventions
 *   - Every pointer argument is a DEVICE pointer unless the comment says host.
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream); every
 *     entry enqueues on it and returns without synchronizing, so all entries are
 *     capturable into a hipGraph.  No entry allocates, frees or reads device
 *     memory from the host.
 *   - Strides are int64 ELEMENT strides (torch's Tensor.stride()).
 *   - Return value: 0 on success, SGD_EINVAL (-22) for arguments outside the
 *     kernels' contract (checked on the host before any launch), otherwise the
 *     hipError_t of the failed launch.  sgd_last_error() gives a message.
 *   - Invalid DEVICE metadata (lengths/splits/active) is never an error code: the
 *     plan sets error=1 and schedules no task, and the merge writes NaN.
 */
#ifndef SGLANG_DECODE_HIP_H
#define SGLANG_DECODE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGD_EINVAL (-22)

enum sgd_dtype { SGD_BF16 = 0, SGD_FP16 = 1 };

/* Attention kernel selection (sgd_decode_args.kernel). */
enum sgd_kernel {
    SGD_KERNEL_AUTO = 0,     /* pick by geometry (see sgd_persistent_decode) */
    SGD_KERNEL_GENERIC = 1,  /* any strides/alignment, any supported geometry */
    SGD_KERNEL_VALU = 2,     /* per-task VALU kernel: LDS-staged K/V tiles, DPP reductions, dot2 (group <= 4) */
    SGD_KERNEL_MFMA = 3      /* MFMA QK^T and PV, K/V straight from HBM into operands (group <= 16) */
};

/* Human-readable description of the last SGD_EINVAL / launch failure (thread-local). */
const char *sgd_last_error(void);

/* Library version string. */
const char *sgd_version(void);

/*
 * Count/scan stage.  Replaces kernels/plan.py:7-27 (count_scan), launched at
 * planning/builder.py:8-10.  For r < bcap: chunk[r] = ceil(ceil(L/S)/32)*32,
 * counts[r] = ceil(L/chunk) (0 for inactive/invalid rows or on error), offsets =
 * exclusive scan with offsets[bcap] = *record_count; *error = 1 when active is
 * outside [0, bcap] or an active row has L < 0, L > max_context, S < 1 or S > smax.
 */
int sgd_count_scan(const int32_t *lengths, const int32_t *splits, const int32_t *active,
                   int32_t *counts, int32_t *offsets, int32_t *chunk, int32_t *record_count,
                   int32_t *error, int32_t bcap, int32_t smax, int32_t max_context, void *stream);

/*
 * Record emission.  Replaces kernels/plan.py:30-45 (emit_records), launched at
 * planning/builder.py:15-18.  Writes SoA records (request, split, begin, end,
 * weight = ceil((end-begin)/block_kv)) at offsets[r] + s for s < counts[r].
 */
int sgd_emit_records(const int32_t *lengths, const int32_t *counts, const int32_t *offsets,
                     const int32_t *chunk, int32_t *request, int32_t *split, int32_t *begin,
                     int32_t *end, int32_t *weight, int32_t bcap, int32_t smax,
                     int32_t block_kv, void *stream);

/*
 * Mode selection, bucket order and packs.  Replaces kernels/plan.py:48-100
 * (make_order_and_packs), launched at planning/builder.py:19-23.  rules is
 * [max(rule_count,1)][5] {min_tasks, max_tasks, min_ratio, max_ratio, mode};
 * last matching rule wins; uniform weights select R1; force_mode >= 0 overrides.
 */
int sgd_order_and_packs(const int32_t *weight, const int32_t *record_count, int32_t *order,
                        int32_t *pack_first, int32_t *pack_count, int32_t *num_packs,
                        int32_t *mode, const int32_t *rules, int32_t rule_count,
                        int32_t force_mode, int32_t kv_heads, int32_t workers, int32_t buckets,
                        int32_t record_capacity, void *stream);

/*
 * Device LPT lists for STATIC mode.  Replaces kernels/plan.py:103-135
 * (greedy_lists), launched at planning/builder.py:24-28.  Does nothing unless
 * *mode == 2.  Produces the lists of planning/reference.py:57-67 (tasks by
 * (-weight, task), each to the (load, worker)-least worker) as static_head /
 * static_next (-1 terminated).
 */
int sgd_greedy_lists(const int32_t *weight, const int32_t *record_count, const int32_t *mode,
                     int32_t *static_head, int32_t *static_next, int32_t kv_heads,
                     int32_t workers, int32_t record_capacity, void *stream);

/* Device plan buffers (all int32, sizes as in runtime/workspace.py:7-23). */
typedef struct sgd_plan_buffers {
    int32_t *lengths, *splits, *active;               /* [bcap], [bcap], [1] */
    int32_t *counts, *offsets, *chunk;                /* [bcap], [bcap+1], [bcap] */
    int32_t *request, *split, *begin, *end, *weight;  /* [E] */
    int32_t *order;                                   /* [E] */
    int32_t *pack_first, *pack_count;                 /* [T] */
    int32_t *record_count, *num_packs, *mode, *error; /* [1] each */
    int32_t *static_head, *static_next;               /* [workers], [T] */
    const int32_t *rules;                             /* [max(rule_count,1)][5] */
    int32_t *dispatch;                                /* optional [T][8] dispatch table, see below; may be NULL */
    int32_t rule_count;
    int32_t batch_capacity, max_splits, max_context, kv_heads, workers, block_kv, buckets;
} sgd_plan_buffers;

/*
 * dispatch (no reference counterpart): one entry per dispatch unit with its first
 * task's record resolved, so that an attention launch goes from a unit to its rows in
 * one round trip instead of pack -> order -> record.  Units are tasks in modes R1 and
 * STATIC (task t), packs in D1/D4 (pack u).  Entry = {first task, tasks in the unit,
 * request, split, begin, end, kv group, kind}, kind 1 = tasks (record t / Hkv; R1's
 * order is the identity), 2 = packs.  Written by sgd_build_plan for the mode it plans
 * (not for R0); a launch uses an entry only when its kind matches the launch's mode
 * (so a table of an R1 plan serves the STATIC lists installed over it).  The table
 * must come from the same plan build as the other buffers.
 *
 * Whole plan build in one launch (count/scan, records, order and packs, and,
 * when run_greedy != 0, the STATIC lists).  Same results as the four stage
 * entries above in the order of planning/builder.py:6-28, including the forced
 * R0 early exit (builder.py:11-14: mode = 0, num_packs = 0, no records).
 * zero_counters/num_counters: optional int32 array cleared by the same launch
 * (per-layer claim counters), may be NULL.
 */
int sgd_build_plan(const sgd_plan_buffers *plan, int32_t force_mode, int32_t run_greedy,
                   int32_t *zero_counters, int32_t num_counters, void *stream);

/*
 * sgd_build_plan with the plan's inputs taken from the step's CSR metadata: replaces
 * the reference adapter's per-step copies before the build
 * (integrations/sglang_backend.py:98-99: plan.lengths[:batch] = kv_indptr[1:batch+1]
 * - kv_indptr[:batch], plan.splits[:batch] = num_kv_splits[:batch]) and the active
 * fill of its metadata hook (:50-55) with reads inside the same launch.  Rows r <
 * batch of plan->lengths / plan->splits and *plan->active (= batch) are also written,
 * as the copies would have; rows >= batch are left as they are (unused).  kv_indptr
 * [>= batch + 1] and num_kv_splits [>= batch] are device int32; 0 <= batch <=
 * batch_capacity.  Lengths and split counts are validated exactly as for
 * sgd_build_plan (a negative length or a split count outside [1, max_splits] sets
 * error).
 */
int sgd_build_plan_csr(const sgd_plan_buffers *plan, const int32_t *kv_indptr, const int32_t *num_kv_splits,
                       int32_t batch, int32_t force_mode, int32_t run_greedy, int32_t *zero_counters,
                       int32_t num_counters, void *stream);

/*
 * The step's CSR metadata from the request pool, in one launch (no counterpart in the
 * reference, which consumes it: integrations/sglang_backend.py:98-107; upstream SGLang
 * v0.4.6.post5 produces it in its triton backend's decode metadata hook).  For rows i <
 * batch: kv_indptr[i+1] = kv_indptr[i] + L_i (kv_indptr[0] = 0), kv_indices[kv_indptr[i]
 * + j] = req_to_token[req_pool_indices[i] * row_stride + j] for j < L_i, with L_i =
 * seq_lens[i].  Split counts by the reference harness rule (benchmarks/workloads.py:
 * 20-21): chunk = max(1, ceil(max L / max_splits)), S_i = clamp(ceil(L_i / chunk), 1,
 * max_splits), written to num_kv_splits when non-NULL.  plan_lengths / plan_splits (both
 * or neither) and plan_active, when non-NULL, receive L_i, S_i and batch: the plan's
 * inputs, so that sgd_build_plan follows without copies.  seq_lens and
 * req_pool_indices are int32 or int64 (flags); req_to_token is int32 [rows, row_stride]
 * with cols usable tokens per row.  A row with L_i < 0, L_i > cols or a pool index outside
 * [0, rows) counts as length 0 and sets *error (when non-NULL); a valid total above
 * indices_capacity makes every row length 0 and sets *error.  Nothing is read or written
 * out of bounds.  0 <= batch <= 4096.
 */
int sgd_csr_metadata(const void *seq_lens, int32_t seq_lens_is_int64, const void *req_pool_indices,
                     int32_t pool_indices_is_int64, const int32_t *req_to_token, int64_t rows,
                     int64_t row_stride, int32_t cols, int32_t batch, int32_t max_splits, int32_t *kv_indptr,
                     int32_t *kv_indices, int64_t indices_capacity, int32_t *num_kv_splits,
                     int32_t *plan_lengths, int32_t *plan_splits, int32_t *plan_active, int32_t *error,
                     void *stream);

/* Arguments of one persistent decode-attention launch. */
typedef struct sgd_decode_args {
    const void *q, *k, *v;          /* q [bcap,Hq,D]; k/v paged [P,page,Hkv,D] or CSR [tok,Hkv,D] */
    const int32_t *pages;           /* paged: table [bcap, max_pages]; CSR: kv_indices */
    const int32_t *indptr;          /* CSR: kv_indptr [bcap+1]; NULL when paged */
    const int32_t *lengths, *request, *split, *begin, *end, *order, *offsets, *chunk;
    const int32_t *active, *record_count, *mode, *pack_first, *pack_count, *num_packs;
    int32_t *counter;               /* per-layer claim counter, zero before the launch */
    int32_t *done_counter;          /* optional (may be NULL): workers that finished; the last
                                       one resets *counter and *done_counter to 0, so the pair is
                                       zero again for the next launch */
    const int32_t *static_head, *static_next;
    float *partial;                 /* [bcap, Hq, smax, D] */
    float *lse;                     /* [bcap, Hq, smax] */
    const int32_t *dispatch;        /* optional: sgd_build_plan's dispatch table of this plan, or NULL */
    float scale;
    int32_t _pad0;
    int64_t q_stride[3], k_stride[4], v_stride[4], pt_stride[2];
    int32_t query_heads, kv_heads, head_dim, max_splits, page_size, csr, dtype, workers;
    int32_t kernel;                 /* enum sgd_kernel */
    int32_t dispatch_units;         /* entries in dispatch; units at or beyond it resolve through
                                       the plan arrays */
    int32_t _pad1;
    void *out;                      /* optional (may be NULL): [bcap, Hq, D] in `dtype`, contiguous.
                                       Every split-0 task also writes its normalized output here,
                                       rounded to dtype.  For a single-split request these are the
                                       bits sgd_merge_splits would write for the row, so
                                       sgd_merge_splits_min(min_splits = 2) can leave it alone; the
                                       other rows hold a split's output until the merge writes them. */
} sgd_decode_args;

/*
 * Persistent paged GQA decode attention.  Replaces kernels/attention.py:87-130
 * (persistent_decode with _attention_task, :12-84), launched at
 * runtime/engine.py:63-70.  One persistent worker per `workers`; tasks are
 * (record, kv head); dispatch follows *mode (R0 binary search, R1 stride,
 * STATIC lists, D1/D4 atomic pack claims on *counter).  Writes the normalized
 * partial output and natural-log LSE of every task into its (request, q head,
 * split) slot.  In D1/D4 worker w runs pack w first (the plan's first wave of
 * packs) and its claims return workers + (counter value): every pack still runs
 * exactly once.
 */
int sgd_persistent_decode(const sgd_decode_args *args, void *stream);

/*
 * The attention kernel (enum sgd_kernel, never AUTO) that sgd_persistent_decode
 * runs for these arguments, or SGD_EINVAL.  No reference counterpart: the
 * reference has one Triton kernel; this reports which gfx950 kernel serves a
 * launch (benchmarks and profiles name it).  Reads no device memory.
 */
int sgd_attention_kernel(const sgd_decode_args *args);

/*
 * Split merge.  Replaces kernels/merge.py:7-30 (merge_splits), launched at
 * runtime/engine.py:71-73.  For every (r < bcap, h): LSE-weighted merge of the
 * counts[r] partials in split order; rows with counts[r] == 0 get 0; *error != 0
 * writes NaN everywhere.  out is [bcap, Hq, D] in `dtype`, contiguous.
 */
int sgd_merge_splits(const float *partial, const float *lse, const int32_t *counts,
                     const int32_t *active, const int32_t *error, void *out, int32_t bcap,
                     int32_t query_heads, int32_t head_dim, int32_t max_splits, int32_t dtype,
                     void *stream);

/*
 * sgd_merge_splits for the rows that need a merge: rows whose request has 1 <= counts[r]
 * < min_splits are left untouched (the attention wrote them through sgd_decode_args.out);
 * rows without splits still get 0 and *error != 0 still writes NaN everywhere.
 * min_splits <= 1 is sgd_merge_splits.  No reference counterpart: the reference merges
 * every row (kernels/merge.py:7-30); with min_splits 2 a batch of mostly single-split
 * requests leaves only its multi-split rows to this launch.
 */
int sgd_merge_splits_min(const float *partial, const float *lse, const int32_t *counts,
                         const int32_t *active, const int32_t *error, void *out, int32_t bcap,
                         int32_t query_heads, int32_t head_dim, int32_t max_splits, int32_t min_splits,
                         int32_t dtype, void *stream);

/*
 * The decode step's writes around the attention, one launch per layer.  Replaces the
 * reference adapter's token_to_kv_pool.set_kv_buffer(layer, out_cache_loc, k, v)
 * (integrations/sglang_backend.py:91-92; upstream two scatters) and
 * qbuf[:batch].copy_(q.view(batch, Hq, D)) (:102-103).  For b < batch:
 *   k_cache[loc[b]] = k_new[b], v_cache[loc[b]] = v_new[b]   ([Hkv, D] rows)
 *   q_out[b] = q_in[b]                                       ([Hq, D] rows)
 * bit for bit (no conversion; 16-bit dtype).  Either part may be skipped: k_new NULL
 * (save_kv_cache off) or q_in NULL.  Strides are element strides of dims 0 and 1 (dim 2
 * has unit stride): new_strides {k0, k1, v0, v1}, cache_strides {k0, k1, v0, v1},
 * q_in_strides / q_out_strides {0, 1}; all multiples of 8 elements and every base
 * 16-byte aligned.  loc is int32, or int64 when loc_is_int64; a slot outside
 * [0, cache_tokens) is skipped on the device.  Returns SGD_EINVAL for misuse.
 */
int sgd_store_kv_stage_q(const void *k_new, const void *v_new, const int64_t *new_strides, const void *loc,
                         int32_t loc_is_int64, void *k_cache, void *v_cache, const int64_t *cache_strides,
                         int64_t cache_tokens, const void *q_in, const int64_t *q_in_strides, void *q_out,
                         const int64_t *q_out_strides, int32_t batch, int32_t kv_heads, int32_t query_heads,
                         int32_t head_dim, int32_t dtype, void *stream);

/*
 * Host (C++) LPT planner: heap assignment of planning/reference.py:57-67 over
 * host records, written as static lists the way benchmarks/bench_decode.py:14-30
 * uploads them.  All pointers are HOST pointers: weight[record_count],
 * static_head[workers], static_next[task_capacity] (every entry written, -1
 * terminated / unused).
 */
int sgd_host_static_lists(const int32_t *weight, int32_t record_count, int32_t kv_heads,
                          int32_t workers, int32_t task_capacity, int32_t *static_head,
                          int32_t *static_next);

/*
 * The same host lists from the step's plan inputs (lengths / splits [batch], host
 * memory): the records of count_scan + emit_records (kernels/plan.py:7-45: chunk =
 * ceil(ceil(L / S) / 32) * 32, weight = ceil(tokens / block_kv)) are formed in C++ and
 * planned by the heap LPT above, as benchmarks/bench_decode.py:14-30 does per call through
 * planning/reference.py:15-67.  Lengths outside [0, max_context], splits outside [1,
 * max_splits] or more than task_capacity tasks are SGD_EINVAL.  *record_count (optional)
 * receives the number of records.
 */
int sgd_host_static_plan(const int32_t *lengths, const int32_t *splits, int32_t batch, int32_t max_splits,
                         int32_t max_context, int32_t block_kv, int32_t kv_heads, int32_t workers,
                         int32_t task_capacity, int32_t *static_head, int32_t *static_next,
                         int32_t *record_count);

/*
 * Upstream SGLang's two-stage split-KV decode on gfx950: the comparator of the reference's
 * benchmark (benchmarks/baselines.py:8-34, over third_party/sglang/decode_attention.py:
 * 245-601 of SGLang v0.4.6.post5: decode_attention_fwd with its grouped stage 1 and its
 * stage 2).  Not on the persistent path.  CSR KV through kv_indptr [batch + 1] /
 * kv_indices; k/v [tokens, kv_heads, 128] with kv_strides = {k token, k head, v token, v
 * head} element strides (unit dim stride), q [batch, Hq, 128] with q_strides.  Stage 1: a
 * grid program per (split s < max_kv_splits, kv head, request b) over tokens [s*c,
 * min((s+1)*c, L_b)), c = ceil(ceil(L_b / S_b) / 32) * 32, S_b = num_kv_splits[b] (clamped
 * to [1, max_kv_splits]), writing the normalized partial and natural-log LSE of each q head
 * to attn_out [batch, Hq, max_kv_splits, 128] / attn_lse [batch, Hq, max_kv_splits] (fp32,
 * contiguous); empty splits write nothing.  Stage 2: out [batch, Hq, 128] (dtype,
 * contiguous) = the LSE merge of each row's non-empty splits (0 for an empty row).  Query
 * groups up to 4.
 */
int sgd_upstream_decode(const void *q, const void *k, const void *v, void *out, const int32_t *kv_indptr,
                        const int32_t *kv_indices, float *attn_out, float *attn_lse, const int32_t *num_kv_splits,
                        int32_t batch, int32_t max_kv_splits, int32_t query_heads, int32_t kv_heads,
                        int32_t head_dim, const int64_t *q_strides, const int64_t *kv_strides, float scale,
                        int32_t dtype, void *stream);

/* Arguments of sgd_decode_noalloc: the inputs of one decode step and its output. */
typedef struct sgd_noalloc_args {
    const void *q, *k, *v;          /* as in sgd_decode_args */
    const int32_t *pages;           /* paged: table [bcap, max_pages]; CSR: kv_indices */
    const int32_t *indptr;          /* CSR: kv_indptr [bcap+1]; NULL when paged */
    const int32_t *lengths, *splits;/* plan inputs [bcap] (as sgd_plan_buffers.lengths / .splits) */
    const int32_t *active;          /* [1] active rows */
    void *out;                      /* [bcap, Hq, D] in `dtype`, contiguous */
    float scale;
    int32_t _pad0;
    int64_t q_stride[3], k_stride[4], v_stride[4], pt_stride[2];
    int32_t batch_capacity, max_splits, max_context, query_heads, kv_heads, head_dim, page_size, csr, dtype,
        workers;
    int32_t force_mode;             /* -1 (R1: no policy rules) or a Mode id to force */
    int32_t kernel;                 /* enum sgd_kernel */
} sgd_noalloc_args;

/*
 * One decode step that allocates nothing: sgd_build_plan (no policy rules, block_kv
 * 128), sgd_persistent_decode and sgd_merge_splits_min on `stream` -- when batch_capacity
 * x Hq exceeds one residency round of the merge (8 rows per CU) the attention writes the
 * single-split rows straight to `out` and the merge takes min_splits 2, otherwise the
 * merge writes every row, as DecodeEngine does -- with the plan and
 * dispatch tables, the claim counters and the split partial/LSE slots in a static
 * device array of 32 MiB held by the library on every GPU it runs on.  No counterpart
 * in the reference: for callers that cannot call hipMalloc (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation); the caller passes
 * only the inputs and `out`.  Geometries whose buffers exceed the array (batch_capacity
 * x max_splits x Hq x head_dim x 4 bytes of split slots, plus the tables) return
 * SGD_EINVAL with the size needed.  The first call on a device looks up the array's
 * address there (make it outside graph capture).  Every call on one GPU reuses that
 * GPU's array: calls that overlap on one GPU race.
 */
int sgd_decode_noalloc(const sgd_noalloc_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SGLANG_DECODE_HIP_H */
