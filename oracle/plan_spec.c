/*
 * ORACLE -- test infrastructure only.
 *
 * CPU restatement of the reference's decode-plan construction and split merge,
 * which the HIP kernels are tested against.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library; the product path never
 * does.  Every function cites the reference file:line it restates (paths are
 * relative to the reference repository root).
 *
 * Integer arithmetic mirrors the reference's 32-bit lane arithmetic: values are
 * int32, "cdiv(a, b)" is (a + b - 1) / b with truncating division, and sums that
 * could overflow are computed through uint32 so they wrap instead of being UB.
 *
 * Pinning: see oracle/__init__.py (the header lists which checks pin each
 * function).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef int32_t i32;

static inline i32 wadd(i32 a, i32 b) { return (i32)((uint32_t)a + (uint32_t)b); }
static inline i32 wsub(i32 a, i32 b) { return (i32)((uint32_t)a - (uint32_t)b); }
static inline i32 wmul(i32 a, i32 b) { return (i32)((uint32_t)a * (uint32_t)b); }
static inline i32 imax(i32 a, i32 b) { return a > b ? a : b; }
static inline i32 imin(i32 a, i32 b) { return a < b ? a : b; }
/* cdiv as the reference's tl.cdiv: (a + b - 1) // b on int32 lanes. */
static inline i32 cdiv(i32 a, i32 b) { return wsub(wadd(a, b), 1) / b; }

/*
 * src/sglang_decode/kernels/plan.py:7-27 (count_scan).
 * Rows r < bcap are all written; rows that are not live get n = 0.
 */
void orc_count_scan(const i32 *lengths, const i32 *splits, i32 active, i32 bcap, i32 smax,
                    i32 max_context, i32 *counts, i32 *offsets, i32 *chunk, i32 *record_count,
                    i32 *error)
{
    i32 any_invalid = 0;
    i32 *n = (i32 *)calloc((size_t)(bcap > 0 ? bcap : 1), sizeof(i32));
    for (i32 r = 0; r < bcap; ++r) {
        i32 live = (r < active) && (r < bcap);
        i32 length = live ? lengths[r] : 0;                 /* plan.py:14 */
        i32 s = live ? splits[r] : 1;                       /* plan.py:15 */
        i32 invalid = live && (length < 0 || length > max_context || s < 1 || s > smax);
        any_invalid |= invalid;
        chunk[r] = wmul(cdiv(cdiv(imax(length, 0), imax(s, 1)), 32), 32);   /* plan.py:18 */
        n[r] = (live && !invalid) ? cdiv(length, imax(chunk[r], 1)) : 0;    /* plan.py:19 */
    }
    i32 err = (active < 0) || (active > bcap) || any_invalid;              /* plan.py:17 */
    i32 running = 0;
    for (i32 r = 0; r < bcap; ++r) {
        i32 v = err ? 0 : n[r];                                            /* plan.py:20 */
        counts[r] = v;
        offsets[r] = running;                                              /* plan.py:21-24 */
        running = wadd(running, v);
    }
    offsets[bcap] = running;                                               /* plan.py:25 */
    *record_count = running;                                               /* plan.py:26 */
    *error = err;                                                          /* plan.py:27 */
    free(n);
}

/* src/sglang_decode/kernels/plan.py:30-45 (emit_records). */
void orc_emit_records(const i32 *lengths, const i32 *counts, const i32 *offsets, const i32 *chunk,
                      i32 bcap, i32 smax, i32 tile, i32 *request, i32 *split, i32 *begin,
                      i32 *end, i32 *weight)
{
    for (i32 r = 0; r < bcap; ++r) {
        i32 n = counts[r];
        for (i32 s = 0; s < smax && s < n; ++s) {
            i32 idx = wadd(offsets[r], s);
            i32 b = wmul(s, chunk[r]);
            i32 e = imin(wadd(b, chunk[r]), lengths[r]);
            request[idx] = r;
            split[idx] = s;
            begin[idx] = b;
            end[idx] = e;
            weight[idx] = cdiv(wsub(e, b), tile);
        }
    }
}

/*
 * src/sglang_decode/kernels/plan.py:48-100 (make_order_and_packs).
 * rules is row-major [rule_count][5] = {min_tasks, max_tasks, min_ratio, max_ratio, mode}.
 */
void orc_order_and_packs(const i32 *weight, i32 total, const i32 *rules, i32 rule_count,
                         i32 force, i32 hkv, i32 workers, i32 buckets, i32 *order,
                         i32 *pack_first, i32 *pack_count, i32 *num_packs, i32 *mode_out)
{
    i32 max_w = 1, min_w = INT32_MAX;
    for (i32 i = 0; i < total; ++i) {
        max_w = imax(max_w, weight[i]);                                    /* plan.py:57 */
        min_w = imin(min_w, weight[i]);                                    /* plan.py:58 */
    }
    i32 ratio = wmul(max_w, 100) / imax(min_w, 1);                         /* plan.py:59 */
    i32 tasks_total = wmul(total, hkv);
    i32 mode = 1;
    for (i32 row = 0; row < rule_count; ++row) {                           /* plan.py:61-66 */
        const i32 *r = rules + 5 * row;
        if (tasks_total >= r[0] && tasks_total <= r[1] && ratio >= r[2] && ratio <= r[3])
            mode = r[4];
    }
    if (max_w == min_w) mode = 1;                                          /* plan.py:68 */
    if (force >= 0) mode = force;                                          /* plan.py:69-70 */
    *mode_out = mode;
    if (mode == 0 || mode == 1) {                                          /* plan.py:72-74 */
        for (i32 i = 0; i < total; ++i) order[i] = i;
        *num_packs = 0;
        return;
    }
    i32 record_base = 0, pack_base = 0;
    for (i32 b = buckets - 1; b >= 0; --b) {                               /* plan.py:83-99 */
        i32 size = 0;
        for (i32 i = 0; i < total; ++i) {
            i32 bucket = 0;                                                /* plan.py:77-79 */
            for (i32 k = 1; k < buckets; ++k) bucket += weight[i] > (1 << (k - 1));
            if (bucket == b) order[record_base + size++] = i;
        }
        i32 tasks = wmul(size, hkv);
        i32 width = (mode == 4) ? imin(4, imax(1, max_w / (1 << b))) : 1;  /* plan.py:90 */
        i32 packed_tasks = imax(0, tasks - workers) / width * width;       /* plan.py:91 */
        i32 packed_packs = packed_tasks / width;
        i32 count = packed_packs + tasks - packed_tasks;
        for (i32 p = 0; p < count; ++p) {                                  /* plan.py:94-97 */
            i32 first = record_base * hkv +
                        (p < packed_packs ? p * width : packed_tasks + p - packed_packs);
            pack_first[pack_base + p] = first;
            pack_count[pack_base + p] = p < packed_packs ? width : 1;
        }
        record_base += size;
        pack_base += count;
    }
    *num_packs = pack_base;                                                /* plan.py:100 */
}

/*
 * src/sglang_decode/kernels/plan.py:103-135 (greedy_lists), the device LPT.
 * Runs only when mode == 2.  static_next entries of unassigned tasks are left
 * untouched, like the reference.
 */
void orc_greedy_lists(const i32 *weight, i32 total, i32 mode, i32 hkv, i32 workers,
                      i32 *static_head, i32 *static_next)
{
    if (mode != 2) return;
    i32 *w = (i32 *)malloc(sizeof(i32) * (size_t)(total > 0 ? total : 1));
    i32 *loads = (i32 *)calloc((size_t)workers, sizeof(i32));
    i32 *tails = (i32 *)malloc(sizeof(i32) * (size_t)workers);
    for (i32 i = 0; i < total; ++i) w[i] = weight[i];
    for (i32 k = 0; k < workers; ++k) { static_head[k] = -1; tails[k] = -1; }
    for (i32 step = 0; step < total; ++step) {
        i32 largest = -1, chosen = 0;
        for (i32 i = 0; i < total; ++i)                                    /* plan.py:121-122 */
            if (w[i] > largest) { largest = w[i]; chosen = i; }
        for (i32 g = 0; g < hkv; ++g) {                                    /* plan.py:123-134 */
            i32 task = chosen * hkv + g, owner = 0;
            for (i32 k = 1; k < workers; ++k)
                if (loads[k] < loads[owner]) owner = k;
            if (tails[owner] < 0) static_head[owner] = task;
            else static_next[tails[owner]] = task;
            static_next[task] = -1;
            loads[owner] += largest;
            tails[owner] = task;
        }
        w[chosen] = -1;                                                    /* plan.py:135 */
    }
    free(w); free(loads); free(tails);
}

/*
 * src/sglang_decode/planning/reference.py:57-67 (greedy_static), the host LPT:
 * tasks sorted by (-weight, task), each popped onto the (load, worker)-minimal
 * worker.  Written as linked lists the way benchmarks/bench_decode.py:16-30
 * converts them: heads[-1 if empty], next[-1 terminated], other links -1.
 */
void orc_greedy_static(const i32 *weight, i32 total, i32 hkv, i32 workers, i32 task_capacity,
                       i32 *static_head, i32 *static_next)
{
    i32 ntask = total * hkv;
    i32 *tasks = (i32 *)malloc(sizeof(i32) * (size_t)(ntask > 0 ? ntask : 1));
    int64_t *loads = (int64_t *)calloc((size_t)workers, sizeof(int64_t));
    i32 *tails = (i32 *)malloc(sizeof(i32) * (size_t)workers);
    /* stable counting order by descending weight, ties by ascending task id */
    i32 maxw = 0;
    for (i32 i = 0; i < total; ++i) maxw = imax(maxw, weight[i]);
    i32 n = 0;
    for (i32 wv = maxw; wv >= 0; --wv)
        for (i32 t = 0; t < ntask; ++t)
            if (weight[t / hkv] == wv) tasks[n++] = t;
    for (i32 k = 0; k < workers; ++k) { static_head[k] = -1; tails[k] = -1; }
    for (i32 t = 0; t < task_capacity; ++t) static_next[t] = -1;
    for (i32 j = 0; j < n; ++j) {
        i32 owner = 0;
        for (i32 k = 1; k < workers; ++k)
            if (loads[k] < loads[owner]) owner = k;
        i32 t = tasks[j];
        if (tails[owner] < 0) static_head[owner] = t;
        else static_next[tails[owner]] = t;
        tails[owner] = t;
        loads[owner] += weight[t / hkv];
    }
    free(tasks); free(loads); free(tails);
}

/*
 * src/sglang_decode/kernels/merge.py:7-30 (merge_splits) in float32.
 * out is float32 [bcap][hq][d]; the caller rounds to the output dtype.
 */
void orc_merge_splits(const float *partial, const float *lse, const i32 *counts, i32 error,
                      i32 bcap, i32 hq, i32 d, i32 smax, float *out)
{
    float *acc = (float *)malloc(sizeof(float) * (size_t)d);
    for (i32 r = 0; r < bcap; ++r) {
        for (i32 h = 0; h < hq; ++h) {
            float m = -INFINITY, den = 0.0f;
            for (i32 k = 0; k < d; ++k) acc[k] = 0.0f;
            for (i32 s = 0; s < counts[r]; ++s) {                           /* merge.py:17-26 */
                int64_t slot = ((int64_t)r * hq + h) * smax + s;
                float l = lse[slot];
                float nm = fmaxf(m, l);
                float ow = expf(m - nm), w = expf(l - nm);
                for (i32 k = 0; k < d; ++k)
                    acc[k] = acc[k] * ow + partial[slot * d + k] * w;
                den = den * ow + w;
                m = nm;
            }
            float *o = out + ((int64_t)r * hq + h) * d;
            for (i32 k = 0; k < d; ++k)                                    /* merge.py:27-30 */
                o[k] = error ? NAN : acc[k] / fmaxf(den, 1.0e-30f);
        }
    }
    free(acc);
}
