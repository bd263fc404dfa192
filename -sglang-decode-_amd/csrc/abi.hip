// C-ABI plumbing shared by the HIP sources: thread-local error text, launch
// status mapping, version string, and the host (C++) LPT static planner.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <queue>
#include <utility>
#include <vector>

#include "common.h"

namespace sgd {

static thread_local char g_error[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int einval(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return SGD_EINVAL;
}

void clear_stale_error() { (void)hipGetLastError(); }

int set_dynamic_lds(const void *kernel, int bytes, bool *done, const char *what) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    const bool cached = dev >= 0 && dev < kOnceDevices;
    if (cached && done[dev]) return 0;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
        return einval("%s: cannot reserve %d B of LDS", what, bytes);
    if (cached) done[dev] = true;
    return 0;
}

int launch_status(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return 0;
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
}

}  // namespace sgd

extern "C" const char *sgd_last_error(void) { return sgd::g_error; }

extern "C" const char *sgd_version(void) { return "sglang_decode_hip 0.1.0 gfx950"; }

namespace {

// Heap LPT of planning/reference.py:57-67 over records with these weights, into
// static_head [workers] / static_next [task_capacity] (see sgd_host_static_lists).
void heap_lpt(const int32_t *weight, int32_t record_count, int32_t kv_heads, int32_t workers,
              int32_t task_capacity, int32_t *static_head, int32_t *static_next) {
    // Records sorted by (-weight, record); a record's tasks are consecutive ids, so
    // this is the (-weight, task) order of the reference.
    std::vector<int32_t> recs(record_count);
    for (int32_t i = 0; i < record_count; ++i) recs[i] = i;
    std::stable_sort(recs.begin(), recs.end(), [&](int32_t a, int32_t b) { return weight[a] > weight[b]; });
    using Entry = std::pair<int64_t, int32_t>;  // (load, worker), min-heap
    std::priority_queue<Entry, std::vector<Entry>, std::greater<Entry>> heap;
    for (int32_t w = 0; w < workers; ++w) heap.emplace(0, w);
    std::vector<int32_t> tail(workers, -1);
    for (int32_t w = 0; w < workers; ++w) static_head[w] = -1;
    for (int32_t t = 0; t < task_capacity; ++t) static_next[t] = -1;
    for (int32_t rec : recs) {
        for (int32_t g = 0; g < kv_heads; ++g) {
            const int32_t task = rec * kv_heads + g;
            const Entry top = heap.top();
            heap.pop();
            const int32_t w = top.second;
            if (tail[w] < 0) static_head[w] = task;
            else static_next[tail[w]] = task;
            tail[w] = task;
            heap.emplace(top.first + weight[rec], w);
        }
    }
}

}  // namespace

// Heap LPT of planning/reference.py:57-67: tasks ordered by (-weight, task id),
// each popped onto the (load, worker)-least worker; lists stored the way
// benchmarks/bench_decode.py:16-30 uploads them (head per worker, -1 terminated
// next links, every other link -1).
extern "C" int sgd_host_static_lists(const int32_t *weight, int32_t record_count, int32_t kv_heads,
                                     int32_t workers, int32_t task_capacity, int32_t *static_head,
                                     int32_t *static_next) {
    if (record_count < 0 || kv_heads <= 0 || workers <= 0 || !static_head || !static_next ||
        (int64_t)record_count * kv_heads > task_capacity)
        return sgd::einval("host_static_lists: bad arguments");
    if (record_count > 0 && !weight) return sgd::einval("host_static_lists: null weight");
    heap_lpt(weight, record_count, kv_heads, workers, task_capacity, static_head, static_next);
    return 0;
}

// The same lists straight from the step's lengths and split counts: the records of
// kernels/plan.py:7-45 (chunk = ceil(ceil(L / S) / 32) * 32, records [s * chunk,
// min((s + 1) * chunk, L)), weight = ceil(tokens / block_kv)) built in C++, then the
// heap LPT -- no per-record host objects on the per-call path.
extern "C" int sgd_host_static_plan(const int32_t *lengths, const int32_t *splits, int32_t batch,
                                    int32_t max_splits, int32_t max_context, int32_t block_kv, int32_t kv_heads,
                                    int32_t workers, int32_t task_capacity, int32_t *static_head,
                                    int32_t *static_next, int32_t *record_count) {
    if (batch < 0 || max_splits <= 0 || max_context < 0 || block_kv <= 0 || kv_heads <= 0 || workers <= 0 ||
        task_capacity < 0 || !static_head || !static_next || (batch > 0 && (!lengths || !splits)))
        return sgd::einval("host_static_plan: bad arguments");
    constexpr int32_t kAlign = 32;  // split alignment of the plan (kernels/plan.py:19)
    std::vector<int32_t> weight;
    weight.reserve((size_t)batch * 2);
    for (int32_t r = 0; r < batch; ++r) {
        const int32_t len = lengths[r], sp = splits[r];
        if (len < 0 || len > max_context || sp < 1 || sp > max_splits)
            return sgd::einval("host_static_plan: request %d has length %d / splits %d outside [0, %d] / [1, %d]", r,
                               len, sp, max_context, max_splits);
        const int32_t chunk = ((len + sp - 1) / sp + kAlign - 1) / kAlign * kAlign;
        for (int32_t b = 0; b < len; b += chunk) {
            const int32_t e = std::min(b + chunk, len);
            weight.push_back((e - b + block_kv - 1) / block_kv);
        }
    }
    const int64_t n = (int64_t)weight.size();
    if (n * kv_heads > task_capacity)
        return sgd::einval("host_static_plan: %lld records x %d kv heads exceed the task capacity %d", (long long)n,
                           kv_heads, task_capacity);
    heap_lpt(weight.data(), (int32_t)n, kv_heads, workers, task_capacity, static_head, static_next);
    if (record_count) *record_count = (int32_t)n;
    return 0;
}
