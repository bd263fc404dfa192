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

int launch_status(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return 0;
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
}

}  // namespace sgd

extern "C" const char *sgd_last_error(void) { return sgd::g_error; }

extern "C" const char *sgd_version(void) { return "sglang_decode_hip 0.1.0 gfx950"; }

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
    return 0;
}
