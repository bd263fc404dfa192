// Task decode and persistent dispatch shared by every attention kernel.
//
// A worker is one workgroup.  Its task stream follows the plan's mode exactly as
// kernels/attention.py:87-130: D1/D4 claim pack indices from the per-layer
// counter (one relaxed atomic per claim, :103-106 and :125-126), STATIC walks the
// worker's linked list (:107-109, :127-128), R0/R1 stride by the worker count
// (:110-112, :129-130).  Tasks are (record, kv head) = (task / Hkv, task % Hkv);
// R0 recovers the request by an upper-bound search of the request offsets
// (:25-39), the other modes read the SoA record, through the bucket order except
// in STATIC mode (:41-47).
#pragma once

#include "common.h"

namespace sgd {

struct TaskInfo {
    int32_t request, split, start, end, group;
};

__device__ __forceinline__ TaskInfo decode_task(const sgd_decode_args &a, int32_t task, int32_t mode) {
    TaskInfo t;
    const int32_t hkv = a.kv_heads;
    t.group = task % hkv;
    int32_t rec = task / hkv;
    if (mode == 0) {
        int32_t lo = 0, hi = *a.active;
        while (lo < hi) {
            const int32_t mid = (lo + hi) >> 1;
            if (rec >= a.offsets[mid + 1]) lo = mid + 1;
            else hi = mid;
        }
        t.request = lo;
        t.split = rec - a.offsets[lo];
        const int32_t c = a.chunk[lo];
        t.start = t.split * c;
        t.end = min(t.start + c, a.lengths[lo]);
    } else {
        if (mode != 2) rec = a.order[rec];
        t.request = a.request[rec];
        t.split = a.split[rec];
        t.start = a.begin[rec];
        t.end = a.end[rec];
    }
    return t;
}

// Orders LDS traffic between lanes of ONE wave without a workgroup barrier.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// This worker's first task as resolved by the plan (sgd_plan_buffers.dispatch0), when
// the launch may use it: modes R1, D1, D4, and a table built for this mode and worker
// count (entry 0's tag).  The host guarantees dispatch0 has an entry per worker.
struct FirstTask {
    bool valid;
    int32_t task, count;
    TaskInfo info;
};

__device__ __forceinline__ FirstTask first_task(const sgd_decode_args &a, int32_t mode) {
    FirstTask f;
    f.valid = false;
    if (!a.dispatch0) return f;
    const int32_t *e = a.dispatch0 + 8 * blockIdx.x;  // loaded with the tag, in one round trip
    const int32_t tag = a.dispatch0[7];
    f.task = e[0];
    f.count = e[1];
    f.info.request = e[2];
    f.info.split = e[3];
    f.info.start = e[4];
    f.info.end = e[5];
    f.info.group = e[6];
    f.valid = (mode == 1 || mode == 3 || mode == 4) && tag == mode + 8 * a.workers;
    return f;
}

// Runs `run(task, mode, pre)` for every task of this worker, where pre is the task's
// resolved TaskInfo when the plan supplied it (the first task; null otherwise).  All
// threads of the workgroup execute it uniformly; `sh_cursor` is one int of LDS.  With
// a first-task table in D1/D4, worker w runs pack w first and its claims are
// workers + (counter): every pack still runs exactly once.
template <class Run>
__device__ void for_each_task(const sgd_decode_args &a, int32_t *sh_cursor, Run &&run) {
    const int32_t worker = blockIdx.x;
    const int32_t mode = *a.mode;
    const FirstTask first = first_task(a, mode);
    const int32_t total = *a.record_count * a.kv_heads;
    const bool dynamic = mode >= 3;
    const int32_t claim_base = (dynamic && first.valid) ? a.workers : 0;
    auto claim = [&]() {
        if (threadIdx.x == 0)
            *sh_cursor = claim_base + __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const int32_t c = *sh_cursor;
        __syncthreads();  // every thread has read the claim before the next one overwrites it
        return c;
    };
    int32_t cursor, limit;
    if (dynamic) {
        limit = *a.num_packs;
        if (first.valid) {
            if (first.task >= 0) {
                for (int32_t i = 0; i < first.count; ++i) run(first.task + i, mode, i == 0 ? &first.info : nullptr);
            }
        }
        cursor = claim();
    } else if (mode == 2) {
        cursor = a.static_head[worker];
        limit = total;
    } else {
        cursor = worker;
        limit = total;
        if (first.valid && cursor < limit) {  // R1: task `worker`, already resolved
            run(cursor, mode, &first.info);
            cursor += a.workers;
        }
    }
    while (cursor >= 0 && cursor < limit) {
        int32_t first_t = cursor, count = 1;
        if (dynamic) {
            first_t = a.pack_first[cursor];
            count = a.pack_count[cursor];
        }
        for (int32_t i = 0; i < count; ++i) run(first_t + i, mode, (const TaskInfo *)nullptr);
        if (dynamic) {
            cursor = claim();
        } else if (mode == 2) {
            cursor = a.static_next[cursor];
        } else {
            cursor += a.workers;
        }
    }
    // The last worker to finish puts the claim counter back to zero for the next
    // launch.  Relaxed is enough: a worker reaches this increment only after its
    // final claim returned (the loop exit depends on that value), so every claim
    // has been performed before the last increment is observed.  (A device-scope
    // release here would write back the XCD's whole L2 once per workgroup.)
    if (a.done_counter && threadIdx.x == 0) {
        const int32_t done = __hip_atomic_fetch_add(a.done_counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == a.workers - 1) {
            __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.done_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

}  // namespace sgd
