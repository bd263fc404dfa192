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

// ---------------------------------------------------------------- dispatch units
// A worker's stream of work is a sequence of units: a task in modes R0, R1 and STATIC,
// a pack of consecutive tasks (pack_first / pack_count) in D1/D4.  The plan's dispatch
// table (sgd_decode_args.dispatch, written by sgd_build_plan) holds one entry per unit
// with its first task's record already resolved: {first task, tasks, request, split,
// begin, end, kv group, kind}.  kind says what the units are -- kTableTasks (task t,
// record t / Hkv: R1 and STATIC) or kTablePacks -- and an entry is used only when it
// matches the launch's mode, so a unit resolves in one round trip instead of the
// pack -> order -> record walk.
constexpr int32_t kTableTasks = 1, kTablePacks = 2;

__device__ __forceinline__ int32_t table_kind(int32_t mode) {
    return mode == 1 || mode == 2 ? kTableTasks : mode >= 3 ? kTablePacks : 0;
}

struct Entry {
    int4 x, y;  // {first task, tasks, request, split}, {begin, end, group, kind}
};

// Uniform load of unit u's entry through the scalar cache: the table is written by an
// earlier launch and never during this one.
__device__ __forceinline__ Entry load_entry(const int32_t *table, int32_t u) {
    typedef int v4i __attribute__((ext_vector_type(4)));
    typedef const __attribute__((address_space(4))) v4i cv4i;
    cv4i *p = (cv4i *)(table + 8 * (int64_t)__builtin_amdgcn_readfirstlane(u));
    const v4i x = p[0], y = p[1];
    return Entry{make_int4(x.x, x.y, x.z, x.w), make_int4(y.x, y.y, y.z, y.w)};
}

struct Unit {
    int32_t first, count;
    bool resolved;  // info holds task `first`'s record
    TaskInfo info;
};

__device__ __forceinline__ Unit unit_of(const sgd_decode_args &a, int32_t u, int32_t mode, bool loaded,
                                        const Entry &e) {
    Unit r;
    if (loaded && e.y.w == table_kind(mode)) {
        r.first = e.x.x;
        r.count = e.x.y;
        r.resolved = true;
        r.info.request = e.x.z;
        r.info.split = e.x.w;
        r.info.start = e.y.x;
        r.info.end = e.y.y;
        r.info.group = e.y.z;
    } else {
        r.first = mode >= 3 ? __builtin_amdgcn_readfirstlane(a.pack_first[u]) : u;
        r.count = mode >= 3 ? __builtin_amdgcn_readfirstlane(a.pack_count[u]) : 1;
        r.resolved = false;
    }
    return r;
}

// A claim the run hook makes itself (for_each_task<true>): in D1/D4 the hook of a
// unit's last task takes the next unit while its last tiles stream -- one relaxed
// atomic on `counter` by one thread -- and stores base + (old value) to `slot` (the
// worker's LDS cursor) before the workgroup barrier that ends its task.  slot is null
// for the other tasks and in the other modes.
struct Preclaim {
    int32_t *slot;
    int32_t *counter;
    int32_t base;
};

// Runs `run(task, info)` (PRECLAIM: `run(task, info, preclaim)`) for every task of this
// worker, info being the task's record (from the dispatch table for a unit's first
// task, else decode_task).  All threads of the workgroup execute it uniformly;
// `sh_cursor` is one int of LDS.  In D1/D4 worker w runs pack w first and its claims
// return workers + (counter): every pack still runs exactly once.  Without PRECLAIM the
// next unit is taken when the current one is done (a claim made while a task is still
// streaming most of its tiles holds work back from workers that free up first, and
// measured slower); with it, the hook claims during its last tile rounds, so the claim
// round trip overlaps them and the unit waits one round at most.
template <bool PRECLAIM = false, class Run>
__device__ void for_each_task(const sgd_decode_args &a, int32_t *sh_cursor, Run &&run) {
    const int32_t worker = blockIdx.x;
    const int32_t mode = __builtin_amdgcn_readfirstlane(*a.mode);
    const int32_t total = __builtin_amdgcn_readfirstlane(*a.record_count) * a.kv_heads;
    const bool dynamic = mode >= 3;
    const int32_t limit = dynamic ? __builtin_amdgcn_readfirstlane(*a.num_packs) : total;
    const bool table = a.dispatch != nullptr && mode != 0;
    const int32_t claim_base = dynamic ? a.workers : 0;

    auto claim = [&]() {  // (LDS-only barriers: the task's output stores stay in flight)
        if (threadIdx.x == 0)
            *sh_cursor = claim_base + __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds_barrier();
        const int32_t c = __builtin_amdgcn_readfirstlane(*sh_cursor);
        lds_barrier();  // every thread has read the claim before the next one overwrites it
        return c;
    };

    int32_t unit = mode == 2 ? __builtin_amdgcn_readfirstlane(a.static_head[worker]) : worker;
    while (unit >= 0 && unit < limit) {
        const bool loaded = table && unit < a.dispatch_units;
        Entry e{};
        if (loaded) e = load_entry(a.dispatch, unit);
        const Unit u = unit_of(a, unit, mode, loaded, e);
        for (int32_t i = 0; i < u.count; ++i) {
            TaskInfo ti = (i == 0 && u.resolved) ? u.info : decode_task(a, u.first + i, mode);
            ti.request = __builtin_amdgcn_readfirstlane(ti.request);
            ti.split = __builtin_amdgcn_readfirstlane(ti.split);
            ti.start = __builtin_amdgcn_readfirstlane(ti.start);
            ti.end = __builtin_amdgcn_readfirstlane(ti.end);
            ti.group = __builtin_amdgcn_readfirstlane(ti.group);
            if constexpr (PRECLAIM)
                run(u.first + i, ti, Preclaim{dynamic && i == u.count - 1 ? sh_cursor : nullptr, a.counter, claim_base});
            else
                run(u.first + i, ti);
        }
        if (dynamic && PRECLAIM)  // the hook stored it before its task's last barrier; the next
            unit = __builtin_amdgcn_readfirstlane(*sh_cursor);  // store follows the next task's first
        else
            unit = dynamic ? claim() : mode == 2 ? __builtin_amdgcn_readfirstlane(a.static_next[unit]) : unit + a.workers;
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
