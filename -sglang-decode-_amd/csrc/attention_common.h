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

// Token position -> (page, row within the page) of a paged layout: shift and mask when
// the page size is a power of two (kPow2), an exact unsigned division otherwise.  Token
// positions are never negative.
template <bool kPow2>
struct PageMap {
    int32_t shift, mask, size;
    __device__ __forceinline__ explicit PageMap(int32_t page_size)
        : shift(__builtin_ctz((unsigned)page_size)), mask(page_size - 1), size(page_size) {}
    __device__ __forceinline__ int32_t page(int32_t tok) const {
        if constexpr (kPow2) return tok >> shift;
        else return (int32_t)((uint32_t)tok / (uint32_t)size);
    }
    __device__ __forceinline__ int32_t row(int32_t tok) const {
        if constexpr (kPow2) return tok & mask;
        else return (int32_t)((uint32_t)tok % (uint32_t)size);
    }
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

// The start of a worker's next task, found by the run hook of for_each_task<true>
// while the current task's last tiles stream, and left in LDS before the workgroup
// barrier that ends the task: the claimed unit (`cursor`, D1/D4), `unit` and its entry
// `e` when the next task opens a new unit (else unit -1), `task` and its record `info`
// (task -1: nothing found).  Unit ids, entries and records do not change within a
// launch, so a reader only matches the id.  Two of them alternate by task parity: the
// hook of a worker's task k fills buffer (k + 1) & 1 before task k's end barrier; it is
// read after that barrier, up to task k + 1's end barrier, and written next by the hook
// of task k + 2, which runs only after task k + 1's end barrier -- so no barrier is
// needed at a task's start.
struct Prefetched {
    int32_t cursor, unit, task;
    Entry e;
    TaskInfo info;
};

// What the run hook of for_each_task<true> is told.  `cur` is the buffer holding what
// was found for this task; the hook fills buffer `next`.  When `claim` is set the hook
// must take the worker's next unit -- one relaxed atomic on `counter` by one thread --
// and store base + (old value) to pf[next].cursor before the task's end barrier.
struct Successor {
    Prefetched *pf;     // the two buffers
    int32_t cur, next;
    bool claim;         // D1/D4, last task of its unit
    int32_t *counter;
    int32_t base;
    int32_t next_task;  // the unit's next task, or -1 when this task is the unit's last
    int32_t next_unit;  // R0/R1/STATIC, last task of its unit: the worker's next unit (-1: none)
    int32_t mode, limit;
    bool table;         // units resolve through the dispatch table
};

__device__ __forceinline__ Entry uniform_entry(const Entry &e) {
    auto f = [](int32_t v) { return __builtin_amdgcn_readfirstlane(v); };
    return Entry{make_int4(f(e.x.x), f(e.x.y), f(e.x.z), f(e.x.w)), make_int4(f(e.y.x), f(e.y.y), f(e.y.z), f(e.y.w))};
}

__device__ __forceinline__ TaskInfo uniform_info(const TaskInfo &t) {
    auto f = [](int32_t v) { return __builtin_amdgcn_readfirstlane(v); };
    return TaskInfo{f(t.request), f(t.split), f(t.start), f(t.end), f(t.group)};
}

__device__ __forceinline__ TaskInfo entry_info(const Entry &e) {
    return TaskInfo{e.x.z, e.x.w, e.y.x, e.y.y, e.y.z};
}

// Makes both prefetch buffers match nothing; all threads call it, before a barrier
// that precedes for_each_task<true>.
__device__ __forceinline__ void clear_prefetched(Prefetched *pf) {
    if (threadIdx.x < 2) {
        pf[threadIdx.x].unit = -1;
        pf[threadIdx.x].task = -1;
    }
}

// The hook's search for the worker's next task (run by one whole wave): the claim
// (D1/D4), the dispatch entry or the record of the next task, and the page/slot indices
// of its first kTokens tokens (0 past its end), all into s.pf[s.next] and idx[s.next].
// `sh_indptr` (LDS, CSR) holds kv_indptr[0 .. iptr_n).
template <bool CSR, int kTokens, bool kPow2>
__device__ __forceinline__ void prefetch_next(const sgd_decode_args &a, const Successor &s, int32_t (*idx)[kTokens],
                                              int lane, const PageMap<kPow2> &pm, const int32_t *sh_indptr,
                                              int32_t iptr_n) {
    Prefetched &out = s.pf[s.next];
    int32_t nt = s.next_task, nu = -1;
    TaskInfo ni{};
    Entry ne{};
    bool opened = false;
    if (nt >= 0) {
        ni = decode_task(a, nt, s.mode);
    } else {
        nu = s.next_unit;
        if (s.claim) {
            int32_t c = 0;
            if (lane == 0) c = __hip_atomic_fetch_add(s.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            nu = s.base + __builtin_amdgcn_readlane(c, 0);
            if (lane == 0) out.cursor = nu;
        }
        if (s.table && nu >= 0 && nu < s.limit && nu < a.dispatch_units) {
            ne = load_entry(a.dispatch, nu);
            if (ne.y.w == table_kind(s.mode)) {
                opened = true;
                nt = ne.x.x;
                ni = entry_info(ne);
            }
        }
    }
    nt = __builtin_amdgcn_readfirstlane(nt);
    ni = uniform_info(ni);
    if (nt >= 0) {
        int32_t ind0 = 0;
        if constexpr (CSR)
            ind0 = __builtin_amdgcn_readfirstlane(ni.request < iptr_n ? sh_indptr[ni.request] : a.indptr[ni.request]);
#pragma unroll
        for (int j = lane; j < kTokens; j += 64) {
            const int32_t tok = ni.start + j;
            int32_t v = 0;
            if (tok < ni.end) {
                if constexpr (CSR) v = a.pages[ind0 + tok];
                else v = a.pages[(int64_t)ni.request * a.pt_stride[0] + (int64_t)pm.page(tok) * a.pt_stride[1]];
            }
            idx[s.next][j] = v;
        }
    }
    if (lane == 0) {
        out.unit = opened ? nu : -1;
        out.e = ne;
        out.task = nt;
        out.info = ni;
    }
}

// Runs `run(task, info)` (PRECLAIM: `run(task, info, successor)`) for every task of
// this worker, info being the task's record (from the dispatch table for a unit's first
// task, else decode_task).  All threads of the workgroup execute it uniformly;
// `sh_cursor` is one int of LDS.  In D1/D4 worker w runs pack w first and its claims
// return workers + (counter): every pack still runs exactly once.  Without PRECLAIM the
// next unit is taken when the current one is done (a claim made while a task is still
// streaming most of its tiles holds work back from workers that free up first, and
// measured slower).  With it, the hook claims during the task's last tile rounds and
// leaves the next task's entry and record in `pf` (two LDS buffers, cleared by
// clear_prefetched), used instead of the table and record loads.
template <bool PRECLAIM = false, class Run>
__device__ void for_each_task(const sgd_decode_args &a, int32_t *sh_cursor, Run &&run, Prefetched *pf = nullptr) {
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

    int32_t k = 0;  // tasks run so far; pf[k & 1] holds what was found for the next one
    int32_t unit = mode == 2 ? __builtin_amdgcn_readfirstlane(a.static_head[worker]) : worker;
    while (unit >= 0 && unit < limit) {
        const bool loaded = table && unit < a.dispatch_units;
        Entry e{};
        if (loaded) {
            if (PRECLAIM && __builtin_amdgcn_readfirstlane(pf[k & 1].unit) == unit) e = uniform_entry(pf[k & 1].e);
            else e = load_entry(a.dispatch, unit);
        }
        const Unit u = unit_of(a, unit, mode, loaded, e);
        const int32_t after = dynamic ? -1 : mode == 2 ? __builtin_amdgcn_readfirstlane(a.static_next[unit])
                                                       : unit + a.workers;
        for (int32_t i = 0; i < u.count; ++i, ++k) {
            const int32_t task = u.first + i;
            TaskInfo ti;
            if (i == 0 && u.resolved) ti = u.info;
            else if (PRECLAIM && __builtin_amdgcn_readfirstlane(pf[k & 1].task) == task) ti = pf[k & 1].info;
            else ti = decode_task(a, task, mode);
            ti = uniform_info(ti);
            if constexpr (PRECLAIM) {
                const bool last = i == u.count - 1;
                run(task, ti,
                    Successor{pf, k & 1, (k + 1) & 1, dynamic && last, a.counter, claim_base, last ? -1 : task + 1,
                              !dynamic && last ? after : -1, mode, limit, table});
            } else {
                run(task, ti);
            }
        }
        if (dynamic && PRECLAIM)  // the hook of the unit's last task stored it before that task's end barrier
            unit = __builtin_amdgcn_readfirstlane(pf[k & 1].cursor);
        else
            unit = dynamic ? claim() : after;
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
