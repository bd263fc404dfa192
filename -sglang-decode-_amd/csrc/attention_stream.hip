// Persistent paged GQA decode attention, streaming form: the same per-tile math
// as attention_valu.hip (valu_ops.h; group <= 4, head_dim 128), scheduled so that
// a CU never waits at a task boundary.
//
// Worker = one workgroup per CU: 15 compute waves and one scheduler wave.
//
// Scheduler wave.  Produces the worker's tasks in the order of the plan's mode
// (kernels/attention.py:99-130: claim/pack for D1/D4, the linked list for
// STATIC, stride by the worker count for R0/R1) and resolves each to its record
// (:23-47: order -> SoA record, or the R0 upper-bound search of the offsets), the
// CSR row start and the group's q rows.  Round-robin tasks are resolved 64 at a
// time, one per lane.  A resolved task is published into a ring of kRing LDS
// slots together with its first global tile number: the worker's tiles form one
// sequence across its tasks.  Dynamic claims are throttled so that about
// kQueueTiles published tiles stay unreserved: claiming further ahead would undo
// the load balance the claims exist for.
//
// Compute waves.  A wave reserves the worker's next global tile from an LDS
// counter, whatever task it belongs to: a faster wave takes more tiles, short
// tasks leave no wave idle, and no barrier separates tasks.  Per tile: stage the
// K/V rows already in registers into the wave's LDS tile, issue the K/V loads of
// the wave's next tile, reserve the tile after it and load its indices (when
// their tasks are published), then QK^T / online softmax / P.V.  When a wave's next tile lies past its current task, it merges its (m,
// den, acc) into the task's slot under an LDS lock; the wave whose merge
// completes the task's tile count writes the normalized partial and the
// natural-log LSE to slot (request, head, split) (kernels/attention.py:81-84) and
// frees the ring slot.
//
// Progress.  A compute wave merges its share of a task before it can block on a
// later, unpublished task; the scheduler reuses a slot only once its task is
// finalized and every compute wave has moved past it (pos[]), so it never waits
// on a wave that waits on it.  No workgroup waits on another.
#include "valu_ops.h"

namespace sgd {
namespace {

using namespace valu;

constexpr int kComputeWaves = 15;
constexpr int kThreads = 64 * (kComputeWaves + 1);
constexpr int kRing = 10;
constexpr int kQueueTiles = 16;
constexpr int32_t kNotYet = -2;  // the tile lies past every published task
constexpr int32_t kNone = -1;    // the task stream ended before the tile
constexpr int32_t kFar = 0x7fffffff;

struct StreamSlot {
    uint4 q[kHeads][kD / 8];  // the group's q rows (heads >= G are zero)
    float acc[kHeads][kD];    // merged, unnormalized P.V of the waves merged so far
    float m[kHeads], den[kHeads];
    int32_t request, split, start, end;
    int32_t group, ind0, base, ntiles;
    int32_t merged, lock, busy, pad;
};

struct StreamShared {
    WaveTile w[kComputeWaves];
    StreamSlot slot[kRing];
    int32_t pos[16];    // per compute wave: the lowest task whose slot it may still read
    int32_t next_tile;  // the worker's next unreserved global tile
    int32_t pub;        // tasks published
    int32_t fin;      // 1 once no task follows the published ones
};

// Flags between the waves of the workgroup live in LDS and order LDS accesses
// only: the fences name the local address space, so a release never waits for
// the wave's global loads (the KV prefetch) or stores to complete.
__device__ __forceinline__ int32_t lds_acquire(int32_t *p) {
    const int32_t v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    return uni(v);
}

// Minimum over the compute waves of their pos[] words, read one word per lane.
__device__ __forceinline__ int32_t lds_acquire_min(int32_t *words, int lane) {
    int32_t v = kFar;
    if (lane < kComputeWaves) v = __hip_atomic_load(&words[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
    return uni(v);
}

__device__ __forceinline__ void lds_release(int32_t *p, int32_t v, int lane) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if (lane == 0) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Task holding global tile x, scanning from task k (k only grows).
__device__ __forceinline__ int32_t find_task(StreamShared &sh, int32_t x, int32_t &k) {
    const int32_t fin = lds_acquire(&sh.fin);
    const int32_t pub = lds_acquire(&sh.pub);
    while (k < pub) {
        const StreamSlot &s = sh.slot[k % kRing];
        if (x < uni(s.base) + uni(s.ntiles)) return k;
        ++k;
    }
    return fin ? kNone : kNotYet;
}

struct Layout {
    int64_t kh, vh;  // byte strides of a kv head
    int64_t kp, kt, vp, vt;
    int32_t page_shift, page_mask;
};

__device__ __forceinline__ TileSrc slot_src(const StreamSlot &s, const sgd_decode_args &a, const Layout &L) {
    TileSrc t;
    t.request = uni(s.request);
    t.start = uni(s.start);
    t.end = uni(s.end);
    t.ind0 = uni(s.ind0);
    const int32_t group = uni(s.group);
    t.kbase = static_cast<const char *>(a.k) + group * L.kh;
    t.vbase = static_cast<const char *>(a.v) + group * L.vh;
    t.kp = L.kp;
    t.kt = L.kt;
    t.vp = L.vp;
    t.vt = L.vt;
    return t;
}

// Merge this wave's state for the task in slot s (cnt tiles); the wave that
// completes the task writes its partial rows and LSE and frees the slot.
__device__ void merge_into_slot(StreamSlot &s, const sgd_decode_args &a, int lane, int32_t G, float m_l,
                                float den_l, float (&acc)[kHeads][4], int32_t cnt) {
    float mh[kHeads], dh[kHeads];
    wave_state(m_l, den_l, acc, mh, dh);
    for (;;) {
        int32_t got = 0;
        if (lane == 0) {
            int32_t expect = 0;
            got = __hip_atomic_compare_exchange_strong(&s.lock, &expect, 1, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        if (uni(got)) break;
        __builtin_amdgcn_s_sleep(1);
    }
    const int32_t merged = uni(s.merged);
    const bool last = merged + cnt == uni(s.ntiles);
    int pd = lane & 31;  // P.V roles: dims 4*pd .. 4*pd+3 (laundered: rebuilt here, not held live)
    asm volatile("" : "+v"(pd));
    if (merged > 0) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
            const float mo = s.m[h], dn = s.den[h];
            const float mx = fmaxf(mo, mh[h]);
            const float so = __builtin_amdgcn_exp2f(mo - mx), sm = __builtin_amdgcn_exp2f(mh[h] - mx);
            mh[h] = mx;
            dh[h] = dn * so + dh[h] * sm;
            const float4 o = *reinterpret_cast<const float4 *>(&s.acc[h][4 * pd]);
            acc[h][0] = o.x * so + acc[h][0] * sm;
            acc[h][1] = o.y * so + acc[h][1] * sm;
            acc[h][2] = o.z * so + acc[h][2] * sm;
            acc[h][3] = o.w * so + acc[h][3] * sm;
        }
    }
    if (!last) {
        if (lane < 32) {
#pragma unroll
            for (int h = 0; h < kHeads; ++h)
                *reinterpret_cast<float4 *>(&s.acc[h][4 * pd]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        }
        if (lane == 0) {
#pragma unroll
            for (int h = 0; h < kHeads; ++h) {
                s.m[h] = mh[h];
                s.den[h] = dh[h];
            }
            s.merged = merged + cnt;
        }
        lds_release(&s.lock, 0, lane);
        return;
    }
    lds_release(&s.lock, 0, lane);
    const int32_t request = uni(s.request), split = uni(s.split), group = uni(s.group);
    const int64_t row0 = ((int64_t)request * a.query_heads + group * G) * a.max_splits + split;
    if (lane < 32) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
            if (h < G) {
                const float inv = __builtin_amdgcn_rcpf(dh[h]);
                *reinterpret_cast<float4 *>(&a.partial[(row0 + (int64_t)h * a.max_splits) * kD + 4 * pd]) =
                    make_float4(acc[h][0] * inv, acc[h][1] * inv, acc[h][2] * inv, acc[h][3] * inv);
            }
    }
    int hl = lane;  // lane h < G writes head h's LSE
    asm volatile("" : "+v"(hl));
    float lv = 0.f;
#pragma unroll
    for (int h = 0; h < kHeads; ++h)
        if (hl == h) lv = (mh[h] + __log2f(dh[h])) * kLn2;
    if (hl < G) a.lse[row0 + (int64_t)hl * a.max_splits] = lv;
    lds_release(&s.busy, 0, lane);
}

// Reserves the worker's next unclaimed global tile.
__device__ __forceinline__ int32_t grab_tile(StreamShared &sh, int lane) {
    int32_t g = 0;
    if (lane == 0) g = __hip_atomic_fetch_add(&sh.next_tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return uni(g);
}

template <int DT, bool CSR>
__device__ void compute_wave(StreamShared &sh, const sgd_decode_args &a, int wave, int lane) {
    WaveTile &wt = sh.w[wave];
    const int32_t G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    Layout L;
    L.kh = a.k_stride[2] * 2;
    L.vh = a.v_stride[2] * 2;
    L.kp = a.k_stride[0] * 2;
    L.kt = a.k_stride[1] * 2;
    L.vp = a.v_stride[0] * 2;
    L.vt = a.v_stride[1] * 2;
    L.page_shift = __builtin_ctz((unsigned)a.page_size);  // page_size is a power of two here
    L.page_mask = a.page_size - 1;

    // Tiles are reserved from the worker's counter in order, so a faster wave takes
    // more of them; a wave holds the tile being computed (g), the tile whose K/V are
    // in flight (gn) and, once gn is issued, the tile whose indices are prefetched.
    int32_t g = grab_tile(sh, lane), kc = 0;
    for (;;) {
        const int32_t f = find_task(sh, g, kc);
        if (f == kNone) {
            lds_release(&sh.pos[wave], kFar, lane);
            return;
        }
        if (f >= 0) break;
        lds_release(&sh.pos[wave], kc, lane);
        __builtin_amdgcn_s_sleep(2);
    }
    lds_release(&sh.pos[wave], kc, lane);

    uint4 kr[kRowsLoads], vr[kRowsLoads];
    int32_t idx_next = 0;
    bool have_idx = false;  // idx_next holds the indices of tile gn

    // Issues the K/V loads of tile x in task kx (indices prefetched when have_idx).
    auto issue = [&](int32_t x, int32_t kx, bool prefetched) {
        const StreamSlot &s = sh.slot[kx % kRing];
        const TileSrc src = slot_src(s, a, L);
        const int32_t t = x - uni(s.base);
        const int32_t idx =
            prefetched ? idx_next : tile_index<CSR>(a, src, src.start + t * kTile, lane, L.page_shift);
        tile_issue<CSR>(src, t, idx, L.page_mask, lane, kr, vr);
    };
    // Loads the indices of tile x if its task is published (searching from task k).
    auto prefetch_index = [&](int32_t x, int32_t k) {
        const int32_t f = find_task(sh, x, k);
        have_idx = f >= 0;
        if (have_idx) {
            const StreamSlot &s = sh.slot[f % kRing];
            const TileSrc src = slot_src(s, a, L);
            idx_next = tile_index<CSR>(a, src, src.start + (x - uni(s.base)) * kTile, lane, L.page_shift);
        }
    };

    issue(g, kc, false);
    int32_t gn = grab_tile(sh, lane);
    prefetch_index(gn, kc);

    float m_l = -INFINITY, den_l = 0.f;
    float acc[kHeads][4];
#pragma unroll
    for (int h = 0; h < kHeads; ++h)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;
    int32_t cnt = 0;

    // Reserves the tile after the one just issued (in task kx) and prefetches its indices.
    auto reserve_after = [&](int32_t kx) -> int32_t {
        const int32_t x = grab_tile(sh, lane);
        prefetch_index(x, kx);
        return x;
    };

    for (;;) {
        int lane_v = lane;
        asm volatile("" : "+v"(lane_v));
        StreamSlot &sc = sh.slot[kc % kRing];
        const int32_t nvalid = min(kTile, uni(sc.end) - (uni(sc.start) + (g - uni(sc.base)) * kTile));
        tile_stage(wt, kr, vr, lane_v, nvalid);
        int32_t kscan = kc;
        int32_t kn = find_task(sh, gn, kscan);
        int32_t gnn = -1;
        const bool issued = kn >= 0;
        if (issued) {
            issue(gn, kn, have_idx);
            gnn = reserve_after(kn);
        }
        wave_sync();
        tile_compute<DT>(wt, sc.q, nvalid, scale2, Roles(lane_v), m_l, den_l, acc);
        ++cnt;
        if (kn != kc) {  // this wave's share of task kc is complete
            merge_into_slot(sc, a, lane, G, m_l, den_l, acc, cnt);
            m_l = -INFINITY;
            den_l = 0.f;
#pragma unroll
            for (int h = 0; h < kHeads; ++h)
#pragma unroll
                for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;
            cnt = 0;
        }
        if (!issued) {  // gn lies past the published tasks: wait, holding no unmerged state
            while (kn == kNotYet) {
                lds_release(&sh.pos[wave], kscan, lane);
                __builtin_amdgcn_s_sleep(2);
                kn = find_task(sh, gn, kscan);
            }
            if (kn == kNone) break;
            issue(gn, kn, false);
            gnn = reserve_after(kn);
        }
        lds_release(&sh.pos[wave], kn, lane);
        kc = kn;
        g = gn;
        gn = gnn;
    }
    lds_release(&sh.pos[wave], kFar, lane);
}

// This lane's 16 bytes of the group's q rows for (request, group): head lane / 16,
// dims 8 * (lane % 16) .. +7; heads >= G are zero.
__device__ __forceinline__ uint4 load_q(const sgd_decode_args &a, int32_t request, int32_t group, int32_t G,
                                        int lane) {
    const int h = lane >> 4, c = lane & 15;
    uint4 w = make_uint4(0, 0, 0, 0);
    if (h < G) {
        const int64_t qd = a.q_stride[2];
        const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (int64_t)request * a.q_stride[0] +
                             (int64_t)(group * G + h) * a.q_stride[1] + (int64_t)(c * 8) * qd;
        if (qd == 1 && (reinterpret_cast<uintptr_t>(qp) & 15) == 0) {
            w = *reinterpret_cast<const uint4 *>(qp);
        } else {
            uint32_t w4[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e) w4[e >> 1] |= (uint32_t)qp[e * qd] << (16 * (e & 1));
            w = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    }
    return w;
}

template <bool CSR>
__device__ void schedule(StreamShared &sh, const sgd_decode_args &a, int lane) {
    const int32_t W = a.workers, hkv = a.kv_heads, G = a.query_heads / a.kv_heads;
    const int32_t mode = uni(*a.mode);
    const int64_t total = (int64_t)uni(*a.record_count) * hkv;
    const bool dynamic = mode >= 3;
    const int32_t num_packs = dynamic ? uni(*a.num_packs) : 0;
    const int32_t active = mode == 0 ? uni(*a.active) : 0;
    // With the plan's dispatch table, units resolve to their records in one round trip
    // (R1 and STATIC per lane, D1/D4 for a pack's first task).  In D1/D4 pack `worker`
    // is taken without a claim; claims then return W + counter (every pack runs once).
    const bool table = a.dispatch != nullptr && mode != 0;
    const int32_t kind = table_kind(mode);
    const int32_t claim_base = dynamic ? W : 0;
    bool first_pack = dynamic;
    int32_t seq = 0, base = 0;
    int64_t rr = 0;                          // R0/R1: tasks enumerated so far
    int32_t chain = -1;                      // STATIC: last task taken from the list
    int32_t pack_next = 0, pack_left = 0;    // D1/D4: rest of the claimed pack
    for (;;) {
        // 1. enumerate up to 64 tasks, one per lane
        int32_t t = -1, nb = 0;
        bool pre0 = false;  // lane 0's task was resolved by the pack's table entry
        TaskInfo p0{};
        if (mode <= 1) {
            const int64_t tt = (int64_t)blockIdx.x + (rr + lane) * W;
            t = tt < total ? (int32_t)tt : -1;
            const int64_t left = total > (int64_t)blockIdx.x + rr * W
                                     ? (total - (int64_t)blockIdx.x - rr * W + W - 1) / W : 0;
            nb = (int32_t)min<int64_t>(left, 64);
            rr += 64;
        } else if (mode == 2) {
            const int32_t nx = uni(chain < 0 ? a.static_head[blockIdx.x] : a.static_next[chain]);
            if (nx >= 0 && nx < total) {
                chain = nx;
                t = nx;
                nb = 1;
            }
        } else {
            if (pack_left == 0) {
                int32_t c = blockIdx.x;
                if (first_pack) {
                    first_pack = false;
                } else {
                    // claim only when fewer than kQueueTiles published tiles are unreserved
                    while (base - lds_acquire(&sh.next_tile) >= kQueueTiles) __builtin_amdgcn_s_sleep(2);
                    c = 0;
                    if (lane == 0) c = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    c = claim_base + uni(c);
                }
                if (c >= 0 && c < num_packs) {
                    const bool use = table && c < a.dispatch_units;
                    Entry e{};
                    if (use) e = load_entry(a.dispatch, c);
                    if (use && e.y.w == kind) {
                        pack_next = e.x.x;
                        pack_left = max(e.x.y, 0);
                        pre0 = true;
                        p0 = TaskInfo{e.x.z, e.x.w, e.y.x, e.y.y, e.y.z};
                    } else {
                        pack_next = uni(a.pack_first[c]);
                        pack_left = max(uni(a.pack_count[c]), 0);
                    }
                }
            }
            nb = min(pack_left, 64);
            t = lane < nb ? pack_next + lane : -1;
            pack_next += nb;
            pack_left -= nb;
        }
        if (nb <= 0) break;

        // 2. resolve each lane's task (kernels/attention.py:23-47)
        int32_t request = 0, split = 0, start = 0, end = 0, group = 0, ind0 = 0;
        if (pre0 && lane == 0) {
            request = p0.request;
            split = p0.split;
            start = p0.start;
            end = p0.end;
            group = p0.group;
            if constexpr (CSR) ind0 = a.indptr[request];
        } else if (lane < nb && t >= 0) {
            const int4 *ep = reinterpret_cast<const int4 *>(a.dispatch + 8 * (int64_t)t);
            int4 ex = make_int4(0, 0, 0, 0), ey = make_int4(0, 0, 0, 0);
            const bool per_task = table && mode <= 2 && t < a.dispatch_units;
            if (per_task) {
                ex = ep[0];
                ey = ep[1];
            }
            if (per_task && ey.w == kind) {
                request = ex.z;
                split = ex.w;
                start = ey.x;
                end = ey.y;
                group = ey.z;
            } else {
                group = t % hkv;
                int32_t rec = t / hkv;
                if (mode == 0) {
                    int32_t lo = 0, hi = active;
                    while (lo < hi) {
                        const int32_t mid = (lo + hi) >> 1;
                        if (rec >= a.offsets[mid + 1]) lo = mid + 1;
                        else hi = mid;
                    }
                    request = lo;
                    split = rec - a.offsets[lo];
                    const int32_t c = a.chunk[lo];
                    start = split * c;
                    end = min(start + c, a.lengths[lo]);
                } else {
                    if (mode != 2) rec = a.order[rec];
                    request = a.request[rec];
                    split = a.split[rec];
                    start = a.begin[rec];
                    end = a.end[rec];
                }
            }
            if constexpr (CSR) ind0 = a.indptr[request];
        }

        // 3. publish in order; each task's q rows are loaded before its slot wait
        for (int32_t i = 0; i < nb; ++i) {
            const int32_t st = __builtin_amdgcn_readlane(start, i);
            const int32_t en = __builtin_amdgcn_readlane(end, i);
            const int32_t ntiles = en > st ? (en - st + kTile - 1) / kTile : 0;
            if (ntiles == 0) continue;  // emit_records never makes an empty record
            const int32_t rq = __builtin_amdgcn_readlane(request, i);
            const int32_t gp = __builtin_amdgcn_readlane(group, i);
            const uint4 qrow = load_q(a, rq, gp, G, lane);
            const int32_t sp = __builtin_amdgcn_readlane(split, i);
            StreamSlot &s = sh.slot[seq % kRing];
            if (seq >= kRing) {
                for (;;) {
                    const int32_t low = lds_acquire_min(sh.pos, lane);
                    if (lds_acquire(&s.busy) == 0 && low > seq - kRing) break;
                    __builtin_amdgcn_s_sleep(2);
                }
            }
            s.q[lane >> 4][lane & 15] = qrow;
            const int32_t i0 = __builtin_amdgcn_readlane(ind0, i);
            if (lane == 0) {
                s.request = rq;
                s.split = sp;
                s.start = st;
                s.end = en;
                s.group = gp;
                s.ind0 = i0;
                s.base = base;
                s.ntiles = ntiles;
                s.merged = 0;
                s.lock = 0;
                s.busy = 1;
            }
            base += ntiles;
            ++seq;
            lds_release(&sh.pub, seq, lane);
        }
    }
    lds_release(&sh.fin, 1, lane);

    // The last worker to finish puts the claim counter back to zero for the next
    // launch (see for_each_task: relaxed is enough, the loop exit depends on the
    // final claim's value).
    if (a.done_counter && lane == 0) {
        const int32_t done = __hip_atomic_fetch_add(a.done_counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == a.workers - 1) {
            __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.done_counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int DT, bool CSR>
__global__ __launch_bounds__(kThreads) void k_attention_stream(sgd_decode_args a) {
    extern __shared__ __align__(16) char dyn_smem[];
    StreamShared &sh = *reinterpret_cast<StreamShared *>(dyn_smem);
    if (threadIdx.x < 16) sh.pos[threadIdx.x] = 0;
    if (threadIdx.x < kRing) sh.slot[threadIdx.x].busy = 0;
    if (threadIdx.x == 0) {
        sh.next_tile = 0;
        sh.pub = 0;
        sh.fin = 0;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
    if (wave == kComputeWaves) schedule<CSR>(sh, a, lane);
    else compute_wave<DT, CSR>(sh, a, wave, lane);
}

template <int DT, bool CSR>
int launch_stream_t(const sgd_decode_args &a, hipStream_t stream) {
    static bool attr = false;
    constexpr int bytes = (int)sizeof(StreamShared);
    if (!attr) {
        if (hipFuncSetAttribute((const void *)k_attention_stream<DT, CSR>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                bytes) != hipSuccess)
            return einval("stream attention: cannot reserve %d B of LDS", bytes);
        attr = true;
    }
    hipLaunchKernelGGL((k_attention_stream<DT, CSR>), dim3(a.workers), dim3(kThreads), bytes, stream, a);
    return launch_status("persistent_decode(stream)");
}

}  // namespace

bool valu_supported(const sgd_decode_args &a);

// The stream kernel writes partial rows with 16-byte stores.
bool stream_supported(const sgd_decode_args &a) {
    return valu_supported(a) && (reinterpret_cast<uintptr_t>(a.partial) & 15) == 0;
}

int launch_attention_stream(const sgd_decode_args &a, hipStream_t stream) {
    if (a.dtype == SGD_BF16)
        return a.csr ? launch_stream_t<SGD_BF16, true>(a, stream) : launch_stream_t<SGD_BF16, false>(a, stream);
    return a.csr ? launch_stream_t<SGD_FP16, true>(a, stream) : launch_stream_t<SGD_FP16, false>(a, stream);
}

}  // namespace sgd
