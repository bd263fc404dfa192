// Persistent paged GQA decode attention, span schedule: the per-tile VALU math of
// attention_valu.hip (valu_ops.h; group <= 4, head_dim 128) with no task boundary
// in any wave's load stream.
//
// The step's work is one sequence of 16-token tiles: requests in order, within a
// request its splits (kernels/attention.py:81 slots), within a split its kv heads,
// within a (split, head) task its tiles.  Request r holds ceil(L_r / 16) tiles per
// kv head, so the plan's tile_prefix locates every tile without the record table
// (sgd_build_plan, stage_spans).  Worker w (a workgroup) takes tiles
// [S_w, S_{w+1}), S_w = floor(w * T / workers); its waves split that range
// evenly and each streams its own contiguous span: two tiles' K/V rows and the
// indices of a third are in flight while a tile is computed, whatever task they
// belong to.  Every wave moves the same number of bytes, so the waves finish
// together; no claim, barrier or descriptor walk sits between tiles.
//
// A wave's piece of a task is the tiles of that task in its span.  A piece that is
// the whole task is normalized and written to slot (request, head, split) at once.
// A cut piece (the span starts or ends inside the task) is left in LDS as soon as its
// wave finishes it -- no wave waits for another -- and the wave whose piece completes
// the task's count within the workgroup combines the task's pieces in wave order
// (online-softmax combination, exp2 domain; the fixed order keeps repeated launches
// bitwise equal) and finishes the task: a task inside the workgroup's range is
// written to its slot; one cut by the range's start or end is written, unnormalized,
// to the workgroup's edge record 0 (task holding its first tile) or 1 (its last
// tile), and the merge kernel (sgd_merge_splits_span) completes it.  The mode only
// shapes the plan; the span schedule runs every task of any mode exactly once.
#include "span_layout.h"
#include "valu_ops.h"

namespace sgd {
namespace {

using namespace valu;

// One softmax state of (part of) a task: unnormalized P.V, running max (log2 domain)
// and denominator per query head.  The edge scratch holds these, [workers][2].
struct Piece {
    float acc[kHeads][kD];
    float m[kHeads], den[kHeads];
};
constexpr int kPieceFloats = span::kPieceFloats;
static_assert(sizeof(Piece) == kPieceFloats * sizeof(float) && kHeads == span::kHeads && kD == span::kD &&
                  kTile == span::kTile && offsetof(Piece, m) == span::kPieceM * sizeof(float) &&
                  offsetof(Piece, den) == span::kPieceDen * sizeof(float),
              "edge record layout");


template <int NW>
struct SpanShared {
    int32_t prog[NW];  // tiles each wave has computed (progress balance of SIMD partners)
    int32_t pad[(16 - NW % 16) % 16];
    WaveTile w[NW];
    // Pieces of the tasks cut inside the workgroup, counted as they arrive.  count[u]
    // (u < NW) belongs to the cut task that starts in wave u's span, count[NW] to the
    // task cut by the workgroup's start: a wave's span starts at most one task that it
    // does not finish, so no two tasks share a counter (the first wave's span may hold
    // both kinds, hence the extra one).  piece[v][0] holds the piece that ends the task
    // wave v's span starts inside of, piece[v][1] the piece that starts the task its
    // span ends inside of.
    int32_t count[NW + 1];
    int32_t pad2[(4 - (NW + 1) % 4) % 4];
    uint4 q[NW][kHeads][kD / 8];  // each wave's q rows of its current task
    Piece piece[NW][2];
};

// Uniform load through the scalar cache (plan tables written by an earlier launch).
__device__ __forceinline__ int32_t sload(const int32_t *p, int32_t i) {
    typedef const __attribute__((address_space(4))) int32_t cint;
    return *((cint *)(p) + uni(i));
}

// The launch arguments read again from the kernarg segment (the kernel's only
// explicit argument, at offset 0), through the constant address space so every field
// is a scalar load.  The laundered pointer keeps the compiler from holding every field
// in SGPRs across the loop: the fields that only the rare paths need (task and
// request changes, piece writes) are loaded there.
typedef const __attribute__((address_space(4))) sgd_decode_args KArgs;

__device__ __forceinline__ KArgs &fresh(const sgd_decode_args &) {
    KArgs *p = (KArgs *)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *p;
}

// What one tile's loads and its task's bookkeeping need (all uniform).
struct Desc {
    int32_t base;  // CSR: the request's first kv_indices entry; paged: its page-table row offset
    int32_t tok0;  // first token of the tile
    int32_t end;   // end token of the task (0: a tile past the span)
    int32_t goff;  // byte offset of the kv head in a token row
    int32_t qoff;  // element offset of the group's q rows
    int32_t slot;  // (request * Hq + group * G) * smax + split: the task's first partial/lse row
    int32_t tl;    // tiles of the task after this one
};

// A request's place in the tile sequence.
struct Req {
    int32_t r, per_head, c, n, L, ind0;
};

template <bool CSR>
__device__ __forceinline__ Req load_req(const sgd_decode_args &a0, int32_t r) {
    KArgs &a = fresh(a0);
    Req q;
    q.r = r;
    if (r >= a.batch_capacity) {  // past the last row: no tiles
        q.per_head = q.c = q.n = q.L = q.ind0 = 0;
        return q;
    }
    const int32_t p0 = sload(a.tile_prefix, r), p1 = sload(a.tile_prefix, r + 1);
    const int32_t o0 = sload(a.offsets, r), o1 = sload(a.offsets, r + 1);
    q.c = sload(a.chunk, r);
    q.L = sload(a.lengths, r);
    // kv_indptr holds active + 1 entries
    q.ind0 = CSR ? sload(a.indptr, min(r, max(sload(a.active, 0), 0))) : 0;
    q.per_head = p1 - p0;
    q.n = o1 - o0;
    return q;
}

// The tile to describe next (its Desc fields, advanced incrementally) and where it
// sits: head g and split s of request q, nt tiles per task of this split starting
// at token begin; `left` tiles of the span are still to be described.
struct Cursor {
    Desc d;
    int32_t g, s, nt, begin, left;
    Req q;
};

// Split s (head 0) of the cursor's request becomes current.
template <bool CSR>
__device__ __forceinline__ void enter_split(Cursor &c, const sgd_decode_args &a0) {
    KArgs &a = fresh(a0);
    const int32_t c16 = c.q.c / kTile, G = a.query_heads / a.kv_heads;
    c.begin = c.s * c.q.c;
    c.nt = c.s == c.q.n - 1 ? c.q.per_head - (c.q.n - 1) * c16 : c16;
    c.d.base = CSR ? c.q.ind0 : c.q.r * (int32_t)a.pt_stride[0];
    c.d.end = min(c.begin + c.q.c, c.q.L);
    c.d.goff = c.g * (int32_t)(a.k_stride[2] * 2);
    c.d.qoff = c.q.r * (int32_t)a.q_stride[0] + c.g * G * (int32_t)a.q_stride[1];
    c.d.slot = (c.q.r * a.query_heads + c.g * G) * a.max_splits + c.s;
}

template <bool CSR>
__device__ __forceinline__ Desc describe(Cursor &c, Req &next, const sgd_decode_args &a0) {
    if (c.left <= 0) {  // past the span: an empty tile
        Desc d;
        d.base = d.tok0 = d.end = d.goff = d.qoff = d.slot = d.tl = 0;
        return d;
    }
    const Desc d = c.d;
    if (--c.left == 0) return d;
    if (c.d.tl > 0) {  // the next tile of the same task
        c.d.tok0 += kTile;
        --c.d.tl;
        return d;
    }
    KArgs &a = fresh(a0);
    const int32_t G = a.query_heads / a.kv_heads;
    c.d.tok0 = c.begin;
    c.d.tl = c.nt - 1;
    if (++c.g < a.kv_heads) {  // the next kv head of the same split
        c.d.goff += (int32_t)(a.k_stride[2] * 2);
        c.d.qoff += G * (int32_t)a.q_stride[1];
        c.d.slot += G * a.max_splits;
        return d;
    }
    c.g = 0;
    if (++c.s >= c.q.n) {  // the next request with tiles
        c.q = next;
        while (c.q.per_head == 0 && c.q.r < a.batch_capacity) c.q = load_req<CSR>(a0, c.q.r + 1);
        next = load_req<CSR>(a0, c.q.r + 1);
        c.s = 0;
    }
    enter_split<CSR>(c, a0);
    c.d.tok0 = c.begin;
    c.d.tl = c.nt - 1;
    return d;
}

// Lane 16r + i (i < 4) gets the page/slot index of token tok0 + 4i + r.  Tokens past
// the end read the task's last token instead (an empty tile reads entry 0 of the
// table): those rows are real rows, so their K/V loads stay in bounds, and their
// scores are masked.  Every lane loads (lanes i >= 4 repeat lane i % 4's address) and
// the value is used as loaded, so no exec-mask branch surrounds the load -- one would
// blur the wait counts of the loads in flight around it.
template <bool CSR>
__device__ __forceinline__ int32_t span_index(const int32_t *pages, const Desc &d, int lane, int page_shift) {
    const int r = lane >> 4, i = lane & 3;
    const int32_t t = min(d.tok0 + 4 * i + r, max(d.end - 1, 0));
    if constexpr (CSR) return pages[d.base + t];
    else return pages[d.base + (t >> page_shift)];  // span_supported: unit column stride
}

// Issues a tile's K and V rows: 4 x 16-byte loads each, every load covering 4 token
// rows of 256 B (16 lanes per row), the row's page/slot index handed over by DPP
// row_newbcast from span_index's lanes.  Rows past the task's end read the task's
// last token (index and in-page offset of the clamped token), so they are real,
// written rows.  A tile past the span (d.end == 0) reads row 0 of page 0: its index
// was loaded like any other (no branch around the load) but is replaced here, since
// entry 0 of a page table may be padding (-1).
template <bool CSR>
__device__ __forceinline__ void span_issue(const char *kpool, const char *vpool, int32_t pstride, int32_t tstride,
                                           const Desc &d, int32_t idxv, int32_t page_mask, int lane,
                                           uint4 (&kr)[kRowsLoads], uint4 (&vr)[kRowsLoads]) {
    const int r = lane >> 4, c = lane & 15;
    const bool live = d.end > 0;
    const int32_t last = max(d.end - 1, 0);
    const char *kb = kpool + d.goff + c * 16, *vb = vpool + d.goff + c * 16;
#define SGD_SPAN_ROW(I)                                                                              \
    {                                                                                                \
        uint32_t phys = (uint32_t)dpp_i<kRowNewBcast + I>(idxv);                                     \
        phys = live ? phys : 0u;                                                                     \
        uint64_t off = (uint64_t)phys * (uint32_t)pstride;                                           \
        if constexpr (!CSR) off += (uint32_t)((min(d.tok0 + 4 * I + r, last) & page_mask) * tstride); \
        kr[I] = load_stream16(kb + off);                                                             \
        vr[I] = load_stream16(vb + off);                                                             \
    }
    static_assert(kRowsLoads == 4, "one SGD_SPAN_ROW per 4-row load");
    SGD_SPAN_ROW(0) SGD_SPAN_ROW(1) SGD_SPAN_ROW(2) SGD_SPAN_ROW(3)
#undef SGD_SPAN_ROW
}

// Writes a tile's rows to the wave's LDS tile as loaded.  Rows past the task's end
// hold the task's last token (span_index), finite data whose scores tile_compute
// masks to -inf, so their probabilities are exactly zero and add nothing to P.V; no
// register of a load in flight is overwritten on one path and not the other.
__device__ __forceinline__ void stage_rows(WaveTile &wt, const uint4 (&kr)[kRowsLoads], const uint4 (&vr)[kRowsLoads],
                                           int lane) {
#pragma unroll
    for (int i = 0; i < kRowsLoads; ++i) {
        wt.k[4 * i + (lane >> 4)][lane & 15] = kr[i];
        wt.v[4 * i + (lane >> 4)][lane & 15] = vr[i];
    }
}

// This lane's 16 bytes of the group's q rows: head lane / 16, dims 8 * (lane % 16) ..
// +7, at element hoff (per lane, fixed) past the group's first row; heads >= G read
// the group's first row (in bounds) and are never used.
__device__ __forceinline__ uint4 load_q16(const uint16_t *q, int32_t hoff, const Desc &d) {
    return *reinterpret_cast<const uint4 *>(q + d.qoff + hoff);
}

// Normalized partial rows and natural-log LSE of a finished task whose first row is
// `slot` (kernels/attention.py:81-84); head h's row is slot + h * smax.
template <class Args>
__device__ __forceinline__ void write_task(Args &a, int32_t G, int32_t slot,
                                           const float (&acc)[kHeads][4], const float (&mh)[kHeads],
                                           const float (&dh)[kHeads], int lane) {
    int pd = lane & 31;
    asm volatile("" : "+v"(pd));
    if (lane < 32) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
            if (h < G) {
                const float inv = __builtin_amdgcn_rcpf(dh[h]);
                *reinterpret_cast<float4 *>(&a.partial[((int64_t)slot + h * a.max_splits) * kD + 4 * pd]) =
                    make_float4(acc[h][0] * inv, acc[h][1] * inv, acc[h][2] * inv, acc[h][3] * inv);
            }
    }
    float lv = 0.f;
#pragma unroll
    for (int h = 0; h < kHeads; ++h)
        if (lane == h) lv = (mh[h] + __log2f(dh[h])) * kLn2;
    if (lane < G) a.lse[(int64_t)slot + lane * a.max_splits] = lv;
}

// A wave's cut piece of the task [tb, te) (tiles of the sequence, first partial row
// `slot`): left in the wave's piece buffer, then counted.  The wave that completes the
// workgroup's count combines the task's pieces in wave order and finishes the task: its
// normalized partial and LSE when the task lies inside the workgroup's range, else its
// unnormalized state to the workgroup's edge record (0: the task holding the range's
// first tile, 1: the one holding its last) for the merge kernel.  first: the piece
// starts at the task's first tile.
template <int NW>
__device__ void merge_piece(SpanShared<NW> &sh, const sgd_decode_args &a0, int32_t G, int32_t tb, int32_t te,
                            int32_t slot, bool first, const float (&acc)[kHeads][4], const float (&mh)[kHeads],
                            const float (&dh)[kHeads], int lane) {
    const int wave = uni(threadIdx.x >> 6);
    int pd = lane & 31;
    asm volatile("" : "+v"(pd));
    {
        Piece &mine = sh.piece[wave][first ? 1 : 0];
        if (lane < 32) {
#pragma unroll
            for (int h = 0; h < kHeads; ++h)
                *reinterpret_cast<float4 *>(&mine.acc[h][4 * pd]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        }
        if (lane < kHeads) {
            mine.m[lane] = lane == 0 ? mh[0] : lane == 1 ? mh[1] : lane == 2 ? mh[2] : mh[3];
            mine.den[lane] = lane == 0 ? dh[0] : lane == 1 ? dh[1] : lane == 2 ? dh[2] : dh[3];
        }
    }
    KArgs &a = fresh(a0);  // the rare path reloads what it needs instead of keeping it live
    const int32_t U = a.span_units, w = blockIdx.x;
    const int64_t T = (int64_t)a.kv_heads * sload(a.tile_prefix, a.batch_capacity);
    const int32_t Sw = (int32_t)span::worker_start(w, T, U), Ew = (int32_t)span::worker_start(w + 1, T, U);
    const int32_t lo = max(tb, Sw), hi = min(te, Ew);
    const int32_t u0 = span::wave_of(lo, T, U), u1 = span::wave_of(hi - 1, T, U);
    int32_t expected = 0;  // the workgroup's waves whose spans hold part of the task
    for (int32_t u = u0; u <= u1; ++u) expected += span::wave_start(u, T, U) < span::wave_start(u + 1, T, U);
    int32_t *count = &sh.count[tb < Sw ? NW : u0 - w * NW];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");  // the piece before the count
    int32_t before = 0;
    if (lane == 0) before = __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (uni(before) + 1 != expected) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");  // every piece after the count

    // the task's pieces in wave order: the first covering wave's piece starts the task
    // unless the task began before the workgroup's range
    float M[kHeads], D[kHeads], X[kHeads][4];
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
        M[h] = -INFINITY;
        D[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) X[h][e] = 0.f;
    }
    for (int32_t u = u0; u <= u1; ++u) {
        if (span::wave_start(u, T, U) == span::wave_start(u + 1, T, U)) continue;  // an empty span
        const Piece &p = sh.piece[u - w * NW][u == u0 && tb >= Sw ? 1 : 0];
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
            const float mp = uni_f(p.m[h]), dp = uni_f(p.den[h]);
            const float mx = fmaxf(M[h], mp);
            const float so = __builtin_amdgcn_exp2f(M[h] - mx), sp = __builtin_amdgcn_exp2f(mp - mx);
            M[h] = mx;
            D[h] = D[h] * so + dp * sp;
            const float4 o = *reinterpret_cast<const float4 *>(&p.acc[h][4 * pd]);
            X[h][0] = X[h][0] * so + o.x * sp;
            X[h][1] = X[h][1] * so + o.y * sp;
            X[h][2] = X[h][2] * so + o.z * sp;
            X[h][3] = X[h][3] * so + o.w * sp;
        }
    }
    if (tb >= Sw && te <= Ew) {
        write_task(a, G, slot, X, M, D, lane);
        return;
    }
    float *e = a.edge + ((int64_t)w * 2 + (tb < Sw ? 0 : 1)) * kPieceFloats;
    if (lane < 32) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
            *reinterpret_cast<float4 *>(&e[h * kD + 4 * pd]) = make_float4(X[h][0], X[h][1], X[h][2], X[h][3]);
    }
    if (lane < kHeads) {
        e[kHeads * kD + lane] = lane == 0 ? M[0] : lane == 1 ? M[1] : lane == 2 ? M[2] : M[3];
        e[kHeads * kD + kHeads + lane] = lane == 0 ? D[0] : lane == 1 ? D[1] : lane == 2 ? D[2] : D[3];
    }
}

template <int DT, bool CSR, int NW, int DEPTH>
__global__ __launch_bounds__(64 * NW, NW > 4 ? 2 : 1) void k_attention_span(sgd_decode_args a) {
    extern __shared__ __align__(16) char dyn_smem[];
    SpanShared<NW> &sh = *reinterpret_cast<SpanShared<NW> *>(dyn_smem);
    const int lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
    WaveTile &wt = sh.w[wave];
    const char *kpool = static_cast<const char *>(a.k), *vpool = static_cast<const char *>(a.v);
    const int32_t *pages = a.pages;
    const uint16_t *qbase = static_cast<const uint16_t *>(a.q);
    const int32_t pstride = (int32_t)(a.k_stride[0] * 2), tstride = (int32_t)(a.k_stride[1] * 2);
    const int32_t hkv = a.kv_heads, G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    const int page_shift = __builtin_ctz((unsigned)a.page_size);
    const int32_t page_mask = a.page_size - 1;
    // this lane's q element offset within the group's rows (head lane / 16, dims 8 * (lane % 16))
    const int32_t qhoff = ((lane >> 4) < G ? (lane >> 4) : 0) * (int32_t)a.q_stride[1] + (lane & 15) * 8;

    if (lane == 0) {
        sh.count[wave] = 0;
        sh.prog[wave] = 0;
        if (wave == 0) sh.count[NW] = 0;
    }
    lds_barrier();  // every counter is cleared before any wave counts a piece

    // ---- this wave's span [x0, x1): its record from the plan (span_layout.h).  Loaded
    // together (one round trip): the record and, for CSR with up to 256 rows, all of
    // kv_indptr (lane l holds entries l, l + 64, ...), so the first tile's indices follow
    // in the next round trip -- under load each trip is microseconds.
    const int32_t *rec = a.span + (int64_t)(blockIdx.x * NW + wave) * span::kRecord;
    const int32_t x0 = sload(rec, 0), x1 = sload(rec, 1);
    const int32_t count = x1 - x0;
    int32_t piece_tb = 0;  // first tile (in the sequence) of the current piece's task
    constexpr int kIndptrLanes = 4;  // rows <= 256 preloaded
    // kv_indptr holds active + 1 entries; an active outside [0, bcap] is a plan error (no tiles)
    const int32_t act = min(max(sload(a.active, 0), 0), a.batch_capacity);
    int32_t iptr[kIndptrLanes];
    if constexpr (CSR) {
#pragma unroll
        for (int k = 0; k < kIndptrLanes; ++k) iptr[k] = a.indptr[min(lane + 64 * k, act)];
    }

    if (count > 0) {
        Cursor c;
        c.q.r = sload(rec, 2);
        c.s = sload(rec, 3);
        c.g = sload(rec, 4);
        const int32_t j = sload(rec, 5);
        c.q.per_head = sload(rec, 7);
        c.q.c = sload(rec, 8);
        c.q.n = sload(rec, 9);
        c.q.L = sload(rec, 10);
        if constexpr (CSR) {
            const int32_t ri = min(c.q.r, act);
            int32_t v = iptr[0];
#pragma unroll
            for (int k = 1; k < kIndptrLanes; ++k)
                if (ri >= 64 * k) v = iptr[k];
            c.q.ind0 = ri < 64 * kIndptrLanes ? __builtin_amdgcn_readlane(v, ri & 63) : sload(a.indptr, ri);
        } else {
            c.q.ind0 = 0;
        }
        Req next = load_req<CSR>(a, c.q.r + 1);
        enter_split<CSR>(c, a);
        c.d.tok0 = c.begin + j * kTile;
        c.d.tl = c.nt - 1 - j;
        c.left = count;
        piece_tb = x0 - j;

        // ---- the pipeline's tile descriptors live in VGPR lanes: lane t % 8 of each ring
        // register holds tile t's field (tiles i .. i + 2 DEPTH - 1 are live), written by a
        // lane select and read with v_readlane, so no SGPRs carry them between stages.
        constexpr int kRing = 2 * DEPTH <= 8 ? 8 : 16;
        static_assert(2 * DEPTH <= kRing, "descriptor ring of 8 or 16 lanes");
        struct Ring {
            int32_t base, tok0, end, goff, qoff, slot, tl;
        } ring{};
        auto ring_put = [&](int32_t t, const Desc &d) {
            const bool at = lane == (t & (kRing - 1));
            ring.base = at ? d.base : ring.base;
            ring.tok0 = at ? d.tok0 : ring.tok0;
            ring.end = at ? d.end : ring.end;
            ring.goff = at ? d.goff : ring.goff;
            ring.qoff = at ? d.qoff : ring.qoff;
            ring.slot = at ? d.slot : ring.slot;
            ring.tl = at ? d.tl : ring.tl;
        };
        auto ring_get = [&](int32_t field, int32_t t) { return __builtin_amdgcn_readlane(field, t & (kRing - 1)); };

        // ---- prologue.  Loads complete in issue order, so a wait for one load is a wait
        // for every older one: each tile's indices are issued before the K/V rows of the
        // tiles ahead of it, and waiting for them never drains those.  Here: indices of
        // tiles 0 .. 2 DEPTH - 2, then the K/V and q of tiles 0 .. DEPTH - 1.
        uint4 kbuf[DEPTH][kRowsLoads], vbuf[DEPTH][kRowsLoads], qbuf[DEPTH];
        int32_t ibuf[DEPTH], ipro[DEPTH];
#pragma unroll
        for (int t = 0; t < 2 * DEPTH - 1; ++t) {
            const Desc d = describe<CSR>(c, next, a);
            ring_put(t, d);
            const int32_t v = span_index<CSR>(pages, d, lane, page_shift);
            if (t < DEPTH) ipro[t] = v;
            else ibuf[t % DEPTH] = v;
        }
#pragma unroll
        for (int t = 0; t < DEPTH; ++t) {
            __builtin_amdgcn_sched_barrier(0);
            Desc d;
            d.tok0 = ring_get(ring.tok0, t);
            d.end = ring_get(ring.end, t);
            d.goff = ring_get(ring.goff, t);
            d.qoff = ring_get(ring.qoff, t);
            span_issue<CSR>(kpool, vpool, pstride, tstride, d, ipro[t], page_mask, lane, kbuf[t], vbuf[t]);
            qbuf[t] = load_q16(qbase, qhoff, d);
        }
        __builtin_amdgcn_sched_barrier(0);

        float m_l = -INFINITY, den_l = 0.f;
        float acc[kHeads][4];
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;
        bool from_start = piece_tb == x0;  // the current piece began at its task's first tile

        // One tile (i): stage its rows (in K/V), describe tile i + 2 DEPTH - 1 and fetch
        // its indices, refill K/V/Q with tile i + DEPTH (whose indices were issued
        // before tile i + 1's rows), compute tile i, and close the piece at the end of
        // its task or span.  While tile i is computed, tiles i + 1 .. i + DEPTH are in
        // flight.  Iu (the index registers of tile i + DEPTH) is refilled with tile
        // i + 2 DEPTH - 1's indices through In (tile i + DEPTH - 1's, used a step ago).
        auto step = [&](uint4 (&Kr)[kRowsLoads], uint4 (&Vr)[kRowsLoads], uint4 &Q, int32_t &Iu, int32_t &In,
                        int32_t i) {
            Desc d;
            d.tok0 = ring_get(ring.tok0, i);
            d.end = ring_get(ring.end, i);
            d.slot = ring_get(ring.slot, i);
            d.tl = ring_get(ring.tl, i);
            int lane_v = lane;
            asm volatile("" : "+v"(lane_v));
            const int32_t nvalid = min(kTile, d.end - d.tok0);
            stage_rows(wt, Kr, Vr, lane_v);
            sh.q[wave][lane_v >> 4][lane_v & 15] = Q;  // d's task's q rows (unchanged within a task)
            {
                const Desc dn = describe<CSR>(c, next, a);
                ring_put(i + 2 * DEPTH - 1, dn);
                In = span_index<CSR>(pages, dn, lane, page_shift);
            }
            __builtin_amdgcn_sched_barrier(0);  // tile i + 2 DEPTH - 1's indices before tile i + DEPTH's rows
            {
                Desc di;
                di.tok0 = ring_get(ring.tok0, i + DEPTH);
                di.end = ring_get(ring.end, i + DEPTH);
                di.goff = ring_get(ring.goff, i + DEPTH);
                di.qoff = ring_get(ring.qoff, i + DEPTH);
                span_issue<CSR>(kpool, vpool, pstride, tstride, di, Iu, page_mask, lane, Kr, Vr);
                Q = load_q16(qbase, qhoff, di);
            }
            __builtin_amdgcn_sched_barrier(0);
            wave_sync();
            // Two waves share a SIMD (slots v and v ^ 4) and the issue arbiter favours
            // the older one; the wave that is behind its partner takes the higher
            // priority, so the pair -- and the workgroup -- finish together.
            if constexpr (NW == 8) {
                if (lane == 0) __hip_atomic_store(&sh.prog[wave], i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                const int32_t partner = uni(__hip_atomic_load(&sh.prog[wave ^ 4], __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_WORKGROUP));
                if (i <= partner) __builtin_amdgcn_s_setprio(2);
                else __builtin_amdgcn_s_setprio(0);
            }
            tile_compute<DT>(wt, sh.q[wave], nvalid, scale2, Roles(lane_v), m_l, den_l, acc);
            const bool task_end = d.tl == 0;
            if (task_end || i == count - 1) {
                float mh[kHeads], dh[kHeads];
                wave_state(m_l, den_l, acc, mh, dh);
                if (task_end && from_start) {
                    write_task(fresh(a), G, d.slot, acc, mh, dh, lane);
                } else {
                    // a cut piece: left for the task's last piece in the workgroup to finish
                    const int32_t tb = piece_tb, te = x0 + i + 1 + d.tl;
                    merge_piece<NW>(sh, a, G, tb, te, d.slot, from_start, acc, mh, dh, lane);
                }
                m_l = -INFINITY;
                den_l = 0.f;
#pragma unroll
                for (int h = 0; h < kHeads; ++h)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
                from_start = true;
                piece_tb = x0 + i + 1;
            }
        };

        // DEPTH tiles per iteration (the K/V/q and index registers rotate) and no exit
        // between them: every path into the loop header has issued the same loads in the
        // same order, so the waits stay partial.  The last count % DEPTH tiles run after
        // the loop.  Step u uses ibuf[u] (tile i + u + DEPTH) and refills
        // ibuf[(u + DEPTH - 1) % DEPTH] (tile i + u + 2 DEPTH - 1).
        int32_t i = 0;
        for (; i + DEPTH - 1 < count; i += DEPTH) {
#pragma unroll
            for (int u = 0; u < DEPTH; ++u)
                step(kbuf[u], vbuf[u], qbuf[u], ibuf[u], ibuf[(u + DEPTH - 1) % DEPTH], i + u);
        }
#pragma unroll
        for (int u = 0; u < DEPTH - 1; ++u)
            if (i + u < count) step(kbuf[u], vbuf[u], qbuf[u], ibuf[u], ibuf[(u + DEPTH - 1) % DEPTH], i + u);
    }

    __builtin_amdgcn_s_setprio(0);
}

template <int DT, bool CSR, int NW, int DEPTH>
int launch_span_d(const sgd_decode_args &a, hipStream_t stream) {
    static bool attr = false;
    constexpr int bytes = (int)sizeof(SpanShared<NW>);
    if (!attr) {
        if (hipFuncSetAttribute((const void *)k_attention_span<DT, CSR, NW, DEPTH>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
            return einval("span attention: cannot reserve %d B of LDS", bytes);
        attr = true;
    }
    hipLaunchKernelGGL((k_attention_span<DT, CSR, NW, DEPTH>), dim3(a.span_units / NW), dim3(64 * NW), bytes, stream,
                       a);
    return launch_status("persistent_decode(span)");
}

// Eight waves per workgroup (one workgroup per CU, two waves per SIMD with up to 256
// VGPRs each), three tiles in flight per wave while one is computed: 192 KB per CU,
// the bytes in flight the HBM needs at its loaded latency.
template <int DT, bool CSR>
int launch_span_t(const sgd_decode_args &a, hipStream_t stream) {
    return launch_span_d<DT, CSR, span::kWaves, 3>(a, stream);
}

}  // namespace

bool valu_supported(const sgd_decode_args &a);

bool span_supported(const sgd_decode_args &a) {
    if (!valu_supported(a)) return false;
    if (!a.tile_prefix || !a.span || !a.edge || a.batch_capacity <= 0) return false;
    if (a.span_units <= 0 || a.span_units % span::kWaves) return false;
    // K and V share their strides; byte strides and table/q offsets fit 32 bits
    for (int i = 0; i < 4; ++i)
        if (a.k_stride[i] != a.v_stride[i]) return false;
    const int64_t lim = 1ll << 31;
    if (a.k_stride[0] * 2 >= lim || a.k_stride[1] * 2 >= lim || a.k_stride[2] * 2 * a.kv_heads >= lim) return false;
    if (a.k_stride[0] < 0 || a.k_stride[1] < 0 || a.k_stride[2] < 0) return false;
    if (!a.csr && (a.pt_stride[1] != 1 || a.pt_stride[0] < 0 || (int64_t)a.batch_capacity * a.pt_stride[0] >= lim))
        return false;
    if ((int64_t)a.batch_capacity * a.q_stride[0] >= lim || a.q_stride[0] < 0 || a.q_stride[1] < 0) return false;
    if ((int64_t)a.batch_capacity * a.query_heads * a.max_splits >= lim) return false;
    // 16-byte q rows and partial rows
    if (a.q_stride[2] != 1 || a.q_stride[0] % 8 || a.q_stride[1] % 8) return false;
    if ((reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.partial) |
         reinterpret_cast<uintptr_t>(a.edge)) & 15)
        return false;
    return true;
}

int launch_attention_span(const sgd_decode_args &a, hipStream_t stream) {
    if (a.dtype == SGD_BF16)
        return a.csr ? launch_span_t<SGD_BF16, true>(a, stream) : launch_span_t<SGD_BF16, false>(a, stream);
    return a.csr ? launch_span_t<SGD_FP16, true>(a, stream) : launch_span_t<SGD_FP16, false>(a, stream);
}

}  // namespace sgd
