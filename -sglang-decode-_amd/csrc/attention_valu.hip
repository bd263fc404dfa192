// Persistent paged GQA decode attention for query-head groups of up to 4 heads
// (Llama-3-8B: 32 q / 8 kv), head_dim 128, unit dim stride -- the VALU path.
//
// Contraction sizes per token are 4 heads x 128 dims for QK^T and for P.V: far
// too narrow for a dense MFMA tile, so the math runs on the VALU with packed
// 16-bit dot products (v_dot2c_f32_bf16 / _f16, fp32 accumulate) and wave64 DPP
// reductions.  The kernel is HBM-bound; the design goal is to keep enough KV
// bytes in flight, touch each KV byte once, and never let a workgroup sit idle
// between tasks.
//
// Worker = one workgroup of 4 waves (two workgroups per CU).  A task (record, kv
// head) is split across the waves in 32-token tiles (tile i -> wave i % 4).  Per
// wave and tile:
//   1. gather: 8 x 16-byte loads for K and 8 for V, each covering 4 token rows of
//      256 B (16 lanes per row, fully coalesced).  Row addresses come from the
//      page table / CSR indices: one load fetches the tile's 32 indices, and
//      DPP row_newbcast hands each 16-lane row its token's index.
//   2. stage: the K and V tile go to the wave's LDS tile (row-major, 256 B rows),
//      shared by all 4 query heads of the group.
//   3. QK^T: 8 lanes per token, each 16 dims, 4 heads -> 32 dot2; a 3-step DPP
//      reduce-scatter leaves each lane with one head's score.
//   4. online softmax in fp32 (exp2 domain); p is rounded to the KV dtype for P.V
//      (kernels/attention.py:78) and written to LDS as token pairs.
//   5. P.V: lane owns 4 dims x 4 heads; dot2 over token pairs (V repacked with
//      v_perm_b32), half-waves take alternate token pairs.
//
// Pipelining.  Each wave streams "items" (its tiles of the current task, then of
// the next task): the K/V loads of the next item and the index load of the item
// after it are in flight while an item is computed, across task boundaries.
// Wave 0 also runs the task scheduler: the dispatch chain of the plan's mode
// (claim -> pack -> order -> record -> indptr, kernels/attention.py:99-130 and
// :23-47) advances one dependent memory access per tile, so the descriptor of
// the task after next is ready at the end of each task, and the next task's q
// rows are staged in LDS meanwhile.  At the end of a task the 4 waves'
// (m, den, acc) are merged through LDS and the normalized partial and
// natural-log LSE go to slot (request, head, split) (kernels/attention.py:81-84).
#include "attention_common.h"

namespace sgd {
namespace {

constexpr int kWavesMax = 16;             // waves per workgroup: 8 (two per CU) or 16 (one per CU)
constexpr int kTile = 16;                 // tokens per wave per tile
constexpr int kRowsLoads = kTile / 4;     // 16-byte loads per K (and per V) tile: 4 rows each
constexpr int kD = 128;                   // head_dim
constexpr int kHeads = 4;                 // padded group
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct WaveTile {
    uint4 k[kTile][kD / 8];          // 4 KB  (also this wave's task-merge area: 4 heads x 128 fp32)
    uint4 v[kTile][kD / 8];          // 4 KB
    uint4 p[kTile / 2];              // token-pair probabilities: [pair] -> 4 heads x (p[2i], p[2i+1])
};

// One resolved task, published by the scheduler in LDS.
struct TaskDesc {
    int32_t request, split, start, end, group, ind0, valid, pad;
};

template <int kWaves>
struct ValuShared {
    WaveTile w[kWaves];
    uint4 q[2][kHeads][kD / 8];      // q rows of the current / next task
    TaskDesc desc[4];                // ring: current, next, and the one being resolved
    float cm[kWaves][kHeads];
    float cd[kWaves][kHeads];
    int32_t cursor;
};

template <int DT>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (DT == SGD_BF16)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                               false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    if constexpr (DT == SGD_BF16) {
        bf16x2 r = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, r);
    } else {
        f16x2 r = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, r);
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf,
                                                                  false));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
    return __builtin_amdgcn_mov_dpp(x, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ int32_t uni(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }

constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor3 = 0x1B;       // quad_perm [3,2,1,0]
constexpr int kRowShl8 = 0x108;       // row_shl:8
constexpr int kRowRor8 = 0x128;       // row_ror:8
constexpr int kRowHalfMirror = 0x141; // row_half_mirror
constexpr int kRowNewBcast = 0x150;   // row_newbcast:n

// ------------------------------------------------------------------ task scheduler
// Produces this worker's tasks in the order of its mode, resolving each to a
// TaskDesc.  step() performs at most one dependent memory access: it consumes the
// load issued by the previous step and issues the next one.  Runs on wave 0 with
// all lanes active (uniform addresses); only lane 0 performs the claim atomic.
enum SchedPhase : int32_t {
    kStart, kStaticWait, kClaimWait, kPackWait, kOrderWait, kRecordWait, kIndWait, kR0Step, kR0Wait,
    kR0FinWait, kReady, kExhausted
};

template <bool CSR>
struct Scheduler {
    int32_t phase, issued, task, rec, pack_next, pack_left, lo, hi, mid;
    int32_t request, split, start, end, ind0;
    int32_t p0, p1, p2, p3;  // loads in flight (uniform values, read at the next step)
    bool started;

    __device__ void init(const sgd_decode_args &a) {
        mode = uni(*a.mode);
        total = uni(*a.record_count) * a.kv_heads;
        num_packs = uni(*a.num_packs);
        active = uni(*a.active);
        phase = kStart;
        issued = 0;
        pack_left = 0;
        pack_next = 0;
        started = false;
        task = 0;
    }

    __device__ bool busy() const { return phase != kReady && phase != kExhausted; }

    __device__ void issue_order(const sgd_decode_args &a) {
        rec = task / a.kv_heads;
        p0 = a.order[rec];
        phase = kOrderWait;
    }

    __device__ void issue_record(const sgd_decode_args &a) {
        p0 = a.request[rec];
        p1 = a.split[rec];
        p2 = a.begin[rec];
        p3 = a.end[rec];
        phase = kRecordWait;
    }

    __device__ void finish_record(const sgd_decode_args &a) {
        if constexpr (CSR) {
            p0 = a.indptr[request];
            phase = kIndWait;
        } else {
            ind0 = 0;
            phase = kReady;
        }
    }

    // mode, total tasks, pack count and active batch are launch constants read once.
    int32_t mode, total, num_packs, active;

    __device__ void step(const sgd_decode_args &a, int32_t lane) {
        switch (phase) {
            case kStart:
                if (mode <= 1) {
                    const int32_t t = (int32_t)blockIdx.x + issued * a.workers;
                    if (t >= total) { phase = kExhausted; return; }
                    ++issued;
                    task = t;
                    if (mode == 1) {
                        issue_order(a);
                    } else {
                        rec = t / a.kv_heads;
                        lo = 0;
                        hi = active;
                        phase = kR0Step;
                    }
                } else if (mode == 2) {
                    p0 = started ? a.static_next[task] : a.static_head[blockIdx.x];
                    started = true;
                    phase = kStaticWait;
                } else if (pack_left > 0) {
                    task = pack_next++;
                    --pack_left;
                    issue_order(a);
                } else {
                    int32_t v = 0;
                    if (lane == 0) v = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    p0 = v;
                    phase = kClaimWait;
                }
                return;
            case kStaticWait: {
                const int32_t t = uni(p0);
                if (t < 0 || t >= total) { phase = kExhausted; return; }
                task = t;
                rec = t / a.kv_heads;
                issue_record(a);
                return;
            }
            case kClaimWait: {
                const int32_t c = uni(p0);
                if (c < 0 || c >= num_packs) { phase = kExhausted; return; }
                p0 = a.pack_first[c];
                p1 = a.pack_count[c];
                phase = kPackWait;
                return;
            }
            case kPackWait:
                task = uni(p0);
                pack_next = task + 1;
                pack_left = uni(p1) - 1;
                issue_order(a);
                return;
            case kOrderWait:
                rec = uni(p0);
                issue_record(a);
                return;
            case kRecordWait:
                request = uni(p0);
                split = uni(p1);
                start = uni(p2);
                end = uni(p3);
                finish_record(a);
                return;
            case kIndWait:
                ind0 = uni(p0);
                phase = kReady;
                return;
            case kR0Step:  // upper-bound search of the request offsets (attention.py:25-39)
                if (lo < hi) {
                    mid = (lo + hi) >> 1;
                    p0 = a.offsets[mid + 1];
                    phase = kR0Wait;
                } else {
                    request = lo;
                    p0 = a.offsets[lo];
                    p1 = a.chunk[lo];
                    p2 = a.lengths[lo];
                    phase = kR0FinWait;
                }
                return;
            case kR0Wait:
                if (rec >= uni(p0)) lo = mid + 1;
                else hi = mid;
                phase = kR0Step;
                return;
            case kR0FinWait: {
                split = rec - uni(p0);
                const int32_t ch = uni(p1);
                start = split * ch;
                end = min(start + ch, uni(p2));
                finish_record(a);
                return;
            }
            default:
                return;
        }
    }

    __device__ void finish(const sgd_decode_args &a, int32_t lane) {
        while (busy()) step(a, lane);
    }

    __device__ TaskDesc desc(int32_t kv_heads) const {
        TaskDesc d;
        d.valid = phase == kReady;
        d.request = request;
        d.split = split;
        d.start = start;
        d.end = end;
        d.group = task % kv_heads;
        d.ind0 = ind0;
        d.pad = 0;
        return d;
    }
};

// ------------------------------------------------------------------ gathers
struct TaskView {
    int32_t request, split, start, end, group, ind0, valid, ntiles;
    const char *kbase, *vbase;
};

__device__ __forceinline__ TaskView view_of(const TaskDesc &d, const sgd_decode_args &a, int64_t kh, int64_t vh) {
    TaskView t;
    t.valid = uni(d.valid);
    t.request = uni(d.request);
    t.split = uni(d.split);
    t.start = uni(d.start);
    t.end = uni(d.end);
    t.group = uni(d.group);
    t.ind0 = uni(d.ind0);
    t.ntiles = t.valid ? (t.end - t.start + kTile - 1) / kTile : 0;
    t.kbase = static_cast<const char *>(a.k) + t.group * kh;
    t.vbase = static_cast<const char *>(a.v) + t.group * vh;
    return t;
}

// lane 16r + i (i < kRowsLoads) fetches the page/slot index of token tok0 + 4i + r
template <bool CSR>
__device__ __forceinline__ int32_t load_tile_index(const sgd_decode_args &a, const TaskView &t, int32_t tok0,
                                                   int lane, int page_shift) {
    const int r = lane >> 4, i = lane & 15;
    const int32_t tok = tok0 + 4 * i + r;
    int32_t v = 0;
    if (i < kRowsLoads && tok < t.end) {
        if constexpr (CSR) v = a.pages[t.ind0 + tok];
        else v = a.pages[(int64_t)t.request * a.pt_stride[0] + (int64_t)(tok >> page_shift) * a.pt_stride[1]];
    }
    return v;
}

struct Strides {
    int64_t kp, kt, vp, vt;
};

template <bool CSR, bool FULL>
__device__ __forceinline__ void load_tile(const TaskView &t, const Strides &st, int32_t tok0, int32_t idxv,
                                          int32_t page_mask, int lane, uint4 (&kr)[kRowsLoads],
                                          uint4 (&vr)[kRowsLoads]) {
    const int r = lane >> 4, c = lane & 15;
#define SGD_LOAD_ROW(I)                                                                              \
    {                                                                                                \
        const uint32_t phys = (uint32_t)dpp_i<kRowNewBcast + I>(idxv);                               \
        const int32_t tok = tok0 + 4 * I + r;                                                        \
        int64_t ko = (int64_t)phys * st.kp + c * 16, vo = (int64_t)phys * st.vp + c * 16;            \
        if constexpr (!CSR) {                                                                        \
            const int32_t inner = tok & page_mask;                                                   \
            ko += (int64_t)inner * st.kt;                                                            \
            vo += (int64_t)inner * st.vt;                                                            \
        }                                                                                            \
        if (FULL || tok < t.end) {                                                                   \
            kr[I] = *reinterpret_cast<const uint4 *>(t.kbase + ko);                                  \
            vr[I] = *reinterpret_cast<const uint4 *>(t.vbase + vo);                                  \
        } else {                                                                                     \
            kr[I] = make_uint4(0, 0, 0, 0);                                                          \
            vr[I] = make_uint4(0, 0, 0, 0);                                                          \
        }                                                                                            \
    }
    static_assert(kRowsLoads == 4, "one SGD_LOAD_ROW per 4-row load");
    SGD_LOAD_ROW(0) SGD_LOAD_ROW(1) SGD_LOAD_ROW(2) SGD_LOAD_ROW(3)
#undef SGD_LOAD_ROW
}

template <bool CSR>
__device__ __forceinline__ void issue_tile(const TaskView &t, const Strides &st, int32_t tile, int32_t idxv,
                                           int32_t page_mask, int lane, uint4 (&kr)[kRowsLoads],
                                           uint4 (&vr)[kRowsLoads]) {
    const int32_t tok0 = t.start + tile * kTile;
    if (tok0 + kTile <= t.end) load_tile<CSR, true>(t, st, tok0, idxv, page_mask, lane, kr, vr);
    else load_tile<CSR, false>(t, st, tok0, idxv, page_mask, lane, kr, vr);
}

// ------------------------------------------------------------------ kernel
template <int DT, bool CSR, int kWaves>
__global__ __launch_bounds__(64 * kWaves, 4) void k_attention_valu(sgd_decode_args a) {
    // 16 waves per CU (two 8-wave or one 16-wave workgroup): the load concurrency the
    // random row gathers need to approach the HBM ceiling (4 waves per SIMD, <= 128
    // VGPRs).
    extern __shared__ __align__(16) char dyn_smem[];
    ValuShared<kWaves> &sh = *reinterpret_cast<ValuShared<kWaves> *>(dyn_smem);
    const int lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
    WaveTile &wt = sh.w[wave];
    const int32_t G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    const int page_shift = __builtin_ctz((unsigned)a.page_size);  // page_size is a power of two here
    const int32_t page_mask = a.page_size - 1;

    // Lane roles (recomputed where used from a laundered lane id, so the compiler
    // rebuilds per-lane LDS addresses each tile instead of holding them all live):
    //  QK:  8 lanes per token; qg = lane / 8 picks the token, qj = lane % 8 owns the
    //       16 B chunks qj and qj + 8; after the reduce-scatter the lane holds head
    //       hs = 2*bit2(qj) + bit1(qj).
    //  P.V: half ph = lane / 32 takes token pairs 2s + ph; pd = lane % 32 owns dims
    //       4*pd .. 4*pd+3.
    auto roles = [](int l, int &qg, int &qj, int &hs, bool &b2, bool &b1, int &ph, int &pd) {
        qg = l >> 3;
        qj = l & 7;
        hs = ((qj >> 2) << 1) | ((qj >> 1) & 1);
        b2 = (qj & 4) != 0;
        b1 = (qj & 2) != 0;
        ph = l >> 5;
        pd = l & 31;
    };

    for_each_task(a, &sh.cursor, [&](int32_t task, int32_t mode) {
        const TaskInfo ti = decode_task(a, task, mode);
        __syncthreads();  // the previous task's merge is done with shared memory
        if (wave == 0) {  // stage the group's q rows; heads >= G are zero
            const int h = lane >> 4, c = lane & 15;
            uint4 w = make_uint4(0, 0, 0, 0);
            if (h < G) {
                const int32_t qd = (int32_t)a.q_stride[2];
                const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (int64_t)ti.request * a.q_stride[0] +
                                     (int64_t)(ti.group * G + h) * a.q_stride[1] + (int64_t)(c * 8) * qd;
                uint32_t w4[4] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 8; ++e) w4[e >> 1] |= (uint32_t)qp[e * qd] << (16 * (e & 1));
                w = make_uint4(w4[0], w4[1], w4[2], w4[3]);
            }
            sh.q[0][h][c] = w;
        }
        TaskView T;
        T.request = uni(ti.request);
        T.split = uni(ti.split);
        T.start = uni(ti.start);
        T.end = uni(ti.end);
        T.group = uni(ti.group);
        T.ind0 = CSR ? uni(a.indptr[T.request]) : 0;
        T.valid = 1;
        T.ntiles = (T.end - T.start + kTile - 1) / kTile;
        T.kbase = static_cast<const char *>(a.k) + T.group * (a.k_stride[2] * 2);
        T.vbase = static_cast<const char *>(a.v) + T.group * (a.v_stride[2] * 2);
        const Strides st{a.k_stride[0] * 2, a.k_stride[1] * 2, a.v_stride[0] * 2, a.v_stride[1] * 2};
        __syncthreads();

        const int32_t n0 = T.ntiles > wave ? (T.ntiles - wave + kWaves - 1) / kWaves : 0;
        uint4 kr[kRowsLoads], vr[kRowsLoads];
        int32_t idx_next = 0;
        if (n0 > 0) {
            const int32_t i0 = load_tile_index<CSR>(a, T, T.start + wave * kTile, lane, page_shift);
            issue_tile<CSR>(T, st, wave, i0, page_mask, lane, kr, vr);
            if (n0 > 1) idx_next = load_tile_index<CSR>(a, T, T.start + (wave + kWaves) * kTile, lane, page_shift);
        }
        float m_l = -INFINITY, den_l = 0.f;  // this lane's head hs (QK roles)
        float acc[kHeads][4];
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;

        for (int32_t e = 0; e < n0; ++e) {
            int lane_v = lane;
            asm volatile("" : "+v"(lane_v));
            int qg, qj, hs, ph, pd;
            bool b2, b1;
            roles(lane_v, qg, qj, hs, b2, b1, ph, pd);
            // stage item e (rows 4i + r, 16 lanes per 256 B row)
#pragma unroll
            for (int i = 0; i < kRowsLoads; ++i) {
                wt.k[4 * i + (lane_v >> 4)][lane_v & 15] = kr[i];
                wt.v[4 * i + (lane_v >> 4)][lane_v & 15] = vr[i];
            }
            const int32_t tile = wave + kWaves * e;
            if (e + 1 < n0) issue_tile<CSR>(T, st, tile + kWaves, idx_next, page_mask, lane, kr, vr);
            if (e + 2 < n0) idx_next = load_tile_index<CSR>(a, T, T.start + (tile + 2 * kWaves) * kTile, lane, page_shift);
            wave_sync();

            const int32_t nvalid = min(kTile, T.end - (T.start + tile * kTile));
            // QK^T: 2 passes of 8 tokens; token 8*pass + qg
            constexpr int kPasses = kTile / 8;
            float s[kPasses];
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) {
                const int tk = 8 * pass + qg;
                const uint4 lo = wt.k[tk][qj], hi = wt.k[tk][qj + 8];
                const uint32_t kv[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                float sh4[kHeads];
#pragma unroll
                for (int h = 0; h < kHeads; ++h) {
                    const uint4 ql = sh.q[0][h][qj], qh = sh.q[0][h][qj + 8];
                    const uint32_t qv[8] = {ql.x, ql.y, ql.z, ql.w, qh.x, qh.y, qh.z, qh.w};
                    float x = 0.f;
#pragma unroll
                    for (int q = 0; q < 8; ++q) x = dot2<DT>(qv[q], kv[q], x);
                    sh4[h] = x;
                }
                // reduce-scatter over the 8 lanes of the token
                float k0 = b2 ? sh4[2] : sh4[0], k1 = b2 ? sh4[3] : sh4[1];
                const float s0 = b2 ? sh4[0] : sh4[2], s1 = b2 ? sh4[1] : sh4[3];
                k0 += dpp<kRowHalfMirror>(s0);
                k1 += dpp<kRowHalfMirror>(s1);
                float kk = b1 ? k1 : k0;
                const float ss = b1 ? k0 : k1;
                kk += dpp<kQuadXor3>(ss);
                kk += dpp<kQuadXor1>(kk);
                s[pass] = (tk < nvalid) ? kk * scale2 : -INFINITY;
            }
            // online softmax (exp2 domain); max over the tile for head hs
            float mx = fmaxf(s[0], s[1]);
            mx = fmaxf(mx, dpp<kRowRor8>(mx));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_l, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_l - m_new);
            m_l = m_new;
            float p[kPasses];
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) p[pass] = __builtin_amdgcn_exp2f(s[pass] - m_new);
            den_l = den_l * alpha + (p[0] + p[1]);
            // pairs (8*pass + qg, +1) for even qg, written once per (pair, head)
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) {
                const float pn = dpp<kRowShl8>(p[pass]);
                if (((qg & 1) == 0) && ((qj & 1) == 0)) {
                    uint32_t *prow = reinterpret_cast<uint32_t *>(&wt.p[4 * pass + (qg >> 1)]);
                    prow[hs] = pack2<DT>(p[pass], pn);
                }
            }
            // per-head rescale of the P.V accumulators (heads are held by lanes 0, 2, 4, 6)
#pragma unroll
            for (int h = 0; h < kHeads; ++h) {
                const int src_lane = ((h >> 1) << 2) | ((h & 1) << 1);
                const float al = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), src_lane));
#pragma unroll
                for (int d = 0; d < 4; ++d) acc[h][d] *= al;
            }
            wave_sync();

            // P.V over token pairs
#pragma unroll
            for (int stp = 0; stp < kTile / 4; ++stp) {
                const int pr = 2 * stp + ph;
                const uint2 va = *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(&wt.v[2 * pr][0]) + pd * 8);
                const uint2 vb = *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(&wt.v[2 * pr + 1][0]) + pd * 8);
                const uint4 pp = wt.p[pr];
                const uint32_t vv[4] = {__builtin_amdgcn_perm(vb.x, va.x, 0x05040100u),
                                        __builtin_amdgcn_perm(vb.x, va.x, 0x07060302u),
                                        __builtin_amdgcn_perm(vb.y, va.y, 0x05040100u),
                                        __builtin_amdgcn_perm(vb.y, va.y, 0x07060302u)};
                const uint32_t pq[4] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
                for (int h = 0; h < kHeads; ++h)
#pragma unroll
                    for (int d = 0; d < 4; ++d) acc[h][d] = dot2<DT>(pq[h], vv[d], acc[h][d]);
            }
            wave_sync();
        }

        // ---- end of the wave's tiles: reduce within the wave, then merge the waves
        int qg, qj, hs, ph, pd;
        bool b2, b1;
        roles(lane, qg, qj, hs, b2, b1, ph, pd);
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[h][d] += __shfl_xor(acc[h][d], 32, 64);
        float dl = den_l;  // sum over the 8 token groups sharing this lane's head
        dl += dpp<kRowRor8>(dl);
        dl += __shfl_xor(dl, 16, 64);
        dl += __shfl_xor(dl, 32, 64);
        float *comb = reinterpret_cast<float *>(&wt.k[0][0]);  // [head][128] fp32, reuses this wave's K tile
        if (lane < 32) {
#pragma unroll
            for (int h = 0; h < kHeads; ++h)
                *reinterpret_cast<float4 *>(&comb[h * kD + pd * 4]) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        }
        if (lane < 8 && (lane & 1) == 0) {
            sh.cm[wave][hs] = m_l;
            sh.cd[wave][hs] = dl;
        }
        __syncthreads();
        if (threadIdx.x < kHeads * kD) {   // one (head, dim) output per thread: 4 heads x 128 dims
            static_assert(kWaves * 64 >= kHeads * kD, "merge maps one thread per output");
            const int h = threadIdx.x / kD, d = threadIdx.x % kD;
            if (h < G) {
                float mm = -INFINITY;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sh.cm[w][h]);
                float dd = 0.f, x = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float sc = __builtin_amdgcn_exp2f(sh.cm[w][h] - mm);
                    dd += sh.cd[w][h] * sc;
                    x += reinterpret_cast<const float *>(&sh.w[w].k[0][0])[h * kD + d] * sc;
                }
                const int64_t slot = ((int64_t)T.request * a.query_heads + T.group * G + h) * a.max_splits + T.split;
                a.partial[slot * kD + d] = x / dd;
                if (d == 0) a.lse[slot] = (mm + __log2f(dd)) * kLn2;
            }
        }
    });
}

template <int DT, bool CSR, int kWaves>
int launch_valu_w(const sgd_decode_args &a, hipStream_t stream) {
    static bool attr = false;
    const int bytes = (int)sizeof(ValuShared<kWaves>);
    if (!attr) {
        if (hipFuncSetAttribute((const void *)k_attention_valu<DT, CSR, kWaves>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
            return einval("valu attention: cannot reserve %d B of LDS", bytes);
        attr = true;
    }
    hipLaunchKernelGGL((k_attention_valu<DT, CSR, kWaves>), dim3(a.workers), dim3(64 * kWaves), bytes, stream, a);
    return launch_status("persistent_decode(valu)");
}

// Waves per workgroup from the environment variable SGD_VALU_WAVES (8 or 16, default 16).
int valu_waves() {
    static int w = [] {
        const char *e = getenv("SGD_VALU_WAVES");
        return (e && atoi(e) == 8) ? 8 : 16;
    }();
    return w;
}

template <int DT, bool CSR>
int launch_valu_t(const sgd_decode_args &a, hipStream_t stream) {
    return valu_waves() == 8 ? launch_valu_w<DT, CSR, 8>(a, stream) : launch_valu_w<DT, CSR, 16>(a, stream);
}

}  // namespace

bool valu_supported(const sgd_decode_args &a) {
    const int g = a.query_heads / a.kv_heads;
    if (g > kHeads || a.head_dim != kD) return false;
    if (a.k_stride[3] != 1 || a.v_stride[3] != 1) return false;
    if ((reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v)) & 15) return false;
    if (a.page_size & (a.page_size - 1)) return false;
    for (int i = 0; i < 3; ++i)
        if (a.k_stride[i] % 8 || a.v_stride[i] % 8) return false;
    // 32-bit page index times the page stride must stay a valid 64-bit byte offset
    return a.k_stride[0] < (1ll << 40) && a.v_stride[0] < (1ll << 40);
}

int launch_attention_valu(const sgd_decode_args &a, hipStream_t stream) {
    if (a.dtype == SGD_BF16)
        return a.csr ? launch_valu_t<SGD_BF16, true>(a, stream) : launch_valu_t<SGD_BF16, false>(a, stream);
    return a.csr ? launch_valu_t<SGD_FP16, true>(a, stream) : launch_valu_t<SGD_FP16, false>(a, stream);
}

}  // namespace sgd
