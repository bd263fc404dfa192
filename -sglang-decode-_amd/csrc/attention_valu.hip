// Persistent paged GQA decode attention for query-head groups of up to 4 heads
// (Llama-3-8B: 32 q / 8 kv), head_dim 64, 128 or 256, unit dim stride -- the
// per-task VALU kernel.
//
// Contraction sizes per token are 4 heads x D dims for QK^T and for P.V: far
// too narrow for a dense MFMA tile, so the math runs on the VALU with packed
// 16-bit dot products (v_dot2_f32_bf16 / _f16, fp32 accumulate) and wave64 DPP
// reductions (valu_ops.h).  The kernel is HBM-bound.
//
// Worker = one workgroup of kWaves = 8 waves, two workgroups per CU: 16 waves per CU,
// the load concurrency the random 256 B row gathers need, and enough waves to hide the
// tile math (~395 VALU instructions per tile and wave, about 40% of the SIMDs' issue
// slots over a launch).  Tasks come from the plan's dispatch (attention_common.h); each
// task (record, kv head) is dealt to the waves in tiles of 2048 / D tokens (4 KB of K
// and of V; tile i -> wave i % kWaves).  Per wave and tile: gather K and V rows (4 x 16
// B loads each), stage
// them in the wave's LDS tile shared by the group's query heads, QK^T with a DPP
// reduce-scatter, online softmax in the exp2 domain, P rounded to the KV dtype
// (kernels/attention.py:78), P.V over token pairs.  The next tile's K/V loads and
// the index load of the tile after it are in flight while a tile is computed.
// At the end of a task the waves' (m, den, acc) are merged through LDS, and the
// normalized partial and natural-log LSE go to slot (request, head, split)
// (kernels/attention.py:81-84).  The last wave, which holds the fewest tiles, finds
// the worker's next task (claim, dispatch entry or record, the first tiles' page/slot
// indices) once its own tiles are done, while the others finish theirs.
//
#include "valu_ops.h"

namespace sgd {
namespace {

using namespace valu;

constexpr int kIndptrLds = 256;  // CSR: kv_indptr entries kept in LDS (rows beyond read memory)

template <int kWaves, int D>
struct ValuShared {
    static constexpr int kTile = Geo<D>::kTile;
    WaveTile<D> w[kWaves];
    uint4 q[kHeads][D / 8];          // q rows of the current task
    float cm[kWaves][kHeads];
    float cd[kWaves][kHeads];
    int32_t indptr[kIndptrLds];
    int32_t cursor;
    Prefetched pf[2];                   // the worker's next task (prefetch_next)
    int32_t pf_idx[2][kTile * kWaves];  // page/slot indices of its first kWaves tiles
};

// ------------------------------------------------------------------ kernel
template <int DT, bool CSR, int kWaves, int D, bool kOut, bool kPow2>
__global__ __launch_bounds__(64 * kWaves, 4) void k_attention_valu(sgd_decode_args a) {
    // 16 waves per CU (two 8-wave workgroups): the load concurrency the random row
    // gathers need to approach the HBM ceiling (4 waves per SIMD, <= 128 VGPRs).
    extern __shared__ __align__(16) char dyn_smem[];
    using Sh = ValuShared<kWaves, D>;
    constexpr int kTile = Geo<D>::kTile, kQChunks = kHeads * D / 8, kQPerLane = (kQChunks + 63) / 64;
    Sh &sh = *reinterpret_cast<Sh *>(dyn_smem);
    const int lane0 = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
    WaveTile<D> &wt = sh.w[wave];
    const int32_t G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    const PageMap<kPow2> pm(a.page_size);
    // CSR: kv_indptr (active + 1 entries) once per launch, so a task's index base is an
    // LDS read rather than a memory round trip between its claim and its first loads.
    int32_t iptr_n = 0;
    if constexpr (CSR) {
        iptr_n = min(__builtin_amdgcn_readfirstlane(*a.active) + 1, kIndptrLds);
        for (int i = threadIdx.x; i < iptr_n; i += 64 * kWaves) sh.indptr[i] = a.indptr[i];
    }
    clear_prefetched(sh.pf);
    lds_barrier();

    for_each_task<true>(a, &sh.cursor, [&](int32_t task, const TaskInfo &ti, const Successor &succ) {
        int lane = lane0;  // laundered per task: per-lane offsets are rebuilt, not held live
        asm volatile("" : "+v"(lane));
        // Global loads first -- q rows (wave 0), then the request's index base, the first
        // tile's indices and its K/V rows into registers -- so that they are in flight
        // across the barriers that hand shared memory over from the previous task.
        // wave 0: 16 B chunk lane + 64 j of the group's q rows (head = chunk / (D / 8)); zero past G
        uint4 qrow[kQPerLane];
#pragma unroll
        for (int j = 0; j < kQPerLane; ++j) {
            qrow[j] = make_uint4(0, 0, 0, 0);
            const int ci = lane + 64 * j, h = ci / (D / 8), c = ci % (D / 8);
            if (wave == 0 && ci < kQChunks && h < G) {
                const int32_t qd = (int32_t)a.q_stride[2];
                const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (int64_t)ti.request * a.q_stride[0] +
                                     (int64_t)(ti.group * G + h) * a.q_stride[1] + (int64_t)(c * 8) * qd;
                uint32_t w4[4] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 8; ++e) w4[e >> 1] |= (uint32_t)qp[e * qd] << (16 * (e & 1));
                qrow[j] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
            }
        }
        TileSrc T;
        T.request = uni(ti.request);
        T.start = uni(ti.start);
        T.end = uni(ti.end);
        const int32_t split = uni(ti.split), group = uni(ti.group);
        // kOut (sgd_decode_args.out set): a request's first split also writes its normalized
        // rows to `out` -- final for a single-split request, overwritten by the merge
        // otherwise.  Testing split 0 needs no load of the request's length.  A separate
        // build, so launches without `out` run the kernel without any of it.
        const bool first = kOut && split == 0;
        T.ind0 = CSR ? uni(T.request < iptr_n ? sh.indptr[T.request] : a.indptr[T.request]) : 0;
        T.kbase = static_cast<const char *>(a.k) + group * (a.k_stride[2] * 2);
        T.vbase = static_cast<const char *>(a.v) + group * (a.v_stride[2] * 2);
        T.kp = a.k_stride[0] * 2;
        T.kt = a.k_stride[1] * 2;
        T.vp = a.v_stride[0] * 2;
        T.vt = a.v_stride[1] * 2;
        const int32_t ntiles = (T.end - T.start + kTile - 1) / kTile;
        const int32_t n0 = ntiles > wave ? (ntiles - wave + kWaves - 1) / kWaves : 0;
        const bool prefetched = uni(sh.pf[succ.cur].task) == task;
        uint4 kr[kRowsLoads], vr[kRowsLoads];
        int32_t idx_next = 0;
        if (n0 > 0) {
            int32_t i0;
            if (prefetched) {
                const int row = index_row<D>(lane);
                i0 = row >= 0 ? sh.pf_idx[succ.cur][wave * kTile + row] : 0;
            } else {
                i0 = tile_index<CSR, D>(a, T, T.start + wave * kTile, lane, pm);
            }
            tile_issue<CSR, D>(T, wave, i0, pm, lane, kr, vr);
            if (n0 > 1) idx_next = tile_index<CSR, D>(a, T, T.start + (wave + kWaves) * kTile, lane, pm);
        }
        lds_barrier();  // the previous task's merge is done with shared memory
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < kQPerLane; ++j) {
                const int ci = lane + 64 * j;
                if (ci < kQChunks) sh.q[ci / (D / 8)][ci % (D / 8)] = qrow[j];
            }
        }
        lds_barrier();
        float m_l = -INFINITY, den_l = 0.f;  // this lane's head (QK roles)
        float acc[kHeads][4];
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;

        for (int32_t e = 0; e < n0; ++e) {
            // Lane roles come from a laundered lane id, so the compiler rebuilds the
            // per-lane LDS addresses each tile instead of holding them all live.
            int lane_v = lane;
            asm volatile("" : "+v"(lane_v));
            const Roles<D> ro(lane_v);
            const int32_t tile = wave + kWaves * e;
            const int32_t nvalid = min(kTile, T.end - (T.start + tile * kTile));
            tile_stage<D>(wt, kr, vr, lane_v, nvalid);
            if (e + 1 < n0) tile_issue<CSR, D>(T, tile + kWaves, idx_next, pm, lane, kr, vr);
            if (e + 2 < n0)
                idx_next = tile_index<CSR, D>(a, T, T.start + (tile + 2 * kWaves) * kTile, lane, pm);
            wave_sync();
            tile_compute<DT, D>(wt, sh.q, nvalid, scale2, ro, m_l, den_l, acc);
        }

        // ---- end of the wave's tiles.  The last wave has the fewest tiles (round-robin
        // deal): with none of its loads in flight, it finds the worker's next task now;
        // the merge barrier below publishes it to for_each_task and to the next task's
        // first tile issue.
        if (wave == kWaves - 1)
            prefetch_next<CSR, kTile * kWaves>(a, succ, sh.pf_idx, lane, pm, sh.indptr, iptr_n);
        // ---- reduce within the wave, then merge the waves
        const Roles<D> ro(lane);
        float mh[kHeads], dh[kHeads];
        wave_state<D>(m_l, den_l, acc, mh, dh);
        float *comb = reinterpret_cast<float *>(&wt.k[0][0]);  // [head][D] fp32, reuses this wave's K tile
        static_assert(sizeof(float) * kHeads * D <= sizeof(wt.k), "the combine rows fit the K tile");
        if (lane < Geo<D>::kPvLanes) {
#pragma unroll
            for (int h = 0; h < kHeads; ++h)
                *reinterpret_cast<float4 *>(&comb[h * D + ro.pd * 4]) =
                    make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        }
        float mv = mh[0], dv = dh[0];
#pragma unroll
        for (int h = 1; h < kHeads; ++h)
            if (lane == h) {
                mv = mh[h];
                dv = dh[h];
            }
        if (lane < kHeads) {
            sh.cm[wave][lane] = mv;
            sh.cd[wave][lane] = dv;
        }
        lds_barrier();
        // one (head, dim) output per thread and round: 4 heads x D dims
#pragma unroll
        for (int o = threadIdx.x; o < kHeads * D; o += 64 * kWaves) {
            const int h = o / D, d = o % D;
            if (h < G) {
                float mm = -INFINITY;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sh.cm[w][h]);
                float dd = 0.f, x = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float sc = __builtin_amdgcn_exp2f(sh.cm[w][h] - mm);
                    dd += sh.cd[w][h] * sc;
                    x += reinterpret_cast<const float *>(&sh.w[w].k[0][0])[h * D + d] * sc;
                }
                const int64_t slot = ((int64_t)T.request * a.query_heads + group * G + h) * a.max_splits + split;
                a.partial[slot * D + d] = x / dd;
                if (d == 0) a.lse[slot] = (mm + __log2f(dd)) * kLn2;
                if (first)
                    static_cast<uint16_t *>(a.out)[((int64_t)T.request * a.query_heads + group * G + h) * D + d] =
                        (uint16_t)from_f32<DT>(x / dd);
            }
        }
    }, sh.pf);
}

template <int DT, bool CSR, int kWaves, int D, bool kOut, bool kPow2>
int launch_valu_o(const sgd_decode_args &a, hipStream_t stream) {
    static bool attr[kOnceDevices] = {};
    const int bytes = (int)sizeof(ValuShared<kWaves, D>);
    if (int rc = set_dynamic_lds((const void *)k_attention_valu<DT, CSR, kWaves, D, kOut, kPow2>, bytes, attr,
                                 "valu attention"))
        return rc;
    hipLaunchKernelGGL((k_attention_valu<DT, CSR, kWaves, D, kOut, kPow2>), dim3(a.workers), dim3(64 * kWaves), bytes,
                       stream, a);
    return launch_status("persistent_decode(valu)");
}

// A power-of-two page (CSR's page of one token included) maps tokens by shift and mask;
// any other page size by division, in a separate build.
template <int DT, bool CSR, int kWaves, int D, bool kOut>
int launch_valu_p(const sgd_decode_args &a, hipStream_t stream) {
    if constexpr (CSR) return launch_valu_o<DT, CSR, kWaves, D, kOut, true>(a, stream);
    else
        return (a.page_size & (a.page_size - 1)) == 0 ? launch_valu_o<DT, CSR, kWaves, D, kOut, true>(a, stream)
                                                      : launch_valu_o<DT, CSR, kWaves, D, kOut, false>(a, stream);
}

template <int DT, bool CSR, int kWaves, int D>
int launch_valu_w(const sgd_decode_args &a, hipStream_t stream) {
    return a.out ? launch_valu_p<DT, CSR, kWaves, D, true>(a, stream) : launch_valu_p<DT, CSR, kWaves, D, false>(a, stream);
}

// 8-wave workgroups, two per CU at the default worker count (one 16-wave workgroup per CU
// measured slower: its task-end barrier idles 16 waves).
template <int DT, bool CSR>
int launch_valu_t(const sgd_decode_args &a, hipStream_t stream) {
    switch (a.head_dim) {
        case 64: return launch_valu_w<DT, CSR, 8, 64>(a, stream);
        case 256: return launch_valu_w<DT, CSR, 8, 256>(a, stream);
        default: return launch_valu_w<DT, CSR, 8, 128>(a, stream);
    }
}

}  // namespace

bool valu_supported(const sgd_decode_args &a) {
    const int g = a.query_heads / a.kv_heads;
    if (g > kHeads || (a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256)) return false;
    if (a.k_stride[3] != 1 || a.v_stride[3] != 1) return false;
    if ((reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v)) & 15) return false;
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
