// Persistent paged GQA decode attention for query-head groups of 8 or 16 heads
// (Llama-3-70B: 64 q / 8 kv), head_dim 64, 128 or 256, unit dim stride -- the MFMA path.
//
// With 8-16 query heads per KV head, QK^T and P.V are real (if small) matrix
// products, so both run on the matrix cores with v_mfma_f32_16x16x32_{bf16,f16}
// (fp32 accumulate); the online softmax stays in fp32 on the VALU.  Lane l of a
// wave is (m, j) = (l % 16, l / 16).  Operand layouts of the 16x16x32 MFMA:
// A[m][8j .. 8j+7], B[8j .. 8j+7][n = l % 16], D[4j + i][n = l % 16].
//
// A 32-token tile of one (record, kv head) per wave, two halves of 16 tokens:
//   S^T = K . Q^T   (M = 16 tokens of a half, N = 16 padded heads, K = 128 dims in
//                    four 32-dim chunks): lane (m, j) loads the 16 bytes of token m's
//                    K row at dims 32c + 8j .. +7 straight into the A operand; the
//                    group's q rows are the B operand, held in registers per task.
//                    Output: lane (n, j) has S[head n][token 16h + 4j + i].
//   softmax        per head n, over the 8 scores of each lane and the 4 lanes
//                    (j = 0..3) of the head's column; P rounded to the KV dtype
//                    (kernels/attention.py:78).
//   O^T += V^T . P^T (M = 16, N = heads, K = 32 tokens): the B operand is P
//                    exactly as S^T left it (k slot s of lane group j = token
//                    4j + s for s < 4, 16 + 4j + s - 4 otherwise), so P never
//                    moves.  The A operand needs, per lane, one dim of those 8
//                    tokens: lane (m, j) loads the 16 bytes at dims 8m .. 8m+7 of
//                    each of the 8 tokens (16 lanes cover a 256 B V row), and MFMA
//                    block b (0..7) takes element b of each -- output row r of
//                    block b is dim 8r + b.  No LDS transpose, just v_perm_b32.
// Output: lane (n, j) accumulates head n, dims 32j .. 32j+31.
//
// Other head dims (MGeo): D = 64 keeps the 32-token tile with two 32-dim QK chunks; a
// 64-dim V row is 8 lanes of 16 B, so lanes m and m + 8 load the same chunk and output
// rows 8..15 of each block are copies that are not stored.  D = 256 holds a double-buffered
// 32-token tile in no register budget, so it takes 16-token tiles: S^T over eight 32-dim
// chunks, and O^T += V^T . P^T on v_mfma_f32_16x16x16 (K = the tile's 16 tokens), whose B
// operand is the S^T output as it stands (k slot i of lane group j = token 4j + i); lane
// (m, j) loads dims 8m .. 8m+7 and 128 + 8m .. of its 4 tokens, 16 output blocks.
//
// Worker = one workgroup of 4 waves (two per CU); tiles of a task are dealt to the
// waves round-robin, each wave double-buffers its next tile's K/V loads in
// registers, and at the end of the task the waves' (m, den, O) are merged through
// LDS into the partial rows and natural-log LSEs of slot (request, head, split)
// (kernels/attention.py:81-84).  Tasks and their order come from
// attention_common.h's dispatch; the last wave, once its tiles are done, claims and
// looks up the worker's next task and the page/slot indices of its first tiles.
#include "valu_ops.h"

namespace sgd {
namespace {

using valu::uni;

constexpr int kWaves = 4;
constexpr int kHeadsM = 16;    // MFMA N: query heads, padded

template <int D>
struct MGeo {
    static_assert(D == 64 || D == 128 || D == 256, "head_dim 64, 128 or 256");
    static constexpr int kTileT = D == 256 ? 16 : 32;  // tokens per tile
    static constexpr int kHalves = kTileT / 16;        // 16-token S^T blocks
    static constexpr int kChunks = D / 32;             // QK contraction chunks of 32 dims
    static constexpr int kVals = kTileT / 4;           // scores / P values per lane and tile
    static constexpr int kBlocks = D == 256 ? 16 : 8;  // O^T blocks (f32x4 each)
};
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A head's row of a wave's output is padded by 4 floats: in the 16-byte stores of the
// end-of-task merge the 16 heads of a lane group then start 4 banks apart instead of
// all on the same bank (a 128-float stride is a multiple of the bank count).
constexpr int kOPad = 4;

template <int D>
struct MfmaShared {
    float o[kWaves][kHeadsM][D + kOPad];  // per-wave unnormalized outputs (33 KB at D = 128)
    float m[kWaves][kHeadsM];
    float d[kWaves][kHeadsM];
    int32_t cursor;
    Prefetched pf[2];                                // the worker's next task (prefetch_next)
    int32_t pf_idx[2][MGeo<D>::kTileT * kWaves];  // page/slot indices of its first kWaves tiles
};

template <int DT>
__device__ __forceinline__ f32x4 mfma(uint4 a, uint4 b, f32x4 c) {
    if constexpr (DT == SGD_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16(uint2 a, uint2 b, f32x4 c) {
    if constexpr (DT == SGD_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b),
                                                          c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                      0, 0);
}

// Token (within the tile) of k slot s for lane group j (the P / V^T order): 32-token
// tiles 4j + s (s < 4) or 16 + 4j + s - 4; 16-token tiles 4j + s.
__device__ __forceinline__ int slot_token(int j, int s) { return s < 4 ? 4 * j + s : 16 + 4 * j + (s - 4); }

template <int D>
struct TileRegs {
    static constexpr int kVS = MGeo<D>::kVals;
    uint4 k[MGeo<D>::kHalves][MGeo<D>::kChunks];  // [half][dim chunk]: token 16h + m, dims 32c + 8j .. +7
    uint4 v[D == 256 ? 2 : 1][kVS];  // [128-dim half][k slot]: token slot_token(j, s), dims 8m .. 8m+7
};

struct Src {
    const char *kbase, *vbase;
    int64_t kp, kt, vp, vt;
    int32_t request, ind0, start, end;
};

// lane l < kTileT fetches the physical page / slot index of token tok0 + l (0 past `end`,
// which addresses an in-bounds row).
template <bool CSR, int D, bool kPow2>
__device__ __forceinline__ int32_t tile_index(const sgd_decode_args &a, const Src &t, const PageMap<kPow2> &pm,
                                              int32_t tok0, int lane) {
    const int32_t tok = tok0 + lane;
    int32_t v = 0;
    if (lane < MGeo<D>::kTileT && tok < t.end) {
        if constexpr (CSR) v = a.pages[t.ind0 + tok];
        else v = a.pages[(int64_t)t.request * a.pt_stride[0] + (int64_t)pm.page(tok) * a.pt_stride[1]];
    }
    return v;
}

// All 16 loads are unconditional, so nothing branches between a tile's loads and
// the compute that overlaps them.
template <bool CSR, int D, bool kPow2>
__device__ __forceinline__ void tile_issue_k(const Src &t, const PageMap<kPow2> &pm, int32_t tok0, int32_t idxv,
                                             int lane, TileRegs<D> &r) {
    using G = MGeo<D>;
    const int m = lane & 15, j = lane >> 4;
#pragma unroll
    for (int h = 0; h < G::kHalves; ++h) {
        const int tt = 16 * h + m;
        const uint32_t phys = (uint32_t)__shfl(idxv, tt, 64);
        int64_t off = (int64_t)phys * t.kp;
        if constexpr (!CSR) off += (int64_t)pm.row(tok0 + tt) * t.kt;
#pragma unroll
        for (int c = 0; c < G::kChunks; ++c)
            r.k[h][c] = load_stream16(t.kbase + off + (32 * c + 8 * j) * 2);
    }
}

template <bool CSR, int D, bool kPow2>
__device__ __forceinline__ void tile_issue_v(const Src &t, const PageMap<kPow2> &pm, int32_t tok0, int32_t idxv,
                                             int lane, TileRegs<D> &r) {
    using G = MGeo<D>;
    const int m = lane & 15, j = lane >> 4;
    // V: dims 8m .. 8m+7 (D = 64: 8 (m % 8) ..; D = 256: also 128 + 8m ..) of the slot tokens
    const int vm = D == 64 ? (m & 7) : m;
#pragma unroll
    for (int s = 0; s < G::kVals; ++s) {
        const int tt = slot_token(j, s);
        const uint32_t phys = (uint32_t)__shfl(idxv, tt, 64);
        int64_t off = (int64_t)phys * t.vp + vm * 16;
        if constexpr (!CSR) off += (int64_t)pm.row(tok0 + tt) * t.vt;
#pragma unroll
        for (int hv = 0; hv < (D == 256 ? 2 : 1); ++hv) r.v[hv][s] = load_stream16(t.vbase + off + hv * 256);
    }
}

template <bool CSR, int D, bool kPow2>
__device__ __forceinline__ void tile_issue(const Src &t, const PageMap<kPow2> &pm, int32_t tok0, int32_t idxv, int lane,
                                           TileRegs<D> &r) {
    tile_issue_k<CSR, D>(t, pm, tok0, idxv, lane, r);
    tile_issue_v<CSR, D>(t, pm, tok0, idxv, lane, r);
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return valu::pack2<DT>(lo, hi); }

// One tile: S^T, online softmax (exp2 domain), O^T += V^T P^T.  m_l / den_l are this
// lane's head's running max and partial denominator (its own 8 tokens per tile).
template <int DT, int D>
__device__ __forceinline__ void tile_compute(TileRegs<D> &r, const uint4 (&q)[MGeo<D>::kChunks], int32_t nvalid,
                                             float scale2, int lane, float &m_l, float &den_l,
                                             f32x4 (&o)[MGeo<D>::kBlocks]) {
    using G = MGeo<D>;
    constexpr int kV = G::kVals;
    const int j = lane >> 4;
    f32x4 s[G::kHalves];
#pragma unroll
    for (int h = 0; h < G::kHalves; ++h) {
        s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < G::kChunks; ++c) s[h] = mfma<DT>(r.k[h][c], q[c], s[h]);
    }
    float x[kV];
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        const int tt = slot_token(j, i);  // s[i / 4][i % 4] is token 16 (i / 4) + 4j + i % 4
        x[i] = tt < nvalid ? s[i >> 2][i & 3] * scale2 : -INFINITY;
    }
    if (nvalid < G::kTileT) {  // rows past the task's end: zero V (their p is exactly zero)
#pragma unroll
        for (int i = 0; i < kV; ++i)
            if (slot_token(j, i) >= nvalid)
#pragma unroll
                for (int hv = 0; hv < (D == 256 ? 2 : 1); ++hv) r.v[hv][i] = make_uint4(0, 0, 0, 0);
    }
    float mx = x[0];
#pragma unroll
    for (int i = 1; i < kV; ++i) mx = fmaxf(mx, x[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_l, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_l - m_new);
    m_l = m_new;
    float p[kV], ps = 0.f;
#pragma unroll
    for (int i = 0; i < kV; ++i) {
        p[i] = __builtin_amdgcn_exp2f(x[i] - m_new);
        ps += p[i];
    }
    den_l = den_l * alpha + ps;
    if constexpr (D != 256) {
        const uint4 pb = make_uint4(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]), pack2<DT>(p[4], p[5]),
                                    pack2<DT>(p[6], p[7]));
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            // A operand of block b: element b (dim 8m + b) of the 8 slot tokens' V chunks
            const int dw = b >> 1;
            const uint32_t sel = (b & 1) ? 0x07060302u : 0x05040100u;
            auto e = [&](int s) { return (&r.v[0][s].x)[dw]; };
            const uint4 av = make_uint4(__builtin_amdgcn_perm(e(1), e(0), sel), __builtin_amdgcn_perm(e(3), e(2), sel),
                                        __builtin_amdgcn_perm(e(5), e(4), sel), __builtin_amdgcn_perm(e(7), e(6), sel));
            o[b] = o[b] * alpha;
            o[b] = mfma<DT>(av, pb, o[b]);
        }
    } else {
        // 16x16x16 over the tile's 16 tokens: B = P as S^T left it (4 tokens per lane group)
        const uint2 pb = make_uint2(pack2<DT>(p[0], p[1]), pack2<DT>(p[2], p[3]));
#pragma unroll
        for (int hv = 0; hv < 2; ++hv)
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                // A operand of block 8 hv + b: element b (dim 128 hv + 8m + b) of the 4 tokens' chunks
                const int dw = b >> 1;
                const uint32_t sel = (b & 1) ? 0x07060302u : 0x05040100u;
                auto e = [&](int s) { return (&r.v[hv][s].x)[dw]; };
                const uint2 av = make_uint2(__builtin_amdgcn_perm(e(1), e(0), sel), __builtin_amdgcn_perm(e(3), e(2), sel));
                o[8 * hv + b] = o[8 * hv + b] * alpha;
                o[8 * hv + b] = mfma16<DT>(av, pb, o[8 * hv + b]);
            }
    }
}

template <int DT, bool CSR, int D, bool kOut, bool kPow2>
__global__ __launch_bounds__(64 * kWaves, 2) void k_attention_mfma(sgd_decode_args a) {
    using MG = MGeo<D>;
    constexpr int kTileT = MG::kTileT;
    extern __shared__ __align__(16) char dyn_smem[];
    MfmaShared<D> &sh = *reinterpret_cast<MfmaShared<D> *>(dyn_smem);
    const int lane0 = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
    const int32_t G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    const PageMap<kPow2> pm(a.page_size);
    clear_prefetched(sh.pf);
    lds_barrier();

    for_each_task<true>(a, &sh.cursor, [&](int32_t task, const TaskInfo &ti, const Successor &succ) {
        // A laundered lane id per task: the compiler rebuilds the per-lane offsets
        // each task instead of holding them (64-bit each) live across the task loop.
        int lane = lane0;
        asm volatile("" : "+v"(lane));
        Src t;
        t.request = uni(ti.request);
        t.start = uni(ti.start);
        t.end = uni(ti.end);
        const int32_t split = uni(ti.split), group = uni(ti.group);
        // kOut (sgd_decode_args.out set, a separate build): a request's first split also
        // writes its rows to `out` (final for a single-split request, overwritten by the
        // merge otherwise)
        const bool first = kOut && split == 0;
        t.ind0 = CSR ? uni(a.indptr[t.request]) : 0;
        t.kbase = static_cast<const char *>(a.k) + group * (a.k_stride[2] * 2);
        t.vbase = static_cast<const char *>(a.v) + group * (a.v_stride[2] * 2);
        t.kp = a.k_stride[0] * 2;
        t.kt = a.k_stride[1] * 2;
        t.vp = a.v_stride[0] * 2;
        t.vt = a.v_stride[1] * 2;
        const int32_t ntiles = (t.end - t.start + kTileT - 1) / kTileT;
        const int32_t n0 = ntiles > wave ? (ntiles - wave + kWaves - 1) / kWaves : 0;
        const bool prefetched = uni(sh.pf[succ.cur].task) == task;

        // q rows as the B operand: head n = lane % 16, dims 32c + 8j .. +7 (zero past G)
        uint4 q[MG::kChunks];
        {
            const int n = lane & 15, j = lane >> 4;
            const int64_t qd = a.q_stride[2];
            const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (int64_t)t.request * a.q_stride[0] +
                                 (int64_t)(group * G + n) * a.q_stride[1];
#pragma unroll
            for (int c = 0; c < MG::kChunks; ++c) {
                q[c] = make_uint4(0, 0, 0, 0);
                if (n < G) {
                    const uint16_t *p = qp + (int64_t)(32 * c + 8 * j) * qd;
                    if (qd == 1 && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
                        q[c] = *reinterpret_cast<const uint4 *>(p);
                    } else {
                        uint32_t w4[4] = {0, 0, 0, 0};
#pragma unroll
                        for (int e = 0; e < 8; ++e) w4[e >> 1] |= (uint32_t)p[e * qd] << (16 * (e & 1));
                        q[c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
                    }
                }
            }
        }

        float m_l = -INFINITY, den_l = 0.f;
        f32x4 o[MG::kBlocks];
#pragma unroll
        for (int b = 0; b < MG::kBlocks; ++b) o[b] = f32x4{0.f, 0.f, 0.f, 0.f};

        TileRegs<D> cur, nxt;
        int32_t tile = wave, idx_next = 0;
        if (n0 > 0) {
            const int32_t idx0 = !prefetched              ? tile_index<CSR, D>(a, t, pm, t.start + tile * kTileT, lane)
                                 : lane < kTileT ? sh.pf_idx[succ.cur][wave * kTileT + lane]
                                                 : 0;
            tile_issue<CSR, D>(t, pm, t.start + tile * kTileT, idx0, lane, cur);
            // indices of the wave's next tile (clamped to its last one)
            idx_next = tile_index<CSR, D>(a, t, pm, t.start + min(tile + kWaves, ntiles - 1) * kTileT, lane);
        }
        if (n0 > 0) {
            if constexpr (D == 256) {
                // Only K is double-buffered (a second 16 KB tile beside q and 16 output blocks
                // exceeds 256 VGPRs): the next tile's V goes into this tile's V registers once
                // its P.V is issued.
                for (int32_t e = 0;; ++e) {
                    const bool more = e + 1 < n0;
                    const int32_t nt = tile + kWaves, idx_nt = idx_next;
                    if (more) {
                        tile_issue_k<CSR, D>(t, pm, t.start + nt * kTileT, idx_nt, lane, nxt);
                        idx_next = tile_index<CSR, D>(a, t, pm, t.start + min(nt + kWaves, ntiles - 1) * kTileT, lane);
                    }
                    tile_compute<DT, D>(cur, q, min(kTileT, t.end - (t.start + tile * kTileT)), scale2, lane,
                                        m_l, den_l, o);
                    if (!more) break;
                    tile_issue_v<CSR, D>(t, pm, t.start + nt * kTileT, idx_nt, lane, cur);
#pragma unroll
                    for (int c = 0; c < MG::kChunks; ++c) cur.k[0][c] = nxt.k[0][c];
                    tile = nt;
                }
            } else {
                for (int32_t e = 0; e + 1 < n0; ++e) {
                    const int32_t nt = tile + kWaves;
                    tile_issue<CSR, D>(t, pm, t.start + nt * kTileT, idx_next, lane, nxt);
                    idx_next = tile_index<CSR, D>(a, t, pm, t.start + min(nt + kWaves, ntiles - 1) * kTileT, lane);
                    tile_compute<DT, D>(cur, q, min(kTileT, t.end - (t.start + tile * kTileT)), scale2, lane,
                                        m_l, den_l, o);
                    cur = nxt;
                    tile = nt;
                }
                tile_compute<DT, D>(cur, q, min(kTileT, t.end - (t.start + tile * kTileT)), scale2, lane, m_l,
                                    den_l, o);
            }
        }

        // The last wave holds the fewest tiles (round-robin deal): once they are done it
        // finds the worker's next task, so those round trips overlap the other waves'
        // last tiles; the barrier below publishes it.
        if (wave == kWaves - 1) prefetch_next<CSR, kTileT * kWaves>(a, succ, sh.pf_idx, lane, pm, nullptr, 0);

        // wave state to LDS: head n = lane % 16, dims 128 hv + 32j + 8i + b (D = 64: lane
        // groups j < 2 only; the others hold copies)
        den_l += __shfl_xor(den_l, 16, 64);
        den_l += __shfl_xor(den_l, 32, 64);
        lds_barrier();  // the previous task's combine is done reading shared memory
        {
            const int n = lane & 15, j = lane >> 4;
            if (D != 64 || j < 2) {
#pragma unroll
                for (int hv = 0; hv < MG::kBlocks / 8; ++hv)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const f32x4 *ob = o + 8 * hv;
                        float *dst = &sh.o[wave][n][128 * hv + 32 * j + 8 * i];
                        *reinterpret_cast<float4 *>(dst) = make_float4(ob[0][i], ob[1][i], ob[2][i], ob[3][i]);
                        *reinterpret_cast<float4 *>(dst + 4) = make_float4(ob[4][i], ob[5][i], ob[6][i], ob[7][i]);
                    }
            }
            if (j == 0) {
                sh.m[wave][n] = m_l;
                sh.d[wave][n] = den_l;
            }
        }
        lds_barrier();
        for (int x = threadIdx.x; x < G * D; x += 64 * kWaves) {
            const int h = x / D, d = x % D;
            float mm = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sh.m[w][h]);
            float dd = 0.f, acc = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float sc = __builtin_amdgcn_exp2f(sh.m[w][h] - mm);
                dd += sh.d[w][h] * sc;
                acc += sh.o[w][h][d] * sc;
            }
            const int64_t slot = ((int64_t)t.request * a.query_heads + group * G + h) * a.max_splits + split;
            a.partial[slot * D + d] = acc / dd;
            if (d == 0) a.lse[slot] = (mm + __log2f(dd)) * kLn2;
            if (first)
                static_cast<uint16_t *>(a.out)[((int64_t)t.request * a.query_heads + group * G + h) * D + d] =
                    (uint16_t)from_f32<DT>(acc / dd);
        }
    }, sh.pf);
}

template <int DT, bool CSR, int D, bool kOut, bool kPow2>
int launch_mfma_o(const sgd_decode_args &a, hipStream_t stream) {
    static bool attr[kOnceDevices] = {};
    constexpr int bytes = (int)sizeof(MfmaShared<D>);
    if (int rc = set_dynamic_lds((const void *)k_attention_mfma<DT, CSR, D, kOut, kPow2>, bytes, attr,
                                 "mfma attention"))
        return rc;
    hipLaunchKernelGGL((k_attention_mfma<DT, CSR, D, kOut, kPow2>), dim3(a.workers), dim3(64 * kWaves), bytes, stream,
                       a);
    return launch_status("persistent_decode(mfma)");
}

// A power-of-two page (CSR's page of one token included) maps tokens by shift and mask;
// any other page size by division, in a separate build.
template <int DT, bool CSR, int D, bool kOut>
int launch_mfma_p(const sgd_decode_args &a, hipStream_t stream) {
    if constexpr (CSR) return launch_mfma_o<DT, CSR, D, kOut, true>(a, stream);
    else
        return (a.page_size & (a.page_size - 1)) == 0 ? launch_mfma_o<DT, CSR, D, kOut, true>(a, stream)
                                                      : launch_mfma_o<DT, CSR, D, kOut, false>(a, stream);
}

template <int DT, bool CSR, int D>
int launch_mfma_d(const sgd_decode_args &a, hipStream_t stream) {
    return a.out ? launch_mfma_p<DT, CSR, D, true>(a, stream) : launch_mfma_p<DT, CSR, D, false>(a, stream);
}

template <int DT, bool CSR>
int launch_mfma_t(const sgd_decode_args &a, hipStream_t stream) {
    switch (a.head_dim) {
        case 64: return launch_mfma_d<DT, CSR, 64>(a, stream);
        case 256: return launch_mfma_d<DT, CSR, 256>(a, stream);
        default: return launch_mfma_d<DT, CSR, 128>(a, stream);
    }
}

}  // namespace

// Any group up to 16 (the padded MFMA N), head_dim 64, 128 or 256, unit dim stride,
// 16-byte aligned rows, any page size.
bool mfma_supported(const sgd_decode_args &a) {
    const int g = a.query_heads / a.kv_heads;
    if (g < 1 || g > kHeadsM || (a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256)) return false;
    if (a.k_stride[3] != 1 || a.v_stride[3] != 1) return false;
    if ((reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.v)) & 15) return false;
    for (int i = 0; i < 3; ++i)
        if (a.k_stride[i] % 8 || a.v_stride[i] % 8) return false;
    return a.k_stride[0] < (1ll << 40) && a.v_stride[0] < (1ll << 40);
}

int launch_attention_mfma(const sgd_decode_args &a, hipStream_t stream) {
    if (a.dtype == SGD_BF16)
        return a.csr ? launch_mfma_t<SGD_BF16, true>(a, stream) : launch_mfma_t<SGD_BF16, false>(a, stream);
    return a.csr ? launch_mfma_t<SGD_FP16, true>(a, stream) : launch_mfma_t<SGD_FP16, false>(a, stream);
}

}  // namespace sgd
