// Wave64 building blocks shared by the VALU decode-attention kernels: packed
// 16-bit dot products, DPP cross-lane moves, the paged/CSR row gather of one tile,
// and the tile's QK^T / online-softmax / P.V math, for head_dim D in {64, 128, 256}.
//
// A tile is 4 KB of K and 4 KB of V whatever D is: Geo<D>::kTile = 2048 / D tokens
// (32, 16, 8), gathered by 4 + 4 16-byte loads per lane.  The lane roles keep the same
// register shape for every D: QK takes 8 lanes per token (D / 64 chunks of 16 B per lane,
// kTile / 8 passes), P.V gives each lane 4 dims of the output and deals the tile's token
// pairs over 256 / D lane groups, so a tile is always 4 P.V steps and the accumulators
// are 4 heads x 4 dims.
#pragma once

#include "attention_common.h"

namespace sgd {
namespace valu {

constexpr int kHeads = 4;                 // padded query-head group
constexpr int kRowsLoads = 4;             // 16-byte loads per lane for a K (and a V) tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int D>
struct Geo {
    static_assert(D == 64 || D == 128 || D == 256, "head_dim 64, 128 or 256");
    static constexpr int kTile = 2048 / D;        // tokens per tile
    static constexpr int kChunks = D / 8;         // 16 B chunks per K/V row (= lanes per row in a load)
    static constexpr int kRowsPerLoad = 64 / kChunks;
    static constexpr int kPasses = kTile / 8;     // QK passes of 8 tokens x 8 lanes
    static constexpr int kLaneChunks = D / 64;    // QK: 16 B chunks per lane and token (qj + 8c)
    static constexpr int kPvLanes = D / 4;        // P.V: lanes per group (4 dims each)
    static constexpr int kPvGroups = 64 / kPvLanes;
    static constexpr int kPvSteps = kTile / 2 / kPvGroups;
    static_assert(kPvSteps == 4 && kTile * D * 2 == 64 * 16 * kRowsLoads, "a tile is 4 KB of K and of V");
};

// One wave's staging area: the K and V rows of a tile and the tile's probabilities as
// token pairs.  For D >= 128, K rows of odd tokens hold their 16 B chunks at c ^ 8
// (k_chunk): the QK reads take 8 lanes per token row, and the 16 lanes the LDS serves
// per cycle then cover all 64 banks instead of the same 32 twice (two rows a multiple
// of 256 B apart).  D = 64 rows are 128 B, so two neighbouring rows already fill the 64
// banks.  V rows are plain: a P.V read covers 256 B per 32 lanes.
template <int D>
struct WaveTile {
    uint4 k[Geo<D>::kTile][D / 8];   // 4 KB
    uint4 v[Geo<D>::kTile][D / 8];   // 4 KB
    uint4 p[Geo<D>::kTile / 2];      // [pair] -> 4 heads x (p[2i], p[2i+1]) in the KV dtype
};

// Position of 16 B chunk c of K row `row` in WaveTile<D>::k.
template <int D>
__device__ __forceinline__ constexpr int k_chunk(int row, int c) {
    return D >= 128 ? c ^ ((row & 1) << 3) : c;
}

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
__device__ __forceinline__ float uni_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}
__device__ __forceinline__ float lane_f(float x, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor3 = 0x1B;       // quad_perm [3,2,1,0]
constexpr int kRowShl8 = 0x108;       // row_shl:8
constexpr int kRowRor8 = 0x128;       // row_ror:8
constexpr int kRowHalfMirror = 0x141; // row_half_mirror
constexpr int kRowNewBcast = 0x150;   // row_newbcast:n

// The lane that holds head h after the QK reduce-scatter (lanes 0, 2, 4, 6).
__device__ __forceinline__ constexpr int head_lane(int h) { return ((h >> 1) << 2) | ((h & 1) << 1); }

// Lane roles.  QK: 8 lanes per token; qg = lane / 8 picks the token, qj = lane % 8
// owns the 16 B chunks qj + 8c (c < D / 64); after the reduce-scatter the lane holds
// head hs = 2*bit2(qj) + bit1(qj).  P.V: group pg = lane / (D / 4) takes token pairs
// kPvGroups * s + pg; pd = lane % (D / 4) owns dims 4*pd .. 4*pd+3.
template <int D>
struct Roles {
    int qg, qj, hs, pg, pd;
    bool b2, b1;
    __device__ __forceinline__ explicit Roles(int l) {
        qg = l >> 3;
        qj = l & 7;
        hs = ((qj >> 2) << 1) | ((qj >> 1) & 1);
        b2 = (qj & 4) != 0;
        b1 = (qj & 2) != 0;
        pg = l / Geo<D>::kPvLanes;
        pd = l % Geo<D>::kPvLanes;
    }
};

// Where a tile's rows come from.
struct TileSrc {
    const char *kbase, *vbase;  // K/V + group * head stride (bytes)
    int64_t kp, kt, vp, vt;     // page and in-page strides (bytes)
    int32_t request, ind0, start, end;
};

// Token row (within the tile) of this lane's 16-byte load `i`.
template <int D>
__device__ __forceinline__ constexpr int load_row(int i, int lane) {
    return i * Geo<D>::kRowsPerLoad + lane / Geo<D>::kChunks;
}

// The tile row whose page/slot index lane 16r + j holds for tile_issue (-1: none).  A
// load's rows start on DPP rows of 16 lanes: for D >= 128 each DPP row reads one token
// row, whose index lane 16r + i sits in for load i < 4; for D = 64 a DPP row reads two
// token rows, the first's index in lane 16r + i, the second's in lane 16r + 8 + i.
template <int D>
__device__ __forceinline__ int index_row(int lane) {
    const int r = lane >> 4, j = lane & 15, i = j & 7;
    if (i >= kRowsLoads || (D >= 128 && j >= 8)) return -1;
    return load_row<D>(i, 16 * r + (j & 8));
}

// Lane 16r + j fetches the page/slot index of token tok0 + index_row(lane) (0 if none).
template <bool CSR, int D, bool kPow2>
__device__ __forceinline__ int32_t tile_index(const sgd_decode_args &a, const TileSrc &t, int32_t tok0, int lane,
                                              const PageMap<kPow2> &pm) {
    const int row = index_row<D>(lane);
    const int32_t tok = tok0 + row;
    int32_t v = 0;
    if (row >= 0 && tok < t.end) {
        if constexpr (CSR) v = a.pages[t.ind0 + tok];
        else v = a.pages[(int64_t)t.request * a.pt_stride[0] + (int64_t)pm.page(tok) * a.pt_stride[1]];
    }
    return v;
}

// 4 x 16-byte loads for K and for V, each covering 1 KB of token rows (D / 8 lanes per
// row); DPP row_newbcast hands each row its token's index (for D = 64 two broadcasts
// and a select, one per half of the DPP row).  The loads are unconditional, so no
// exec-mask branch sits between a tile's loads and the compute they overlap: rows past
// `end` got index 0 from tile_index, which addresses a row of page 0 (in bounds), and
// tile_stage zeroes them.
template <bool CSR, int D, bool kPow2>
__device__ __forceinline__ void tile_issue(const TileSrc &t, int32_t tile, int32_t idxv, const PageMap<kPow2> &pm,
                                           int lane, uint4 (&kr)[kRowsLoads], uint4 (&vr)[kRowsLoads]) {
    const int c = lane % Geo<D>::kChunks;
    const int32_t tok0 = t.start + tile * Geo<D>::kTile;
#define SGD_LOAD_ROW(I)                                                                              \
    {                                                                                                \
        uint32_t phys = (uint32_t)dpp_i<kRowNewBcast + I>(idxv);                                     \
        if constexpr (D == 64) {                                                                     \
            const uint32_t hi = (uint32_t)dpp_i<kRowNewBcast + 8 + I>(idxv);                         \
            phys = (lane & 8) ? hi : phys;                                                           \
        }                                                                                            \
        int64_t ko = (int64_t)phys * t.kp + c * 16, vo = (int64_t)phys * t.vp + c * 16;              \
        if constexpr (!CSR) {                                                                        \
            const int32_t inner = pm.row(tok0 + load_row<D>(I, lane));                               \
            ko += (int64_t)inner * t.kt;                                                             \
            vo += (int64_t)inner * t.vt;                                                             \
        }                                                                                            \
        kr[I] = load_stream16(t.kbase + ko);                                                           \
        vr[I] = load_stream16(t.vbase + vo);                                                           \
    }
    static_assert(kRowsLoads == 4, "one SGD_LOAD_ROW per 1 KB load");
    SGD_LOAD_ROW(0) SGD_LOAD_ROW(1) SGD_LOAD_ROW(2) SGD_LOAD_ROW(3)
#undef SGD_LOAD_ROW
}

// Writes the tile's rows to the wave's LDS tile.  In a partial tile (nvalid < kTile,
// uniform) the rows past the task's end are zero: their probabilities are exactly
// zero, and zero V keeps P.V finite whatever page 0 holds.
template <int D>
__device__ __forceinline__ void tile_stage(WaveTile<D> &wt, uint4 (&kr)[kRowsLoads], uint4 (&vr)[kRowsLoads],
                                           int lane, int32_t nvalid) {
    const int c = lane % Geo<D>::kChunks;
    if (nvalid < Geo<D>::kTile) {
#pragma unroll
        for (int i = 0; i < kRowsLoads; ++i)
            if (load_row<D>(i, lane) >= nvalid) {
                kr[i] = make_uint4(0, 0, 0, 0);
                vr[i] = make_uint4(0, 0, 0, 0);
            }
    }
#pragma unroll
    for (int i = 0; i < kRowsLoads; ++i) {
        const int row = load_row<D>(i, lane);
        wt.k[row][k_chunk<D>(row, c)] = kr[i];
        wt.v[row][c] = vr[i];
    }
}

// One staged tile: QK^T against the group's q rows `qs` (LDS), online softmax in
// the exp2 domain, P.V into acc.  m_l/den_l are this lane's head's running max and
// denominator (QK roles); acc holds 4 heads x 4 dims (P.V roles).
template <int DT, int D>
__device__ __forceinline__ void tile_compute(WaveTile<D> &wt, const uint4 (*qs)[D / 8], int32_t nvalid, float scale2,
                                             const Roles<D> &ro, float &m_l, float &den_l, float (&acc)[kHeads][4]) {
    constexpr int kPasses = Geo<D>::kPasses;
    float s[kPasses];
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
        const int tk = 8 * pass + ro.qg;
        float sh4[kHeads] = {0.f, 0.f, 0.f, 0.f};
        // chunks qj + 8c in pairs (one chunk for D = 64): K once, then every head's q
#pragma unroll
        for (int c0 = 0; c0 < Geo<D>::kLaneChunks; c0 += 2) {
            constexpr int kN = Geo<D>::kLaneChunks >= 2 ? 2 : 1;
            uint32_t kv[4 * kN];
#pragma unroll
            for (int c = 0; c < kN; ++c) {
                const uint4 kc = wt.k[tk][k_chunk<D>(tk, ro.qj + 8 * (c0 + c))];
                kv[4 * c] = kc.x, kv[4 * c + 1] = kc.y, kv[4 * c + 2] = kc.z, kv[4 * c + 3] = kc.w;
            }
#pragma unroll
            for (int h = 0; h < kHeads; ++h) {
                uint32_t qv[4 * kN];
#pragma unroll
                for (int c = 0; c < kN; ++c) {
                    const uint4 qc = qs[h][ro.qj + 8 * (c0 + c)];
                    qv[4 * c] = qc.x, qv[4 * c + 1] = qc.y, qv[4 * c + 2] = qc.z, qv[4 * c + 3] = qc.w;
                }
                float x = sh4[h];
#pragma unroll
                for (int q = 0; q < 4 * kN; ++q) x = dot2<DT>(qv[q], kv[q], x);
                sh4[h] = x;
            }
        }
        // reduce-scatter over the 8 lanes of the token
        float k0 = ro.b2 ? sh4[2] : sh4[0], k1 = ro.b2 ? sh4[3] : sh4[1];
        const float s0 = ro.b2 ? sh4[0] : sh4[2], s1 = ro.b2 ? sh4[1] : sh4[3];
        k0 += dpp<kRowHalfMirror>(s0);
        k1 += dpp<kRowHalfMirror>(s1);
        float kk = ro.b1 ? k1 : k0;
        const float ss = ro.b1 ? k0 : k1;
        kk += dpp<kQuadXor3>(ss);
        kk += dpp<kQuadXor1>(kk);
        s[pass] = (tk < nvalid) ? kk * scale2 : -INFINITY;
    }
    // max over the tile for head hs
    float mx = s[0];
#pragma unroll
    for (int pass = 1; pass < kPasses; ++pass) mx = fmaxf(mx, s[pass]);
    mx = fmaxf(mx, dpp<kRowRor8>(mx));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_l, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_l - m_new);
    m_l = m_new;
    float p[kPasses];
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) p[pass] = __builtin_amdgcn_exp2f(s[pass] - m_new);
    float psum = p[0];
#pragma unroll
    for (int pass = 1; pass < kPasses; ++pass) psum += p[pass];
    den_l = den_l * alpha + psum;
    // pairs (8*pass + qg, +1) for even qg, written once per (pair, head)
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
        const float pn = dpp<kRowShl8>(p[pass]);
        if (((ro.qg & 1) == 0) && ((ro.qj & 1) == 0)) {
            uint32_t *prow = reinterpret_cast<uint32_t *>(&wt.p[4 * pass + (ro.qg >> 1)]);
            prow[ro.hs] = pack2<DT>(p[pass], pn);
        }
    }
    // per-head rescale of the P.V accumulators
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
        const float al = lane_f(alpha, head_lane(h));
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[h][d] *= al;
    }
    wave_sync();
    // P.V over token pairs, dealt to the lane groups in turn
#pragma unroll
    for (int stp = 0; stp < Geo<D>::kPvSteps; ++stp) {
        const int pr = Geo<D>::kPvGroups * stp + ro.pg;
        const uint2 va = *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(&wt.v[2 * pr][0]) + ro.pd * 8);
        const uint2 vb =
            *reinterpret_cast<const uint2 *>(reinterpret_cast<const char *>(&wt.v[2 * pr + 1][0]) + ro.pd * 8);
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

// Reduce this wave's state to per-head values: m[h], den[h] (uniform) and acc
// summed over the P.V lane groups (valid in lanes < D / 4).
template <int D>
__device__ __forceinline__ void wave_state(float m_l, float den_l, float (&acc)[kHeads][4], float (&mh)[kHeads],
                                           float (&dh)[kHeads]) {
#pragma unroll
    for (int off = Geo<D>::kPvLanes; off < 64; off *= 2)
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[h][d] += __shfl_xor(acc[h][d], off, 64);
    float dl = den_l;  // sum over the 8 token groups sharing this lane's head
    dl += dpp<kRowRor8>(dl);
    dl += __shfl_xor(dl, 16, 64);
    dl += __shfl_xor(dl, 32, 64);
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
        mh[h] = lane_f(m_l, head_lane(h));
        dh[h] = lane_f(dl, head_lane(h));
    }
}

}  // namespace valu
}  // namespace sgd
