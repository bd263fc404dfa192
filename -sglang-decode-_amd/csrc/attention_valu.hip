// Persistent paged GQA decode attention for query-head groups of up to 4 heads
// (Llama-3-8B: 32 q / 8 kv), head_dim 128, unit dim stride -- the VALU path.
//
// Contraction sizes per token are 4 heads x 128 dims for QK^T and for P.V: far
// too narrow for a dense MFMA tile, so the math runs on the VALU with packed
// 16-bit dot products (v_dot2c_f32_bf16 / _f16, fp32 accumulate) and wave64 DPP
// reductions.  The kernel is HBM-bound; the design goal is to keep enough KV
// bytes in flight and touch each KV byte once.
//
// Worker = one workgroup of 4 waves; a task (record, kv head) is split across the
// waves in 32-token tiles (tile i -> wave i % 4).  Per wave and tile:
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
// Prefetch: the next tile's K/V loads and the tile-after-next's indices are in
// flight while a tile is computed.  At task end the 4 waves' (m, den, acc) are
// merged through LDS and the normalized partial + natural-log LSE are written to
// slot (request, head, split) (kernels/attention.py:81-84).
#include "attention_common.h"

namespace sgd {
namespace {

constexpr int kWaves = 4;
constexpr int kTile = 32;                 // tokens per wave per tile
constexpr int kD = 128;                   // head_dim
constexpr int kHeads = 4;                 // padded group
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct WaveTile {
    uint4 k[kTile][kD / 8];          // 8 KB  (also the task-merge area of this wave)
    uint4 v[kTile][kD / 8];          // 8 KB
    uint4 p[kTile / 2];              // token-pair probabilities: [pair] -> 4 heads x (p[2i], p[2i+1])
};

struct ValuShared {
    WaveTile w[kWaves];
    uint4 q[kHeads][kD / 8];
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

constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor3 = 0x1B;       // quad_perm [3,2,1,0]
constexpr int kRowShl8 = 0x108;       // row_shl:8
constexpr int kRowRor8 = 0x128;       // row_ror:8
constexpr int kRowHalfMirror = 0x141; // row_half_mirror
constexpr int kRowNewBcast = 0x150;   // row_newbcast:n

// Where the tile's K/V rows live: one 32-token tile of one task.
struct TileSrc {
    const char *kbase, *vbase;  // K/V + group * head stride (bytes)
    int64_t kp, kt, vp, vt;     // page / in-page strides in bytes
    int32_t tok0, end;          // first token of the tile, end of the task's split
};

template <bool CSR>
__device__ __forceinline__ int32_t load_tile_index(const sgd_decode_args &a, const TaskInfo &t, int32_t ind0,
                                                   int32_t tok0, int lane, int page_shift) {
    // lane 16r + i (i < 8) fetches the index of token tok0 + 4i + r
    const int r = lane >> 4, i = lane & 15;
    const int32_t tok = tok0 + 4 * i + r;
    int32_t v = 0;
    if (i < 8 && tok < t.end) {
        if constexpr (CSR) v = a.pages[ind0 + tok];
        else v = a.pages[(int64_t)t.request * a.pt_stride[0] + (int64_t)(tok >> page_shift) * a.pt_stride[1]];
    }
    return v;
}

template <bool CSR, bool FULL>
__device__ __forceinline__ void load_tile(const TileSrc &s, int32_t idxv, int32_t page_mask, int lane, uint4 (&kr)[8],
                                          uint4 (&vr)[8]) {
    const int r = lane >> 4, c = lane & 15;
#define SGD_LOAD_ROW(I)                                                                              \
    {                                                                                                \
        const uint32_t phys = (uint32_t)dpp_i<kRowNewBcast + I>(idxv);                               \
        const int32_t tok = s.tok0 + 4 * I + r;                                                      \
        int64_t ko = (int64_t)phys * s.kp + c * 16, vo = (int64_t)phys * s.vp + c * 16;              \
        if constexpr (!CSR) {                                                                        \
            const int32_t inner = tok & page_mask;                                                   \
            ko += (int64_t)inner * s.kt;                                                             \
            vo += (int64_t)inner * s.vt;                                                             \
        }                                                                                            \
        if (FULL || tok < s.end) {                                                                   \
            kr[I] = *reinterpret_cast<const uint4 *>(s.kbase + ko);                                  \
            vr[I] = *reinterpret_cast<const uint4 *>(s.vbase + vo);                                  \
        } else {                                                                                     \
            kr[I] = make_uint4(0, 0, 0, 0);                                                          \
            vr[I] = make_uint4(0, 0, 0, 0);                                                          \
        }                                                                                            \
    }
    SGD_LOAD_ROW(0) SGD_LOAD_ROW(1) SGD_LOAD_ROW(2) SGD_LOAD_ROW(3)
    SGD_LOAD_ROW(4) SGD_LOAD_ROW(5) SGD_LOAD_ROW(6) SGD_LOAD_ROW(7)
#undef SGD_LOAD_ROW
}

template <int DT, bool CSR>
__global__ __launch_bounds__(64 * kWaves, 2) void k_attention_valu(sgd_decode_args a) {
    extern __shared__ __align__(16) char dyn_smem[];
    ValuShared &sh = *reinterpret_cast<ValuShared *>(dyn_smem);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    WaveTile &wt = sh.w[wave];
    const int32_t G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    const int64_t kp = a.k_stride[0] * 2, kt = a.k_stride[1] * 2, kh = a.k_stride[2] * 2;
    const int64_t vp = a.v_stride[0] * 2, vt = a.v_stride[1] * 2, vh = a.v_stride[2] * 2;
    const uint16_t *q16 = static_cast<const uint16_t *>(a.q);
    const int page_shift = __builtin_ctz((unsigned)a.page_size);  // page_size is a power of two here
    const int32_t page_mask = a.page_size - 1;

    // QK lane roles: 8 lanes per token; j = lane % 8 owns 16 B chunks j and j + 8.
    const int qg = lane >> 3, qj = lane & 7;
    // after the reduce-scatter this lane holds head hs = 2*bit2(j) + bit1(j)
    const int hs = ((qj >> 2) << 1) | ((qj >> 1) & 1);
    const bool b2 = (qj & 4) != 0, b1 = (qj & 2) != 0;
    // P.V lane roles: half = lane / 32 takes token pairs 2s + half; dims 4*(lane % 32) .. +3
    const int ph = lane >> 5, pd = lane & 31;

    for_each_task(a, &sh.cursor, [&](int32_t task, int32_t mode) {
        const TaskInfo t = decode_task(a, task, mode);
        __syncthreads();  // the previous task's merge is done with shared memory
        if (wave == 0) {  // stage the group's q rows (any strides), heads >= G are zero
            const int h = lane >> 4, c = lane & 15;
            uint32_t w4[4] = {0, 0, 0, 0};
            if (h < G) {
                const int64_t base = (int64_t)t.request * a.q_stride[0] + (int64_t)(t.group * G + h) * a.q_stride[1];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t bits = q16[base + (int64_t)(c * 8 + e) * a.q_stride[2]];
                    w4[e >> 1] |= bits << (16 * (e & 1));
                }
            }
            sh.q[h][c] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        __syncthreads();
        uint32_t qr[kHeads][8];
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
            const uint4 lo = sh.q[h][qj], hi = sh.q[h][qj + 8];
            qr[h][0] = lo.x; qr[h][1] = lo.y; qr[h][2] = lo.z; qr[h][3] = lo.w;
            qr[h][4] = hi.x; qr[h][5] = hi.y; qr[h][6] = hi.z; qr[h][7] = hi.w;
        }

        const int32_t ntiles = (t.end - t.start + kTile - 1) / kTile;
        TileSrc src;
        src.kbase = static_cast<const char *>(a.k) + t.group * kh;
        src.vbase = static_cast<const char *>(a.v) + t.group * vh;
        src.kp = kp; src.kt = kt; src.vp = vp; src.vt = vt;
        src.end = t.end;
        const int32_t ind0 = CSR ? a.indptr[t.request] : 0;

        float m_l = -INFINITY, den_l = 0.f;  // this lane's head hs (QK roles)
        float acc[kHeads][4];
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;

        uint4 kr[8], vr[8];
        int32_t tile = wave;
        int32_t idx_next = 0;
        if (tile < ntiles) {
            const int32_t tok0 = t.start + tile * kTile;
            const int32_t idx0 = load_tile_index<CSR>(a, t, ind0, tok0, lane, page_shift);
            src.tok0 = tok0;
            if (tok0 + kTile <= t.end) load_tile<CSR, true>(src, idx0, page_mask, lane, kr, vr);
            else load_tile<CSR, false>(src, idx0, page_mask, lane, kr, vr);
            if (tile + kWaves < ntiles)
                idx_next = load_tile_index<CSR>(a, t, ind0, t.start + (tile + kWaves) * kTile, lane, page_shift);
        }
        for (; tile < ntiles; tile += kWaves) {
            const int32_t tok0 = t.start + tile * kTile;
            const int32_t nvalid = min(kTile, t.end - tok0);
            // stage this tile (rows 4i + r, 16 lanes per 256 B row)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                wt.k[4 * i + (lane >> 4)][lane & 15] = kr[i];
                wt.v[4 * i + (lane >> 4)][lane & 15] = vr[i];
            }
            // prefetch: next tile's K/V, the tile after's indices
            const int32_t nt = tile + kWaves;
            if (nt < ntiles) {
                src.tok0 = t.start + nt * kTile;
                if (src.tok0 + kTile <= t.end) load_tile<CSR, true>(src, idx_next, page_mask, lane, kr, vr);
                else load_tile<CSR, false>(src, idx_next, page_mask, lane, kr, vr);
                if (nt + kWaves < ntiles)
                    idx_next = load_tile_index<CSR>(a, t, ind0, t.start + (nt + kWaves) * kTile, lane, page_shift);
            }
            wave_sync();

            // QK^T: 4 passes of 8 tokens; token 8*pass + qg
            float s[4];
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const int tk = 8 * pass + qg;
                const uint4 lo = wt.k[tk][qj], hi = wt.k[tk][qj + 8];
                const uint32_t kv[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                float sh4[kHeads];
#pragma unroll
                for (int h = 0; h < kHeads; ++h) {
                    float x = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) x = dot2<DT>(qr[h][e], kv[e], x);
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
            float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mx = fmaxf(mx, dpp<kRowRor8>(mx));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_l, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_l - m_new);
            m_l = m_new;
            float p[4];
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) p[pass] = __builtin_amdgcn_exp2f(s[pass] - m_new);
            den_l = den_l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
            // pairs (8*pass + qg, +1) for even qg, written once per (pair, head)
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const float pn = dpp<kRowShl8>(p[pass]);
                if (((qg & 1) == 0) && ((qj & 1) == 0)) {
                    uint32_t *prow = reinterpret_cast<uint32_t *>(&wt.p[4 * pass + (qg >> 1)]);
                    prow[hs] = pack2<DT>(p[pass], pn);
                }
            }
            // per-head rescale of the P.V accumulators (heads are held by lanes 0, 2, 4, 6)
            float al[kHeads];
#pragma unroll
            for (int h = 0; h < kHeads; ++h) {
                const int src_lane = ((h >> 1) << 2) | ((h & 1) << 1);
                al[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), src_lane));
            }
#pragma unroll
            for (int h = 0; h < kHeads; ++h)
#pragma unroll
                for (int d = 0; d < 4; ++d) acc[h][d] *= al[h];
            wave_sync();

            // P.V over token pairs
#pragma unroll
            for (int st = 0; st < kTile / 4; ++st) {
                const int pr = 2 * st + ph;
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
        // ---- end of the wave's tiles: reduce within the wave, then merge the 4 waves
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
        {
            const int h = threadIdx.x >> 6, d = (threadIdx.x & 63) * 2;
            if (h < G) {
                float mm = -INFINITY;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sh.cm[w][h]);
                float dd = 0.f, x0 = 0.f, x1 = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float sc = __builtin_amdgcn_exp2f(sh.cm[w][h] - mm);
                    const float *cw = reinterpret_cast<const float *>(&sh.w[w].k[0][0]) + h * kD + d;
                    dd += sh.cd[w][h] * sc;
                    x0 += cw[0] * sc;
                    x1 += cw[1] * sc;
                }
                const int64_t slot = ((int64_t)t.request * a.query_heads + t.group * G + h) * a.max_splits + t.split;
                const float inv = 1.0f / dd;
                *reinterpret_cast<float2 *>(&a.partial[slot * kD + d]) = make_float2(x0 * inv, x1 * inv);
                if (d == 0) a.lse[slot] = (mm + __log2f(dd)) * kLn2;
            }
        }
    });
}

template <int DT, bool CSR>
int launch_valu_t(const sgd_decode_args &a, hipStream_t stream) {
    static bool attr = false;
    const int bytes = (int)sizeof(ValuShared);
    if (!attr) {
        if (hipFuncSetAttribute((const void *)k_attention_valu<DT, CSR>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                bytes) != hipSuccess)
            return einval("valu attention: cannot reserve %d B of LDS", bytes);
        attr = true;
    }
    hipLaunchKernelGGL((k_attention_valu<DT, CSR>), dim3(a.workers), dim3(64 * kWaves), bytes, stream, a);
    return launch_status("persistent_decode(valu)");
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
