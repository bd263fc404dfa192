// Upstream SGLang's two-stage split-KV decode, rebuilt for gfx950 as the comparator of
// the reference's benchmark (benchmarks/baselines.py:8-34, which runs the pinned Triton
// file third_party/sglang/decode_attention.py:245-601 of SGLang v0.4.6.post5).  It is the
// schedule the persistent path replaces, so it uses the same VALU tile math
// (valu_ops.h) and only the scheduling differs:
//
// stage 1: a grid of one workgroup per (split s < max_kv_splits, kv head, request b).
//          Request b's L tokens are cut into chunks of c = ceil(ceil(L / S) / 32) * 32
//          tokens, S = num_kv_splits[b]; split s covers [s*c, min((s+1)*c, L)) and an
//          empty one returns at once (upstream launches every (b, head, s) program and
//          masks).  The workgroup's 8 waves take the split's 16-token tiles round-robin;
//          the normalized partial and the natural-log LSE of each q head of the group go
//          to attn_out[b, h, s, :] / attn_lse[b, h, s].
// stage 2: one wave per (b, q head) merges the row's non-empty splits (s < ceil(L / c))
//          by LSE in split order into out[b, h, :].
#include "merge_ops.h"
#include "valu_ops.h"

namespace sgd {
namespace {

using namespace valu;

constexpr int kUpWaves = 8;
constexpr int kD = 128;  // upstream's comparator runs the 8B head shape only
constexpr int kTile = Geo<kD>::kTile;

struct UpShared {
    WaveTile<kD> w[kUpWaves];
    uint4 q[kHeads][kD / 8];
    float cm[kUpWaves][kHeads];
    float cd[kUpWaves][kHeads];
};

// Split geometry of request b: (first token, end) of split s, or an empty range.
__device__ __forceinline__ int2 split_range(const int32_t *indptr, const int32_t *num_splits, int32_t b, int32_t s,
                                            int32_t max_splits, int32_t &chunk, int32_t &length) {
    length = max(indptr[b + 1] - indptr[b], 0);
    const int32_t S = min(max(num_splits[b], 1), max_splits);
    chunk = ((length + S - 1) / S + 31) / 32 * 32;
    const int64_t t0 = (int64_t)chunk * s;
    const int64_t t1 = min(t0 + chunk, (int64_t)length);
    return t1 > t0 ? make_int2((int32_t)t0, (int32_t)t1) : make_int2(0, 0);
}

template <int DT>
__global__ __launch_bounds__(64 * kUpWaves, 4) void k_upstream_split(sgd_decode_args a, const int32_t *num_splits) {
    extern __shared__ __align__(16) char dyn_smem[];
    UpShared &sh = *reinterpret_cast<UpShared *>(dyn_smem);
    const int32_t split = blockIdx.x, group = blockIdx.y, b = blockIdx.z;
    int32_t chunk, length;
    const int2 range = split_range(a.indptr, num_splits, b, split, a.max_splits, chunk, length);
    if (range.y <= range.x) return;  // uniform over the workgroup
    const int lane = threadIdx.x & 63, wave = uni(threadIdx.x >> 6);
    WaveTile<kD> &wt = sh.w[wave];
    const int32_t G = a.query_heads / a.kv_heads;
    const float scale2 = a.scale * kLog2e;
    const PageMap<true> csr_pages(1);  // CSR: one token per page (no page arithmetic)

    TileSrc T;
    T.request = b;
    T.start = range.x;
    T.end = range.y;
    T.ind0 = uni(a.indptr[b]);
    T.kbase = static_cast<const char *>(a.k) + group * (a.k_stride[2] * 2);
    T.vbase = static_cast<const char *>(a.v) + group * (a.v_stride[2] * 2);
    T.kp = a.k_stride[0] * 2;
    T.kt = 0;
    T.vp = a.v_stride[0] * 2;
    T.vt = 0;
    const int32_t ntiles = (T.end - T.start + kTile - 1) / kTile;
    const int32_t n0 = ntiles > wave ? (ntiles - wave + kUpWaves - 1) / kUpWaves : 0;
    uint4 kr[kRowsLoads], vr[kRowsLoads];
    int32_t idx_next = 0;
    if (n0 > 0) {
        const int32_t i0 = tile_index<true, kD>(a, T, T.start + wave * kTile, lane, csr_pages);
        tile_issue<true, kD>(T, wave, i0, csr_pages, lane, kr, vr);
        if (n0 > 1) idx_next = tile_index<true, kD>(a, T, T.start + (wave + kUpWaves) * kTile, lane, csr_pages);
    }
    if (wave == 0) {  // q rows of the group: head lane / 16, dims 8 (lane % 16) ..; zero past G
        const int h = lane >> 4, c = lane & 15;
        uint4 qrow = make_uint4(0, 0, 0, 0);
        if (h < G) {
            const int64_t qd = a.q_stride[2];
            const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (int64_t)b * a.q_stride[0] +
                                 (int64_t)(group * G + h) * a.q_stride[1] + (int64_t)(c * 8) * qd;
            uint32_t w4[4] = {0, 0, 0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e) w4[e >> 1] |= (uint32_t)qp[e * qd] << (16 * (e & 1));
            qrow = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
        sh.q[h][c] = qrow;
    }
    lds_barrier();
    float m_l = -INFINITY, den_l = 0.f;
    float acc[kHeads][4];
#pragma unroll
    for (int h = 0; h < kHeads; ++h)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[h][d] = 0.f;
    for (int32_t e = 0; e < n0; ++e) {
        const Roles<kD> ro(lane);
        const int32_t tile = wave + kUpWaves * e;
        const int32_t nvalid = min(kTile, T.end - (T.start + tile * kTile));
        tile_stage<kD>(wt, kr, vr, lane, nvalid);
        if (e + 1 < n0) tile_issue<true, kD>(T, tile + kUpWaves, idx_next, csr_pages, lane, kr, vr);
        if (e + 2 < n0) idx_next = tile_index<true, kD>(a, T, T.start + (tile + 2 * kUpWaves) * kTile, lane, csr_pages);
        wave_sync();
        tile_compute<DT, kD>(wt, sh.q, nvalid, scale2, ro, m_l, den_l, acc);
    }
    // the waves' states: per-head (m, den) to LDS, acc into the wave's K tile area
    const Roles<kD> ro(lane);
    float mh[kHeads], dh[kHeads];
    wave_state<kD>(m_l, den_l, acc, mh, dh);
    float *comb = reinterpret_cast<float *>(&wt.k[0][0]);
    if (lane < 32) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h)
            *reinterpret_cast<float4 *>(&comb[h * kD + ro.pd * 4]) =
                make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    }
    if (lane < kHeads) {
        float mv = mh[0], dv = dh[0];
#pragma unroll
        for (int h = 1; h < kHeads; ++h)
            if (lane == h) {
                mv = mh[h];
                dv = dh[h];
            }
        sh.cm[wave][lane] = mv;
        sh.cd[wave][lane] = dv;
    }
    lds_barrier();
    static_assert(kUpWaves * 64 >= kHeads * kD, "one thread per (head, dim) output");
    const int h = threadIdx.x / kD, d = threadIdx.x % kD;
    if (h < G) {
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < kUpWaves; ++w) mm = fmaxf(mm, sh.cm[w][h]);
        float dd = 0.f, x = 0.f;
#pragma unroll
        for (int w = 0; w < kUpWaves; ++w) {
            const float sc = __builtin_amdgcn_exp2f(sh.cm[w][h] - mm);
            dd += sh.cd[w][h] * sc;
            x += reinterpret_cast<const float *>(&sh.w[w].k[0][0])[h * kD + d] * sc;
        }
        const int64_t slot = ((int64_t)b * a.query_heads + group * G + h) * a.max_splits + split;
        a.partial[slot * kD + d] = x / dd;
        if (d == 0) a.lse[slot] = (mm + __log2f(dd)) * kLn2;
    }
}

template <int DT>
__global__ __launch_bounds__(64) void k_upstream_merge(const float *__restrict__ attn_out,
                                                       const float *__restrict__ attn_lse,
                                                       const int32_t *__restrict__ indptr,
                                                       const int32_t *__restrict__ num_splits,
                                                       uint16_t *__restrict__ out, int32_t hq, int32_t max_splits) {
    const int32_t b = blockIdx.x, h = blockIdx.y;
    int32_t chunk, length;
    (void)split_range(indptr, num_splits, b, 0, max_splits, chunk, length);
    const int32_t n = length > 0 ? __builtin_amdgcn_readfirstlane((length + chunk - 1) / chunk) : 0;
    const int lane = threadIdx.x;
    float m, den, acc[2];
    mergeops::merge_part<2>(attn_out, attn_lse, (int64_t)b * hq + h, max_splits, 0, n, lane, m, den, acc);
    mergeops::store_row<DT, 2>(out, (int64_t)b * hq + h, den, acc, false, lane);
}

template <int DT>
int launch_upstream(const sgd_decode_args &a, const int32_t *num_splits, void *out, int32_t batch,
                    hipStream_t stream) {
    static bool attr[kOnceDevices] = {};
    const int bytes = (int)sizeof(UpShared);
    if (int rc = set_dynamic_lds((const void *)k_upstream_split<DT>, bytes, attr, "upstream_decode")) return rc;
    hipLaunchKernelGGL(k_upstream_split<DT>, dim3(a.max_splits, a.kv_heads, batch), dim3(64 * kUpWaves), bytes,
                       stream, a, num_splits);
    if (int rc = launch_status("upstream_decode(stage 1)")) return rc;
    hipLaunchKernelGGL(k_upstream_merge<DT>, dim3(batch, a.query_heads), dim3(64), 0, stream, a.partial, a.lse,
                       a.indptr, num_splits, static_cast<uint16_t *>(out), a.query_heads, a.max_splits);
    return launch_status("upstream_decode(stage 2)");
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_upstream_decode(const void *q, const void *k, const void *v, void *out, const int32_t *kv_indptr,
                                   const int32_t *kv_indices, float *attn_out, float *attn_lse,
                                   const int32_t *num_kv_splits, int32_t batch, int32_t max_kv_splits,
                                   int32_t query_heads, int32_t kv_heads, int32_t head_dim,
                                   const int64_t *q_strides, const int64_t *kv_strides, float scale, int32_t dtype,
                                   void *stream) {
    if (!q || !k || !v || !out || !kv_indptr || !kv_indices || !attn_out || !attn_lse || !num_kv_splits ||
        !q_strides || !kv_strides)
        return einval("upstream_decode: null argument");
    if (batch < 0 || batch > 65535 || max_kv_splits < 1 || max_kv_splits > 65535)
        return einval("upstream_decode: batch %d / max_kv_splits %d out of range", batch, max_kv_splits);
    if (kv_heads <= 0 || query_heads <= 0 || query_heads % kv_heads || query_heads / kv_heads > valu::kHeads ||
        kv_heads > 65535)
        return einval("upstream_decode: heads %d/%d (the tile math takes groups of up to %d)", query_heads, kv_heads,
                      valu::kHeads);
    if (head_dim != kD) return einval("upstream_decode: head_dim %d (128 only)", head_dim);
    if (dtype != SGD_BF16 && dtype != SGD_FP16) return einval("upstream_decode: dtype %d", dtype);
    for (int i = 0; i < 4; ++i)
        if (kv_strides[i] % 8 || kv_strides[i] <= 0 || kv_strides[i] >= (1ll << 40))
            return einval("upstream_decode: K/V token and head strides must be positive multiples of 8");
    if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) & 15)
        return einval("upstream_decode: K/V not 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(attn_out) & 15) return einval("upstream_decode: attn_out not 16-byte aligned");
    if (batch == 0) return 0;
    sgd_decode_args a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.pages = kv_indices;
    a.indptr = kv_indptr;
    a.partial = attn_out;
    a.lse = attn_lse;
    a.scale = scale;
    for (int i = 0; i < 3; ++i) a.q_stride[i] = q_strides[i];
    a.k_stride[0] = kv_strides[0];
    a.k_stride[1] = 0;
    a.k_stride[2] = kv_strides[1];
    a.k_stride[3] = 1;
    a.v_stride[0] = kv_strides[2];
    a.v_stride[1] = 0;
    a.v_stride[2] = kv_strides[3];
    a.v_stride[3] = 1;
    a.query_heads = query_heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.max_splits = max_kv_splits;
    a.page_size = 1;
    a.csr = 1;
    a.dtype = dtype;
    clear_stale_error();
    if (dtype == SGD_BF16) return launch_upstream<SGD_BF16>(a, num_kv_splits, out, batch, (hipStream_t)stream);
    return launch_upstream<SGD_FP16>(a, num_kv_splits, out, batch, (hipStream_t)stream);
}
