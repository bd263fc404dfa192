// Split merge: per (request, query head), LSE-weighted combination of the
// normalized partial outputs of its splits (kernels/merge.py:7-30).
//
// The merge is latency-bound (a few KB per row): the split count, then the split
// LSEs together with up to kRowsInFlight partial rows (each a coalesced 256-1024 B
// burst, lanes owning head_dim/64 consecutive dims), all issued before any is used.
// A row with more splits is cut over the workgroup's waves (k_merge).  The max and
// the weights exp(lse_s - max) come from wave reductions, combined online from block
// to block and wave to wave in a fixed order: the value of the reference's running-max
// merge up to rounding.  Rows with no split produce exact zeros (0 / max(den, 1e-30));
// a plan error produces NaN.
#include "common.h"
#include "span_layout.h"

namespace sgd {
namespace {

constexpr int kMergeWaves = 1;  // span merge: one (request, head) per workgroup
constexpr int kRowsInFlight = 16;  // split rows (and the span merge's edge rows) per round trip
constexpr float kLog2e = 1.4426950408889634f;

template <int DPL>
__device__ __forceinline__ void load_row(const float *src, float (&v)[DPL]) {
    if constexpr (DPL == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(src);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else if constexpr (DPL == 2) {
        const float2 t = *reinterpret_cast<const float2 *>(src);
        v[0] = t.x; v[1] = t.y;
    } else {
        v[0] = src[0];
    }
}

// One wave's LSE-weighted sum over splits [s0, s1) of the (request, head) row `row`:
// its running max m (log2 domain), denominator and unnormalized sum acc (this lane's
// DPL dims), built in blocks of kRowsInFlight split rows -- each block's rows and
// LSEs in flight together -- combined online from block to block.  An empty range
// leaves (-inf, 0, 0).
template <int DPL>
__device__ __forceinline__ void merge_part(const float *__restrict__ partial, const float *__restrict__ lse,
                                           int64_t row, int32_t smax, int32_t s0, int32_t s1, int lane,
                                           float &m, float &den, float (&acc)[DPL]) {
    constexpr int D = DPL * 64;
    const float *lrow = lse + row * smax;
    const float *prow = partial + row * smax * D + lane * DPL;
    m = -INFINITY;
    den = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    for (int b = s0; b < s1; b += kRowsInFlight) {
        float v[kRowsInFlight][DPL];
#pragma unroll
        for (int s = 0; s < kRowsInFlight; ++s) {
            if (b + s < s1) load_row<DPL>(prow + (int64_t)(b + s) * D, v[s]);
            else
#pragma unroll
                for (int i = 0; i < DPL; ++i) v[s][i] = 0.f;
        }
        // lane l < kRowsInFlight holds split b + l's LSE
        const bool mine = lane < kRowsInFlight && b + lane < s1;
        const float l2 = mine ? lrow[b + lane] * kLog2e : -INFINITY;
        const float mb = fmaxf(m, wave_max(l2));
        const float so = __builtin_amdgcn_exp2f(m - mb);  // 0 for the first block (m = -inf)
        const float w = mine ? __builtin_amdgcn_exp2f(l2 - mb) : 0.f;
        den = den * so + wave_sum(w);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] *= so;
#pragma unroll
        for (int s = 0; s < kRowsInFlight; ++s) {
            if (b + s < s1) {
                const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s));
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[i] += v[s][i] * ws;
            }
        }
        m = mb;
    }
}

// The merged row out = acc / den (0 for a row without splits, NaN on a plan error).
template <int DT, int DPL>
__device__ __forceinline__ void store_row(uint16_t *__restrict__ out, int64_t row, float den,
                                          const float (&acc)[DPL], bool bad, int lane) {
    const float inv = 1.0f / fmaxf(den, 1.0e-30f);
    uint16_t *dst = out + row * (DPL * 64) + lane * DPL;
#pragma unroll
    for (int i = 0; i < DPL; ++i) dst[i] = (uint16_t)from_f32<DT>(bad ? __builtin_nanf("") : acc[i] * inv);
}

// The merge of one (request, head) row by one wave: n splits of partial/lse rows.
template <int DT, int DPL>  // DPL = dims per lane
__device__ __forceinline__ void merge_row(const float *__restrict__ partial, const float *__restrict__ lse,
                                          int32_t n, bool bad, uint16_t *__restrict__ out, int64_t row,
                                          int32_t smax, int lane) {
    float m, den, acc[DPL];
    merge_part<DPL>(partial, lse, row, smax, 0, n, lane, m, den, acc);
    store_row<DT, DPL>(out, row, den, acc, bad, lane);
}

// One workgroup of kSplitWaves waves per (request, head).  A row with at most
// kRowsInFlight splits is merged by wave 0 alone (one round trip for its data); a
// longer one is cut into kSplitWaves contiguous split ranges, merged by the waves side
// by side and combined in wave order through LDS -- so a 64-split row costs a block's
// round trip, not four.
constexpr int kSplitWaves = 4;

template <int DT, int DPL>
__global__ __launch_bounds__(64 * kSplitWaves) void k_merge(const float *__restrict__ partial,
                                                            const float *__restrict__ lse,
                                                            const int32_t *__restrict__ counts,
                                                            const int32_t *__restrict__ error,
                                                            uint16_t *__restrict__ out, int32_t hq,
                                                            int32_t smax) {
    __shared__ float sm[kSplitWaves], sd[kSplitWaves], sacc[kSplitWaves][DPL * 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = blockIdx.x, head = blockIdx.y;
    const int32_t n = __builtin_amdgcn_readfirstlane(counts[r]);
    const bool bad = *error != 0;
    const int64_t row = (int64_t)r * hq + head;
    if (n <= kRowsInFlight) {
        if (wave == 0) merge_row<DT, DPL>(partial, lse, n, bad, out, row, smax, lane);
        return;  // n is the workgroup's: no wave waits below
    }
    const int32_t q = (n + kSplitWaves - 1) / kSplitWaves;
    float m, den, acc[DPL];
    merge_part<DPL>(partial, lse, row, smax, min(wave * q, n), min((wave + 1) * q, n), lane, m, den, acc);
    if (lane == 0) {
        sm[wave] = m;
        sd[wave] = den;
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i) sacc[wave][lane * DPL + i] = acc[i];
    lds_barrier();
    if (wave != 0) return;
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kSplitWaves; ++k) M = fmaxf(M, sm[k]);
    float D = 0.f, X[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) X[i] = 0.f;
#pragma unroll
    for (int k = 0; k < kSplitWaves; ++k) {
        if (sd[k] == 0.f) continue;  // an empty range
        const float sc = __builtin_amdgcn_exp2f(sm[k] - M);
        D += sd[k] * sc;
#pragma unroll
        for (int i = 0; i < DPL; ++i) X[i] += sacc[k][lane * DPL + i] * sc;
    }
    store_row<DT, DPL>(out, row, D, X, bad, lane);
}

// The common case of the span merge in two memory round trips: the row's split
// geometry (scalar loads issued together), then every split's LSE -- or, for a split
// whose task a workgroup boundary cut, the two edge states it left (record 1 of the
// workgroup where it starts, record 0 of the next) -- together with every split's
// row(s), all issued before any is used.  Cut splits are combined in registers (their
// slots are written for the API; nothing re-reads them) and all splits merged by LSE.
// Returns false, having written nothing, when a split's task spans more than two
// workgroups (the general path handles that).
template <int DT>
__device__ __forceinline__ bool merge_span_fast(float *__restrict__ partial, float *__restrict__ lse,
                                                uint16_t *__restrict__ out, const float *__restrict__ edge,
                                                int32_t hq, int32_t hkv, int32_t smax, int32_t units, int head,
                                                int32_t n, int32_t p0, int32_t p1, int32_t pT, int32_t chunk_r,
                                                bool bad, int64_t row, int lane) {
    using namespace span;
    constexpr int D = kD, DPL = kD / 64;
    const int32_t G = hq / hkv, g = head / G, hl = head - g * G;
    const int32_t c16 = chunk_r / kTile;
    const int64_t T = (int64_t)hkv * pT;
    const int32_t t0 = hkv * p0, nt_last = (p1 - p0) - (n - 1) * c16;
    // lane s: split s's task tiles [c0, c0 + nt) and the workgroups holding its ends
    const int s = lane;
    const bool valid = s < n;
    const int32_t nt = s == n - 1 ? nt_last : c16;
    const int64_t c0 = t0 + (int64_t)s * hkv * c16 + (int64_t)g * nt;
    const int32_t w0 = valid ? worker_of(c0, T, units) : 0, w1 = valid ? worker_of(c0 + nt - 1, T, units) : 0;
    const bool cut = valid && w0 != w1;
    bool far = cut && w1 - w0 > 1;
    if (far) {  // a workgroup in between with no tiles holds nothing
        far = false;
        for (int32_t w = w0 + 1; w < w1; ++w)
            if (worker_start(w, T, units) != worker_start(w + 1, T, units)) far = true;
    }
    if (__ballot(far)) return false;
    // ---- one round trip: LSEs or edge statistics (lane = split) and the rows of the first
    // kRowsInFlight splits (a cut split's two edge rows, else its partial row)
    const float *e0 = edge + ((int64_t)w0 * 2 + 1) * kPieceFloats, *e1 = edge + ((int64_t)w1 * 2) * kPieceFloats;
    const float l_in = valid && !cut ? lse[row * smax + s] : 0.f;
    const float m0 = cut ? e0[kPieceM + hl] : 0.f, d0 = cut ? e0[kPieceDen + hl] : 0.f;
    const float m1 = cut ? e1[kPieceM + hl] : 0.f, d1 = cut ? e1[kPieceDen + hl] : 0.f;
    const float *prow = partial + row * smax * D + lane * DPL;
    const uint64_t cutmask = __ballot(cut);
    float va[kRowsInFlight][DPL], vb[kRowsInFlight][DPL];
    // Unconditional loads (no branch around any): a slot past the last split re-reads
    // the last split's row, and its weight (lane >= n) is zero.
    auto load_block = [&](int b) {
#pragma unroll
        for (int k = 0; k < kRowsInFlight; ++k) {
            const int sp = min(b + k, n - 1);
            const bool ck = (cutmask >> sp) & 1;
            const int32_t a0 = __builtin_amdgcn_readlane(w0, sp), a1 = __builtin_amdgcn_readlane(w1, sp);
            const float *ra = ck ? edge + ((int64_t)a0 * 2 + 1) * kPieceFloats + hl * D + lane * DPL
                                 : prow + (int64_t)sp * D;
            const float *rb = ck ? edge + ((int64_t)a1 * 2) * kPieceFloats + hl * D + lane * DPL : ra;
            load_row<DPL>(ra, va[k]);
            load_row<DPL>(rb, vb[k]);
        }
    };
    load_block(0);
    // the split's log2-domain LSE (cut: combined from the two states) and the merge weights
    const float Mc = fmaxf(m0, m1);
    const float sa = __builtin_amdgcn_exp2f(m0 - Mc), sb = __builtin_amdgcn_exp2f(m1 - Mc);
    const float Dc = d0 * sa + d1 * sb;
    const float l2 = !valid ? -INFINITY : cut ? Mc + __log2f(Dc) : l_in * kLog2e;
    const float mx = wave_max(l2);
    const float wgt = valid ? __builtin_amdgcn_exp2f(l2 - mx) : 0.f;
    const float den = wave_sum(wgt);
    if (cut) lse[row * smax + s] = l2 / kLog2e;
    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    for (int b = 0; b < n; b += kRowsInFlight) {
        if (b > 0) load_block(b);
#pragma unroll
        for (int k = 0; k < kRowsInFlight; ++k) {
            const int sp = b + k;
            if (sp >= n) continue;
            const float ws = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), sp));
            if ((cutmask >> sp) & 1) {
                const float fa = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sa), sp));
                const float fb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sb), sp));
                const float fd = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, Dc), sp));
                const float inv = 1.0f / fd;
                float nr[DPL];
#pragma unroll
                for (int i = 0; i < DPL; ++i) nr[i] = (va[k][i] * fa + vb[k][i] * fb) * inv;
                // the split's slot, as the per-task kernels leave it
                float *dst = partial + (row * smax + sp) * D + lane * DPL;
#pragma unroll
                for (int i = 0; i < DPL; ++i) dst[i] = nr[i];
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[i] += nr[i] * ws;
            } else {
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[i] += va[k][i] * ws;
            }
        }
    }
    const float inv = 1.0f / fmaxf(den, 1.0e-30f);
    uint16_t *dst = out + row * D + lane * DPL;
#pragma unroll
    for (int i = 0; i < DPL; ++i) dst[i] = (uint16_t)from_f32<DT>(bad ? __builtin_nanf("") : acc[i] * inv);
    return true;
}

// Span schedule (attention_span.hip): a task cut by a workgroup boundary left its
// softmax state in the edge records of the workgroups it spans -- record 1 of the
// one where it starts, record 0 of each later one.  Those are combined first and
// written to the task's slot (so every slot holds its split's normalized partial and
// LSE, as after the per-task kernels), then the row is merged as usual.
template <int DT>
__global__ __launch_bounds__(64 * kMergeWaves) void k_merge_span(
    float *__restrict__ partial, float *__restrict__ lse, const int32_t *__restrict__ counts,
    const int32_t *__restrict__ error, uint16_t *__restrict__ out, const int32_t *__restrict__ tile_prefix,
    const int32_t *__restrict__ chunk, const float *__restrict__ edge, int32_t bcap, int32_t hq, int32_t hkv,
    int32_t smax, int32_t units) {
    using namespace span;
    const int lane = threadIdx.x & 63;
    const int head = blockIdx.y * kMergeWaves + (threadIdx.x >> 6);
    const int r = blockIdx.x;
    if (head >= hq) return;
    // the row's geometry in one round trip: lanes 0..5 gather counts[r], tile_prefix[r],
    // tile_prefix[r + 1], tile_prefix[bcap], chunk[r] and the error flag
    const int32_t *src = lane == 0   ? counts + r
                         : lane == 1 ? tile_prefix + r
                         : lane == 2 ? tile_prefix + r + 1
                         : lane == 3 ? tile_prefix + bcap
                         : lane == 4 ? chunk + r
                                     : error;
    const int32_t gv = *src;
    const int32_t n = __builtin_amdgcn_readlane(gv, 0), p0 = __builtin_amdgcn_readlane(gv, 1);
    const int32_t p1 = __builtin_amdgcn_readlane(gv, 2), pT = __builtin_amdgcn_readlane(gv, 3);
    const int32_t chunk_r = __builtin_amdgcn_readlane(gv, 4), err = __builtin_amdgcn_readlane(gv, 5);
    const int64_t row = (int64_t)r * hq + head;
    if (n > 0 && n <= 64 &&
        merge_span_fast<DT>(partial, lse, out, edge, hq, hkv, smax, units, head, n, p0, p1, pT, chunk_r, err != 0,
                            row, lane))
        return;
    if (n > 0) {
        const int32_t G = hq / hkv, g = head / G, hl = head - g * G;
        const int32_t p0 = __builtin_amdgcn_readfirstlane(tile_prefix[r]);
        const int32_t p1 = __builtin_amdgcn_readfirstlane(tile_prefix[r + 1]);
        const int32_t c16 = __builtin_amdgcn_readfirstlane(chunk[r]) / kTile;
        const int64_t T = (int64_t)hkv * __builtin_amdgcn_readfirstlane(tile_prefix[bcap]);
        const int32_t t0 = hkv * p0, nt_last = (p1 - p0) - (n - 1) * c16;
        bool wrote = false;
        for (int32_t s = 0; s < n; ++s) {
            const bool last = s == n - 1;
            const int32_t nt = last ? nt_last : c16;
            const int64_t c0 = t0 + (int64_t)s * hkv * c16 + (int64_t)g * nt;
            const int32_t w0 = worker_of(c0, T, units), w1 = worker_of(c0 + nt - 1, T, units);
            if (w0 == w1) continue;
            // the states of the first and the last worker, then those in between
            const float *e0 = edge + ((int64_t)w0 * 2 + 1) * kPieceFloats;
            const float *e1 = edge + ((int64_t)w1 * 2 + 0) * kPieceFloats;
            const float2 a0 = *reinterpret_cast<const float2 *>(e0 + hl * kD + 2 * lane);
            const float2 a1 = *reinterpret_cast<const float2 *>(e1 + hl * kD + 2 * lane);
            const float m0 = e0[kPieceM + hl], d0 = e0[kPieceDen + hl];
            const float m1 = e1[kPieceM + hl], d1 = e1[kPieceDen + hl];
            float M = fmaxf(m0, m1);
            float s0 = __builtin_amdgcn_exp2f(m0 - M), s1 = __builtin_amdgcn_exp2f(m1 - M);
            float Dn = d0 * s0 + d1 * s1;
            float x = a0.x * s0 + a1.x * s1, y = a0.y * s0 + a1.y * s1;
            for (int32_t w = w0 + 1; w < w1; ++w) {
                if (worker_start(w, T, units) == worker_start(w + 1, T, units)) continue;  // empty workgroup
                const float *e = edge + ((int64_t)w * 2 + 0) * kPieceFloats;
                const float2 av = *reinterpret_cast<const float2 *>(e + hl * kD + 2 * lane);
                const float mv = e[kPieceM + hl], dv = e[kPieceDen + hl];
                const float mx = fmaxf(M, mv);
                const float so = __builtin_amdgcn_exp2f(M - mx), sv = __builtin_amdgcn_exp2f(mv - mx);
                M = mx;
                Dn = Dn * so + dv * sv;
                x = x * so + av.x * sv;
                y = y * so + av.y * sv;
            }
            const float inv = 1.0f / Dn;
            const int64_t slot = row * smax + s;
            *reinterpret_cast<float2 *>(partial + slot * kD + 2 * lane) = make_float2(x * inv, y * inv);
            if (lane == 0) lse[slot] = (M + __log2f(Dn)) / kLog2e;
            wrote = true;
        }
        if (wrote) {  // the row merge below reads these slots (other lanes read the LSE)
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        }
    }
    merge_row<DT, kD / 64>(partial, lse, n, *error != 0, out, row, smax, lane);
}

template <int DT>
int launch_merge(const float *partial, const float *lse, const int32_t *counts, const int32_t *error, void *out,
                 int32_t bcap, int32_t hq, int32_t d, int32_t smax, hipStream_t stream) {
    const dim3 grid(bcap, hq), block(64 * kSplitWaves);
    auto *o = static_cast<uint16_t *>(out);
    switch (d) {
        case 64: hipLaunchKernelGGL((k_merge<DT, 1>), grid, block, 0, stream, partial, lse, counts, error, o, hq, smax); break;
        case 128: hipLaunchKernelGGL((k_merge<DT, 2>), grid, block, 0, stream, partial, lse, counts, error, o, hq, smax); break;
        case 256: hipLaunchKernelGGL((k_merge<DT, 4>), grid, block, 0, stream, partial, lse, counts, error, o, hq, smax); break;
        default: return einval("merge_splits: head_dim %d not in {64,128,256}", d);
    }
    return launch_status("merge_splits");
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_merge_splits(const float *partial, const float *lse, const int32_t *counts,
                                const int32_t *active, const int32_t *error, void *out, int32_t bcap,
                                int32_t query_heads, int32_t head_dim, int32_t max_splits, int32_t dtype,
                                void *stream) {
    (void)active;  // every row r < bcap is written; inactive rows have counts[r] == 0
    if (bcap <= 0 || query_heads <= 0 || max_splits <= 0) return einval("merge_splits: bad geometry");
    if ((reinterpret_cast<uintptr_t>(partial) & 15) != 0) return einval("merge_splits: partial not 16B aligned");
    clear_stale_error();
    if (dtype == SGD_BF16)
        return launch_merge<SGD_BF16>(partial, lse, counts, error, out, bcap, query_heads, head_dim, max_splits,
                                      (hipStream_t)stream);
    if (dtype == SGD_FP16)
        return launch_merge<SGD_FP16>(partial, lse, counts, error, out, bcap, query_heads, head_dim, max_splits,
                                      (hipStream_t)stream);
    return einval("merge_splits: dtype %d", dtype);
}

extern "C" int sgd_merge_splits_span(float *partial, float *lse, const int32_t *counts, const int32_t *error,
                                     void *out, const int32_t *tile_prefix, const int32_t *chunk,
                                     const float *edge, int32_t bcap, int32_t query_heads, int32_t kv_heads,
                                     int32_t head_dim, int32_t max_splits, int32_t span_units, int32_t dtype,
                                     void *stream) {
    if (bcap <= 0 || query_heads <= 0 || kv_heads <= 0 || query_heads % kv_heads || max_splits <= 0 ||
        span_units <= 0 || span_units % span::kWaves)
        return einval("merge_splits_span: bad geometry");
    if (head_dim != span::kD || query_heads / kv_heads > span::kHeads)
        return einval("merge_splits_span: head_dim %d / group %d outside the span schedule", head_dim,
                      query_heads / kv_heads);
    if (!partial || !lse || !counts || !error || !out || !tile_prefix || !chunk || !edge)
        return einval("merge_splits_span: null buffer");
    if ((reinterpret_cast<uintptr_t>(partial) | reinterpret_cast<uintptr_t>(edge)) & 15)
        return einval("merge_splits_span: partial / edge not 16B aligned");
    if (dtype != SGD_BF16 && dtype != SGD_FP16) return einval("merge_splits_span: dtype %d", dtype);
    clear_stale_error();
    const dim3 grid(bcap, (query_heads + kMergeWaves - 1) / kMergeWaves), block(64 * kMergeWaves);
    auto *o = static_cast<uint16_t *>(out);
    if (dtype == SGD_BF16)
        hipLaunchKernelGGL(k_merge_span<SGD_BF16>, grid, block, 0, (hipStream_t)stream, partial, lse, counts,
                           error, o, tile_prefix, chunk, edge, bcap, query_heads, kv_heads, max_splits, span_units);
    else
        hipLaunchKernelGGL(k_merge_span<SGD_FP16>, grid, block, 0, (hipStream_t)stream, partial, lse, counts,
                           error, o, tile_prefix, chunk, edge, bcap, query_heads, kv_heads, max_splits, span_units);
    return launch_status("merge_splits_span");
}
