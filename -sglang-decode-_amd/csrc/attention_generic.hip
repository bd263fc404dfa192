// Generic persistent paged GQA decode attention: any element strides (including
// a non-unit head_dim stride), any 16-bit dtype, head_dim 64/128/256, group 1..16,
// paged or CSR.  It is the fallback for layouts the tuned kernels do not take and
// the cross-check for them.
//
// Per task (record, kv head), kernels/attention.py:48-84: the group's q rows are
// staged in LDS as fp32; each of the 4 waves takes 64-token tiles of the split in
// turn (wave w: tokens start + 64w + 256i + lane).  A lane scores its own token for
// every head of the group; the wave reduces the tile max/sum with shuffles, keeps
// fp32 online-softmax state per head, rounds p to the KV dtype for P.V like
// kernels/attention.py:78, and accumulates P.V with lanes owning head_dim/64
// consecutive dims.  The four waves' states are merged through LDS and the
// normalized partial + natural-log LSE go to slot (request, head, split).
#include "attention_common.h"

namespace sgd {
namespace {

constexpr int kWaves = 4;

template <int GP, int D>
struct GenericShared {
    float q[GP][D];
    float p[kWaves][GP][64];
    int64_t vrow[kWaves][64];
    float cacc[kWaves][D];
    float cm[kWaves], cd[kWaves];
    int32_t cursor;
};

template <int DT, int GP, int D, bool VEC>
__global__ __launch_bounds__(64 * kWaves) void k_attention_generic(sgd_decode_args a) {
    constexpr int DPL = D / 64;
    __shared__ GenericShared<GP, D> sh;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int32_t G = a.query_heads / a.kv_heads;
    const uint16_t *__restrict__ q16 = static_cast<const uint16_t *>(a.q);
    const uint16_t *__restrict__ k16 = static_cast<const uint16_t *>(a.k);
    const uint16_t *__restrict__ v16 = static_cast<const uint16_t *>(a.v);
    const int64_t KP = a.k_stride[0], KT = a.k_stride[1], KH = a.k_stride[2], KD = a.k_stride[3];
    const int64_t VP = a.v_stride[0], VT = a.v_stride[1], VH = a.v_stride[2], VD = a.v_stride[3];

    for_each_task(a, &sh.cursor, [&](int32_t, const TaskInfo &t) {
        __syncthreads();  // previous task is done with the shared buffers
        for (int i = threadIdx.x; i < GP * D; i += 64 * kWaves) {
            const int j = i / D, d = i % D;
            float qv = 0.f;
            if (j < G) {
                const int64_t off = (int64_t)t.request * a.q_stride[0] + (int64_t)(t.group * G + j) * a.q_stride[1] +
                                    (int64_t)d * a.q_stride[2];
                qv = to_f32<DT>(q16[off]);
            }
            sh.q[j][d] = qv;
        }
        __syncthreads();
        const int32_t length = a.lengths[t.request];
        // a request's first split also writes its rows to `out` (final for a single-split
        // request, overwritten by the merge otherwise)
        const bool first = a.out != nullptr && t.split == 0;
        float m[GP], den[GP], acc[GP][DPL];
#pragma unroll
        for (int j = 0; j < GP; ++j) {
            m[j] = -INFINITY;
            den[j] = 0.f;
#pragma unroll
            for (int i = 0; i < DPL; ++i) acc[j][i] = 0.f;
        }
        for (int32_t base = t.start + wave * 64; base < t.end; base += 64 * kWaves) {
            const int32_t tok = base + lane;
            const bool live = tok < t.end && tok < length;
            int64_t krow = 0, vrow = -1;
            if (live) {
                int64_t phys, inner;
                if (a.csr) {
                    phys = a.pages[a.indptr[t.request] + tok];
                    inner = 0;
                } else {
                    phys = a.pages[(int64_t)t.request * a.pt_stride[0] + (int64_t)(tok / a.page_size) * a.pt_stride[1]];
                    inner = tok % a.page_size;
                }
                krow = phys * KP + inner * KT + (int64_t)t.group * KH;
                vrow = phys * VP + inner * VT + (int64_t)t.group * VH;
            }
            float s[GP];
#pragma unroll
            for (int j = 0; j < GP; ++j) s[j] = 0.f;
            if (live) {
                if constexpr (VEC) {
                    const uint4 *kp = reinterpret_cast<const uint4 *>(k16 + krow);
                    for (int c = 0; c < D / 8; ++c) {
                        const uint4 raw = kp[c];
                        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
                        float kv[8];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            kv[2 * e] = to_f32<DT>(w[e] & 0xffffu);
                            kv[2 * e + 1] = to_f32<DT>(w[e] >> 16);
                        }
#pragma unroll
                        for (int j = 0; j < GP; ++j) {
#pragma unroll
                            for (int e = 0; e < 8; ++e) s[j] += sh.q[j][c * 8 + e] * kv[e];
                        }
                    }
                } else {
                    for (int d = 0; d < D; ++d) {
                        const float kv = to_f32<DT>(k16[krow + d * KD]);
#pragma unroll
                        for (int j = 0; j < GP; ++j) s[j] += sh.q[j][d] * kv;
                    }
                }
            }
            sh.vrow[wave][lane] = vrow;
#pragma unroll
            for (int j = 0; j < GP; ++j) {
                if (j >= G) break;
                const float sj = live ? s[j] * a.scale : -INFINITY;
                const float nm = fmaxf(m[j], wave_max(sj));
                const float alpha = __expf(m[j] - nm);
                const float p = live ? __expf(sj - nm) : 0.f;
                den[j] = den[j] * alpha + wave_sum(p);
#pragma unroll
                for (int i = 0; i < DPL; ++i) acc[j][i] *= alpha;
                m[j] = nm;
                sh.p[wave][j][lane] = round_to<DT>(p);
            }
            wave_sync();
            const int nlive = min(64, min(t.end, length) - base);
            for (int u = 0; u < nlive; ++u) {
                const int64_t vr = sh.vrow[wave][u];
                float vv[DPL];
                if constexpr (VEC) {
                    const uint16_t *src = v16 + vr + lane * DPL;
                    if constexpr (DPL == 1) {
                        vv[0] = to_f32<DT>(src[0]);
                    } else if constexpr (DPL == 2) {
                        const uint32_t w = *reinterpret_cast<const uint32_t *>(src);
                        vv[0] = to_f32<DT>(w & 0xffffu);
                        vv[1] = to_f32<DT>(w >> 16);
                    } else {
                        const uint2 w = *reinterpret_cast<const uint2 *>(src);
                        vv[0] = to_f32<DT>(w.x & 0xffffu);
                        vv[1] = to_f32<DT>(w.x >> 16);
                        vv[2] = to_f32<DT>(w.y & 0xffffu);
                        vv[3] = to_f32<DT>(w.y >> 16);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < DPL; ++i) vv[i] = to_f32<DT>(v16[vr + (int64_t)(lane * DPL + i) * VD]);
                }
#pragma unroll
                for (int j = 0; j < GP; ++j) {
                    if (j >= G) break;
                    const float pj = sh.p[wave][j][u];
#pragma unroll
                    for (int i = 0; i < DPL; ++i) acc[j][i] += pj * vv[i];
                }
            }
            wave_sync();
        }
        // Merge the four waves' online-softmax states, one head at a time.
#pragma unroll
        for (int j = 0; j < GP; ++j) {
            if (j >= G) break;
            __syncthreads();
            if (lane == 0) {
                sh.cm[wave] = m[j];
                sh.cd[wave] = den[j];
            }
#pragma unroll
            for (int i = 0; i < DPL; ++i) sh.cacc[wave][lane * DPL + i] = acc[j][i];
            __syncthreads();
            float mm = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sh.cm[w]);
            float dd = 0.f, sc[kWaves];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                sc[w] = __expf(sh.cm[w] - mm);
                dd += sh.cd[w] * sc[w];
            }
            const int64_t slot = ((int64_t)t.request * a.query_heads + t.group * G + j) * a.max_splits + t.split;
            for (int d = threadIdx.x; d < D; d += 64 * kWaves) {
                float x = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) x += sh.cacc[w][d] * sc[w];
                a.partial[slot * D + d] = x / dd;
                if (first)
                    static_cast<uint16_t *>(a.out)[((int64_t)t.request * a.query_heads + t.group * G + j) * D + d] =
                        (uint16_t)from_f32<DT>(x / dd);
            }
            if (threadIdx.x == 0) a.lse[slot] = mm + __logf(dd);
        }
    });
}

template <int DT, int GP, int D>
int launch_generic_vec(const sgd_decode_args &a, bool vec, hipStream_t stream) {
    const dim3 grid(a.workers), block(64 * kWaves);
    if (vec) hipLaunchKernelGGL((k_attention_generic<DT, GP, D, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_attention_generic<DT, GP, D, false>), grid, block, 0, stream, a);
    return launch_status("persistent_decode(generic)");
}

template <int DT, int GP>
int launch_generic_d(const sgd_decode_args &a, bool vec, hipStream_t stream) {
    switch (a.head_dim) {
        case 64: return launch_generic_vec<DT, GP, 64>(a, vec, stream);
        case 128: return launch_generic_vec<DT, GP, 128>(a, vec, stream);
        case 256: return launch_generic_vec<DT, GP, 256>(a, vec, stream);
    }
    return einval("head_dim %d", a.head_dim);
}

template <int DT>
int launch_generic_g(const sgd_decode_args &a, bool vec, hipStream_t stream) {
    const int g = a.query_heads / a.kv_heads;
    if (g <= 1) return launch_generic_d<DT, 1>(a, vec, stream);
    if (g <= 2) return launch_generic_d<DT, 2>(a, vec, stream);
    if (g <= 4) return launch_generic_d<DT, 4>(a, vec, stream);
    if (g <= 8) return launch_generic_d<DT, 8>(a, vec, stream);
    return launch_generic_d<DT, 16>(a, vec, stream);
}

}  // namespace

int launch_attention_generic(const sgd_decode_args &a, bool vec, hipStream_t stream) {
    if (a.dtype == SGD_BF16) return launch_generic_g<SGD_BF16>(a, vec, stream);
    return launch_generic_g<SGD_FP16>(a, vec, stream);
}

}  // namespace sgd
