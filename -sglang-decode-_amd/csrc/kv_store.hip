// The decode step's writes around the attention, in one launch: the new tokens' K and
// V rows into the layer's KV pool at their cache slots (what the reference adapter's
// token_to_kv_pool.set_kv_buffer does, integrations/sglang_backend.py:91-92) and the
// step's q rows into the engine's stable per-layer query buffer (the qbuf.copy_ of
// :102-103).  Upstream these are three device operations per layer (two scatters and
// a copy); here one workgroup per token moves its 2 x Hkv x D + Hq x D 16-bit values
// as 16-byte vector copies.
//
// The data is copied bit for bit (no dtype conversion); K/V rows go to the pool with
// ordinary stores (the next step's attention reads them), q rows likewise.  A slot
// outside [0, cache_tokens) is skipped: a kernel cannot raise the way torch's
// index_put does, so the host checks what it can and the device never writes out of
// bounds.
#include "common.h"

namespace sgd {
namespace {

constexpr int kStoreThreads = 256;

struct StoreArgs {
    const char *k_new, *v_new;   // [batch, Hkv, D] (may be null: no KV write)
    char *k_cache, *v_cache;     // [cache_tokens, Hkv, D]
    const void *loc;             // [batch] slot per token, int32 or int64
    const char *q_in;            // [batch, Hq, D] (may be null: no q staging)
    char *q_out;                 // [>= batch, Hq, D]
    int64_t kn[2], vn[2], kc[2], vc[2], qi[2], qo[2];  // byte strides of dims 0 and 1
    int64_t cache_tokens;
    int32_t batch, hkv, hq, chunks;  // chunks: 16-byte pieces per (token, head) row
    int32_t loc64;
};

__device__ __forceinline__ void copy16(char *dst, const char *src) {
    *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
}

__global__ __launch_bounds__(kStoreThreads) void k_store_kv_stage_q(StoreArgs a) {
    const int32_t b = blockIdx.x;
    const int32_t kv_pieces = a.k_new ? a.hkv * a.chunks : 0;
    const int32_t q_pieces = a.q_in ? a.hq * a.chunks : 0;
    int64_t slot = -1;
    if (kv_pieces) {
        slot = a.loc64 ? static_cast<const int64_t *>(a.loc)[b] : static_cast<const int32_t *>(a.loc)[b];
        if (slot < 0 || slot >= a.cache_tokens) slot = -1;
    }
    // pieces [0, kv) are K rows, [kv, 2 kv) V rows, then q rows; piece = (head, chunk)
    for (int32_t p = threadIdx.x; p < 2 * kv_pieces + q_pieces; p += kStoreThreads) {
        if (p < 2 * kv_pieces) {
            if (slot < 0) continue;
            const bool is_v = p >= kv_pieces;
            const int32_t r = is_v ? p - kv_pieces : p;
            const int32_t h = r / a.chunks, c = r - h * a.chunks;
            const int64_t *ns = is_v ? a.vn : a.kn, *cs = is_v ? a.vc : a.kc;
            const char *src = (is_v ? a.v_new : a.k_new) + b * ns[0] + h * ns[1] + c * 16;
            char *dst = (is_v ? a.v_cache : a.k_cache) + slot * cs[0] + h * cs[1] + c * 16;
            copy16(dst, src);
        } else {
            const int32_t r = p - 2 * kv_pieces;
            const int32_t h = r / a.chunks, c = r - h * a.chunks;
            copy16(a.q_out + b * a.qo[0] + h * a.qo[1] + c * 16, a.q_in + b * a.qi[0] + h * a.qi[1] + c * 16);
        }
    }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_store_kv_stage_q(const void *k_new, const void *v_new, const int64_t *new_strides,
                                    const void *loc, int32_t loc_is_int64, void *k_cache, void *v_cache,
                                    const int64_t *cache_strides, int64_t cache_tokens, const void *q_in,
                                    const int64_t *q_in_strides, void *q_out, const int64_t *q_out_strides,
                                    int32_t batch, int32_t kv_heads, int32_t query_heads, int32_t head_dim,
                                    int32_t dtype, void *stream) {
    if (dtype != SGD_BF16 && dtype != SGD_FP16) return einval("store_kv_stage_q: dtype %d", dtype);
    if (batch < 0 || kv_heads <= 0 || query_heads <= 0 || (head_dim * 2) % 16 != 0 || head_dim <= 0)
        return einval("store_kv_stage_q: batch %d, heads %d/%d, head_dim %d", batch, query_heads, kv_heads,
                      head_dim);
    const bool kv = k_new != nullptr, q = q_in != nullptr;
    if (kv && (!v_new || !new_strides || !loc || !k_cache || !v_cache || !cache_strides || cache_tokens <= 0))
        return einval("store_kv_stage_q: KV write needs k/v, their strides, loc and both caches");
    if (q && (!q_out || !q_in_strides || !q_out_strides))
        return einval("store_kv_stage_q: q staging needs q_in, q_out and their strides");
    StoreArgs a{};
    a.batch = batch;
    a.hkv = kv_heads;
    a.hq = query_heads;
    a.chunks = head_dim * 2 / 16;
    a.loc64 = loc_is_int64 != 0;
    a.cache_tokens = cache_tokens;
    // element strides (dims 0, 1; dim 2 has unit stride) -> byte strides, 16-byte aligned
    auto bytes = [](const int64_t *s, int64_t *out) {
        out[0] = s[0] * 2;
        out[1] = s[1] * 2;
        return (out[0] % 16) == 0 && (out[1] % 16) == 0 && s[0] >= 0 && s[1] >= 0;
    };
    if (kv) {
        a.k_new = static_cast<const char *>(k_new);
        a.v_new = static_cast<const char *>(v_new);
        a.k_cache = static_cast<char *>(k_cache);
        a.v_cache = static_cast<char *>(v_cache);
        a.loc = loc;
        if (!bytes(new_strides, a.kn) || !bytes(new_strides + 2, a.vn) || !bytes(cache_strides, a.kc) ||
            !bytes(cache_strides + 2, a.vc))
            return einval("store_kv_stage_q: K/V strides must be non-negative multiples of 8 elements");
        if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_cache) || !aligned16(v_cache))
            return einval("store_kv_stage_q: K/V rows must be 16-byte aligned");
    }
    if (q) {
        a.q_in = static_cast<const char *>(q_in);
        a.q_out = static_cast<char *>(q_out);
        if (!bytes(q_in_strides, a.qi) || !bytes(q_out_strides, a.qo))
            return einval("store_kv_stage_q: q strides must be non-negative multiples of 8 elements");
        if (!aligned16(q_in) || !aligned16(q_out)) return einval("store_kv_stage_q: q rows must be 16-byte aligned");
    }
    if (batch == 0 || (!kv && !q)) return 0;
    clear_stale_error();
    hipLaunchKernelGGL(k_store_kv_stage_q, dim3(batch), dim3(kStoreThreads), 0, (hipStream_t)stream, a);
    return launch_status("store_kv_stage_q");
}
