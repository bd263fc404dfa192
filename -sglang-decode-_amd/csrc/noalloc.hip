// sgd_decode_noalloc: one decode step (plan build, persistent attention, split merge)
// that allocates nothing.  The plan tables, the dispatch table, the claim counters and
// the split partial/LSE slots live in `scratch`, a file-scope device array of
// kScratchBytes; the caller passes only the inputs and the output.
//
// In host code `scratch` names a host-side stand-in, not device memory: its device
// address is taken once per device with hipGetSymbolAddress (with that device current)
// and only that address is used from then on -- as the kernels' buffer arguments.  Each
// GPU holds its own copy of the array until the process ends.
//
// Every call on one GPU shares that GPU's array and leaves the last call's contents
// there; the plan launch clears the claim counters, which are the only words that
// must start at zero (the plan rewrites every table entry the attention reads, and the
// attention writes every split slot the merge reads).  Calls that overlap on one GPU
// (two streams, two threads) race on the array.
#include <mutex>

#include "common.h"

namespace sgd {
int merge_rows_resident();  // merge.hip

namespace {

constexpr size_t kScratchBytes = size_t(32) << 20;
constexpr size_t kAlign = 256;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
unsigned char *g_scratch[kMaxDevices] = {};

// Device address of the current device's scratch array (found once per device), or
// nullptr with the error text set.
unsigned char *device_scratch() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("decode_noalloc: no current device (or device index >= %d)", kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("decode_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                      hipGetErrorString(e));
            return nullptr;
        }
        g_scratch[dev] = static_cast<unsigned char *>(p);
    }
    return g_scratch[dev];
}

// Offsets of the step's buffers inside the scratch array, each kAlign-aligned.
struct Layout {
    size_t counts, offsets, chunk, request, split, begin, end, weight, order, pack_first, pack_count,
        static_head, static_next, scalars, rules, dispatch, sync, partial, lse, total;
};

Layout layout_for(int64_t bcap, int64_t smax, int64_t hkv, int64_t hq, int64_t d, int64_t workers) {
    Layout L{};
    size_t at = 0;
    auto take = [&](int64_t bytes) {
        const size_t o = at;
        at += ((size_t)bytes + kAlign - 1) / kAlign * kAlign;
        return o;
    };
    const int64_t e = bcap * smax, t = e * hkv;
    L.counts = take(4 * bcap);
    L.offsets = take(4 * (bcap + 1));
    L.chunk = take(4 * bcap);
    L.request = take(4 * e);
    L.split = take(4 * e);
    L.begin = take(4 * e);
    L.end = take(4 * e);
    L.weight = take(4 * e);
    L.order = take(4 * e);
    L.pack_first = take(4 * t);
    L.pack_count = take(4 * t);
    L.static_head = take(4 * workers);
    L.static_next = take(4 * t);
    L.scalars = take(4 * 4);  // record_count, num_packs, mode, error
    L.rules = take(4 * 5);    // one unused rule row (rule_count 0)
    L.dispatch = take(4 * 8 * t);
    L.sync = take(4 * 2);     // claim counter, finished workers
    L.partial = take(4 * bcap * hq * smax * d);
    L.lse = take(4 * bcap * hq * smax);
    L.total = at;
    return L;
}

int32_t buckets_for(int32_t max_context, int32_t block_kv) {
    const int32_t tiles = (max_context + block_kv - 1) / block_kv - 1;
    int32_t bits = 0;
    for (int32_t v = tiles; v > 0; v >>= 1) ++bits;
    return bits + 1;
}

}  // namespace
}  // namespace sgd

using namespace sgd;

extern "C" int sgd_decode_noalloc(const sgd_noalloc_args *args, void *stream) {
    if (!args) return einval("decode_noalloc: null args");
    const sgd_noalloc_args &a = *args;
    if (!a.q || !a.k || !a.v || !a.pages || !a.lengths || !a.splits || !a.active || !a.out)
        return einval("decode_noalloc: null buffer");
    if (a.batch_capacity <= 0 || a.max_splits <= 0 || a.max_context <= 0 || a.query_heads <= 0 ||
        a.kv_heads <= 0 || a.head_dim <= 0 || a.workers <= 0)
        return einval("decode_noalloc: capacities, heads, head_dim and workers must be positive");
    // bounds that keep the size arithmetic below exact (the plan and attention entries
    // check the geometry in full)
    if (a.batch_capacity > 4096 || (int64_t)a.batch_capacity * a.max_splits > 16384 || a.query_heads > 4096 ||
        a.kv_heads > a.query_heads || a.head_dim > 256 || a.workers > 4096)
        return einval("decode_noalloc: batch_capacity %d, max_splits %d, heads %d/%d, head_dim %d or workers %d "
                      "beyond the planner's bounds", a.batch_capacity, a.max_splits, a.query_heads, a.kv_heads,
                      a.head_dim, a.workers);
    constexpr int32_t kBlockKv = 128;
    const Layout L = layout_for(a.batch_capacity, a.max_splits, a.kv_heads, a.query_heads, a.head_dim, a.workers);
    if (L.total > kScratchBytes)
        return einval("decode_noalloc: batch_capacity %d x max_splits %d x %d q heads x head_dim %d needs %zu bytes "
                      "of scratch; the library holds %zu (use sgd_build_plan / sgd_persistent_decode / "
                      "sgd_merge_splits with caller-allocated buffers)",
                      a.batch_capacity, a.max_splits, a.query_heads, a.head_dim, L.total, kScratchBytes);
    unsigned char *base = device_scratch();
    if (!base) return SGD_EINVAL;
    auto i32 = [&](size_t off) { return reinterpret_cast<int32_t *>(base + off); };
    int32_t *scalars = i32(L.scalars), *sync = i32(L.sync);

    sgd_plan_buffers p{};
    p.lengths = const_cast<int32_t *>(a.lengths);  // read, never written, by sgd_build_plan
    p.splits = const_cast<int32_t *>(a.splits);
    p.active = const_cast<int32_t *>(a.active);
    p.counts = i32(L.counts);
    p.offsets = i32(L.offsets);
    p.chunk = i32(L.chunk);
    p.request = i32(L.request);
    p.split = i32(L.split);
    p.begin = i32(L.begin);
    p.end = i32(L.end);
    p.weight = i32(L.weight);
    p.order = i32(L.order);
    p.pack_first = i32(L.pack_first);
    p.pack_count = i32(L.pack_count);
    p.record_count = scalars;
    p.num_packs = scalars + 1;
    p.mode = scalars + 2;
    p.error = scalars + 3;
    p.static_head = i32(L.static_head);
    p.static_next = i32(L.static_next);
    p.rules = i32(L.rules);
    p.dispatch = i32(L.dispatch);
    p.rule_count = 0;
    p.batch_capacity = a.batch_capacity;
    p.max_splits = a.max_splits;
    p.max_context = a.max_context;
    p.kv_heads = a.kv_heads;
    p.workers = a.workers;
    p.block_kv = kBlockKv;
    p.buckets = buckets_for(a.max_context, kBlockKv);
    sgd_decode_args d{};
    d.q = a.q;
    d.k = a.k;
    d.v = a.v;
    d.pages = a.pages;
    d.indptr = a.indptr;
    d.lengths = a.lengths;
    d.request = p.request;
    d.split = p.split;
    d.begin = p.begin;
    d.end = p.end;
    d.order = p.order;
    d.offsets = p.offsets;
    d.chunk = p.chunk;
    d.active = a.active;
    d.record_count = p.record_count;
    d.mode = p.mode;
    d.pack_first = p.pack_first;
    d.pack_count = p.pack_count;
    d.num_packs = p.num_packs;
    d.counter = sync;
    d.done_counter = sync + 1;
    d.static_head = p.static_head;
    d.static_next = p.static_next;
    d.partial = reinterpret_cast<float *>(base + L.partial);
    d.lse = reinterpret_cast<float *>(base + L.lse);
    d.dispatch = p.dispatch;
    d.dispatch_units = a.batch_capacity * a.max_splits * a.kv_heads;
    d.scale = a.scale;
    for (int i = 0; i < 3; ++i) d.q_stride[i] = a.q_stride[i];
    for (int i = 0; i < 4; ++i) d.k_stride[i] = a.k_stride[i];
    for (int i = 0; i < 4; ++i) d.v_stride[i] = a.v_stride[i];
    for (int i = 0; i < 2; ++i) d.pt_stride[i] = a.pt_stride[i];
    d.query_heads = a.query_heads;
    d.kv_heads = a.kv_heads;
    d.head_dim = a.head_dim;
    d.max_splits = a.max_splits;
    d.page_size = a.page_size;
    d.csr = a.csr;
    d.dtype = a.dtype;
    d.workers = a.workers;
    d.kernel = a.kernel;
    // Beyond one residency round of merge rows, each request's first split also writes
    // its rows and the merge takes only the multi-split ones (as DecodeEngine does).
    const bool direct = (int64_t)a.batch_capacity * a.query_heads > merge_rows_resident();
    d.out = direct ? a.out : nullptr;
    // Every refusal happens before the first device call: the attention's geometry and
    // kernel checks (the plan entry checks its own arguments before it launches).
    if (const int rc = sgd_attention_kernel(&d); rc < 0) return rc;
    if (int rc = sgd_build_plan(&p, a.force_mode, a.force_mode == 2, sync, 2, stream)) return rc;
    if (int rc = sgd_persistent_decode(&d, stream)) return rc;
    return sgd_merge_splits_min(d.partial, d.lse, p.counts, a.active, p.error, a.out, a.batch_capacity,
                                a.query_heads, a.head_dim, a.max_splits, direct ? 2 : 1, a.dtype, stream);
}
