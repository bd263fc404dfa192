// sgd_persistent_decode: host-side validation of one attention launch and the
// choice of kernel.  Geometry and layout checks happen here, before any launch,
// so a bad argument is an SGD_EINVAL and never a device fault.
#include "attention_common.h"

namespace sgd {
int launch_attention_generic(const sgd_decode_args &a, bool vec, hipStream_t stream);
int launch_attention_valu(const sgd_decode_args &a, hipStream_t stream);
int launch_attention_mfma(const sgd_decode_args &a, hipStream_t stream);
bool valu_supported(const sgd_decode_args &a);
bool mfma_supported(const sgd_decode_args &a);
}

using namespace sgd;

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 16-byte vector loads need unit head_dim stride and 16-byte aligned rows.
bool vector_layout(const sgd_decode_args &a) {
    if (a.k_stride[3] != 1 || a.v_stride[3] != 1) return false;
    if (!aligned16(a.k) || !aligned16(a.v)) return false;
    for (int i = 0; i < 3; ++i)
        if (a.k_stride[i] % 8 != 0 || a.v_stride[i] % 8 != 0) return false;
    return true;
}

}  // namespace

namespace {

// Host checks of the launch geometry; SGD_EINVAL (with the reason) or 0.
int check_args(const sgd_decode_args *args) {
    if (!args) return einval("persistent_decode: null args");
    const sgd_decode_args &a = *args;
    if (a.kv_heads <= 0 || a.query_heads <= 0 || a.query_heads % a.kv_heads != 0)
        return einval("persistent_decode: heads %d/%d", a.query_heads, a.kv_heads);
    const int g = a.query_heads / a.kv_heads;
    if (g != 1 && g != 2 && g != 4 && g != 8 && g != 16) return einval("persistent_decode: group %d", g);
    if (a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256)
        return einval("persistent_decode: head_dim %d", a.head_dim);
    if (a.dtype != SGD_BF16 && a.dtype != SGD_FP16) return einval("persistent_decode: dtype %d", a.dtype);
    if (a.workers <= 0 || a.max_splits <= 0 || a.page_size <= 0)
        return einval("persistent_decode: workers/max_splits/page_size");
    if (a.csr && (a.page_size != 1 || !a.indptr)) return einval("persistent_decode: CSR needs page_size 1 + indptr");
    if (!a.q || !a.k || !a.v || !a.pages || !a.partial || !a.lse || !a.counter)
        return einval("persistent_decode: null buffer");
    if (a.dispatch && a.dispatch_units < 0)
        return einval("persistent_decode: dispatch_units %d < 0", a.dispatch_units);
    if (a.out && (reinterpret_cast<uintptr_t>(a.out) & 1)) return einval("persistent_decode: out not 2-byte aligned");
    return 0;
}

// The kernel a launch with these arguments runs (enum sgd_kernel), or SGD_EINVAL.
int resolve_kernel(const sgd_decode_args &a) {
    switch (a.kernel) {
        case SGD_KERNEL_AUTO:
            // The VALU kernel for groups <= 4 (1-2% faster than the MFMA kernel, whose 16
            // MFMA columns are then three-quarters padding, on the Llama-3-8B layers
            // measured), else the MFMA one (groups up to 16), else the generic kernel.
            // All three merge a task's wave states in a fixed order, so a launch is
            // bitwise repeatable whatever the worker count.
            if (valu_supported(a)) return SGD_KERNEL_VALU;
            if (mfma_supported(a)) return SGD_KERNEL_MFMA;
            return SGD_KERNEL_GENERIC;
        case SGD_KERNEL_GENERIC:
            return SGD_KERNEL_GENERIC;
        case SGD_KERNEL_VALU:
            if (!valu_supported(a))
                return einval("persistent_decode: the VALU kernel needs group <= 4, head_dim 64/128/256, unit dim "
                              "stride and 16-byte aligned rows");
            return SGD_KERNEL_VALU;
        case SGD_KERNEL_MFMA:
            if (!mfma_supported(a))
                return einval("persistent_decode: the MFMA kernel needs group <= 16, head_dim 64/128/256, unit dim "
                              "stride and 16-byte aligned rows");
            return SGD_KERNEL_MFMA;
        default:
            return einval("persistent_decode: kernel %d not available", a.kernel);
    }
}

}  // namespace

extern "C" int sgd_attention_kernel(const sgd_decode_args *args) {
    if (int rc = check_args(args)) return rc;
    return resolve_kernel(*args);
}

extern "C" int sgd_persistent_decode(const sgd_decode_args *args, void *stream) {
    if (int rc = check_args(args)) return rc;
    const sgd_decode_args &a = *args;
    const int kernel = resolve_kernel(a);
    if (kernel < 0) return kernel;
    clear_stale_error();
    switch (kernel) {
        case SGD_KERNEL_VALU:
            return launch_attention_valu(a, (hipStream_t)stream);
        case SGD_KERNEL_MFMA:
            return launch_attention_mfma(a, (hipStream_t)stream);
        default:
            return launch_attention_generic(a, vector_layout(a), (hipStream_t)stream);
    }
}
