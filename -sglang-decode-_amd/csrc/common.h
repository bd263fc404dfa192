// Shared helpers of the gfx950 decode-attention library: error reporting for the
// C ABI, 16-bit float conversions and workgroup-level scans/reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sglang_decode_hip.h"

namespace sgd {

// ------------------------------------------------------------------ host side

void set_error(const char *fmt, ...);
int einval(const char *fmt, ...);
// Clears a stale error, checks the launch just issued and maps it to the ABI code.
int launch_status(const char *what);
void clear_stale_error();

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once per device:
// `done` is the kernel's flag array (kOnceDevices entries, zero-initialised); devices past
// it are set on every call.  SGD_EINVAL naming `what` if the runtime refuses.
constexpr int kOnceDevices = 64;
int set_dynamic_lds(const void *kernel, int bytes, bool *done, const char *what);

// ------------------------------------------------------------------ device side

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN, quiet).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}

__device__ __forceinline__ uint32_t f32_to_f16(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

template <int DT>
__device__ __forceinline__ float to_f32(uint32_t bits16) {
    if constexpr (DT == SGD_BF16) return bf16_to_f32(bits16);
    else return f16_to_f32(bits16);
}

template <int DT>
__device__ __forceinline__ uint32_t from_f32(float f) {
    if constexpr (DT == SGD_BF16) return f32_to_bf16(f);
    else return f32_to_f16(f);
}

// 16-byte load of KV-cache data that a launch reads exactly once.  The nontemporal
// hint (the `nt` bit) streams the line through L2 and the Infinity Cache instead of
// keeping it there; on random 256 B row gathers over 2 GiB pools it raises the
// chip-wide rate from ~5.8 to ~6.6 TB/s.
__device__ __forceinline__ uint4 load_stream16(const void *p) {
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// Round an fp32 value through the 16-bit storage type (the reference casts the
// softmax probabilities to the KV dtype before P.V, kernels/attention.py:78).
template <int DT>
__device__ __forceinline__ float round_to(float f) {
    return to_f32<DT>(from_f32<DT>(f));
}

// Workgroup barrier that orders LDS only: unlike __syncthreads() it does not wait for
// the waves' outstanding global loads and stores (prefetches stay in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Inclusive scan over the 64 lanes of a wave.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        T u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    return v;
}

// Exclusive scan over the whole workgroup (blockDim.x a multiple of 64, <= 1024).
// `tmp` must hold 16 T in LDS.  Returns the exclusive prefix; *total = block sum.
template <typename T>
__device__ T block_exclusive_scan(T v, T *tmp, T *total) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    T inc = wave_inclusive_scan(v);
    lds_barrier();
    if (lane == 63) tmp[wid] = inc;
    lds_barrier();
    T base = 0, sum = 0;
    for (int w = 0; w < nw; ++w) {
        T t = tmp[w];
        if (w < wid) base += t;
        sum += t;
    }
    *total = sum;
    return base + inc - v;
}

}  // namespace sgd
