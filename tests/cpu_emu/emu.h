// CPU executor for the library's HIP kernels (test infrastructure, never shipped).
//
// The kernel sources under -sglang-decode-_amd/csrc are compiled as host C++ against
// this header (through include/hip/hip_runtime.h).  Every thread of a workgroup runs
// as a fiber on one OS thread; workgroups run one after another.  A fiber runs until it
// reaches a meeting point:
//   * a cross-lane operation (shuffles, readlane/readfirstlane, ballot, DPP moves,
//     wave barriers, MFMA): the wave's op is evaluated once every live lane of the wave
//     has stopped, over the lanes that reached it (the active lanes);
//   * a workgroup barrier: released when every live thread of the workgroup is there;
//   * s_sleep: the fiber yields, so spin-waits let the other waves progress.
// Memory is ordinary host memory, so the tests run the executor under AddressSanitizer:
// an access outside a buffer, the dynamic LDS block or a static LDS array is reported
// with the kernel, workgroup and thread that made it.
//
// Cross-lane semantics follow the wave64 definitions the kernels are written for:
// DPP quad_perm / row_shl / row_shr / row_ror / row_mirror / row_half_mirror /
// row_newbcast with bound_ctrl, HIP's __shfl / __shfl_xor / __shfl_up, and
// v_mfma_f32_16x16x32_{bf16,f16} with lane l = (l % 16, l / 16) holding A[m][8j..8j+7],
// B[8j..8j+7][n] and D[4j..4j+3][n].  Reading an inactive lane is reported as an error.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <tuple>
#include <type_traits>
#include <utility>

// ------------------------------------------------------------------ HIP keywords
#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
// The sources cast pointers into the constant address space (scalar loads); on the CPU
// that attribute is dropped: `__attribute__((address_space(4)))` becomes `__attribute__(())`.
#define address_space(n)

#define __HIP_MEMORY_SCOPE_SINGLETHREAD 1
#define __HIP_MEMORY_SCOPE_WAVEFRONT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __HIP_MEMORY_SCOPE_SYSTEM 5

// ------------------------------------------------------------------ vector types
struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned x_ = 1, unsigned y_ = 1, unsigned z_ = 1) : x(x_), y(y_), z(z_) {}
};
struct alignas(16) uint4 { unsigned x, y, z, w; };
struct alignas(16) int4 { int x, y, z, w; };
struct alignas(16) float4 { float x, y, z, w; };
struct alignas(8) uint2 { unsigned x, y; };
struct alignas(8) int2 { int x, y; };
struct alignas(8) float2 { float x, y; };
inline uint4 make_uint4(unsigned x, unsigned y, unsigned z, unsigned w) { return uint4{x, y, z, w}; }
inline int4 make_int4(int x, int y, int z, int w) { return int4{x, y, z, w}; }
inline float4 make_float4(float x, float y, float z, float w) { return float4{x, y, z, w}; }
inline uint2 make_uint2(unsigned x, unsigned y) { return uint2{x, y}; }
inline int2 make_int2(int x, int y) { return int2{x, y}; }
inline float2 make_float2(float x, float y) { return float2{x, y}; }

template <class A, class B>
inline constexpr std::common_type_t<A, B> min(A a, B b) { return a < b ? a : b; }
template <class A, class B>
inline constexpr std::common_type_t<A, B> max(A a, B b) { return a < b ? b : a; }

inline float __uint_as_float(unsigned u) { float f; memcpy(&f, &u, 4); return f; }
inline unsigned __float_as_uint(float f) { unsigned u; memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; memcpy(&f, &u, 4); return f; }
inline int __float_as_int(float f) { int u; memcpy(&u, &f, 4); return u; }
inline float __expf(float x) { return expf(x); }
inline float __logf(float x) { return logf(x); }
inline float __log2f(float x) { return log2f(x); }
inline float __fdividef(float a, float b) { return a / b; }

// ------------------------------------------------------------------ executor core
namespace emu {

struct Idx3 { unsigned x, y, z; };

const Idx3 &thread_idx();
const Idx3 &block_idx();
const Idx3 &block_dim();
const Idx3 &grid_dim();

enum XKind {
    X_SHFL = 1, X_SHFL_XOR, X_SHFL_UP, X_READLANE, X_READFIRST, X_BALLOT, X_DPP, X_MFMA, X_WAVE_BARRIER
};

// One lane's part of a cross-lane operation.
struct XOp {
    int kind, line;
    int p0, p1, p2;        // source lane / xor mask / delta / DPP control; width; bound_ctrl
    uint64_t v, old, r;    // operand, DPP old value, result
    int bytes;             // operand size (4 or 8)
    uint32_t a[4], b[4];   // MFMA A and B (8 x 16-bit each)
    float c[4], d[4];      // MFMA C and D
    int dt;                // MFMA element type: 0 bf16, 1 fp16
};

void cross_lane(XOp &op);
void barrier(int line);
void sleep_yield();
void *dynamic_lds();
[[noreturn]] void fatal(const char *fmt, ...);

template <class T>
inline uint64_t bits_of(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lane values");
    uint64_t u = 0;
    memcpy(&u, &v, sizeof(T));
    return u;
}
template <class T>
inline T from_bits(uint64_t u) {
    T v;
    memcpy(&v, &u, sizeof(T));
    return v;
}

template <class T>
inline T xlane(int kind, T v, int p0, int p1, int line) {
    XOp op{};
    op.kind = kind;
    op.v = bits_of(v);
    op.bytes = sizeof(T);
    op.p0 = p0;
    op.p1 = p1;
    op.line = line;
    cross_lane(op);
    return from_bits<T>(op.r);
}

inline int readfirstlane(int v, int line) { return xlane(X_READFIRST, v, 0, 64, line); }
inline int readlane(int v, int l, int line) { return xlane(X_READLANE, v, l, 64, line); }
inline unsigned long long ballot(bool p, int line) {
    return (unsigned long long)xlane(X_BALLOT, (uint64_t)(p ? 1 : 0), 0, 64, line);
}
inline int update_dpp(int old, int src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl, int line) {
    if (row_mask != 0xf || bank_mask != 0xf) fatal("DPP row/bank masks other than 0xf are not emulated (line %d)", line);
    XOp op{};
    op.kind = X_DPP;
    op.v = (uint32_t)src;
    op.old = (uint32_t)old;
    op.bytes = 4;
    op.p0 = ctrl;
    op.p2 = bound_ctrl ? 1 : 0;
    op.line = line;
    cross_lane(op);
    return (int)(uint32_t)op.r;
}
inline void wave_barrier(int line) {
    XOp op{};
    op.kind = X_WAVE_BARRIER;
    op.bytes = 4;
    op.line = line;
    cross_lane(op);
}

template <class VA, class VC>
inline VC mfma_16x16x32(int dt, VA a, VA b, VC c, int line) {
    static_assert(sizeof(VA) == 16 && sizeof(VC) == 16, "16x16x32: 8 x 16-bit A/B, 4 x fp32 C/D");
    XOp op{};
    op.kind = X_MFMA;
    op.dt = dt;
    op.bytes = 16;
    op.p0 = 32;  // K
    op.line = line;
    memcpy(op.a, &a, 16);
    memcpy(op.b, &b, 16);
    memcpy(op.c, &c, 16);
    cross_lane(op);
    VC d;
    memcpy(&d, op.d, 16);
    return d;
}

// v_mfma_f32_16x16x16_{bf16,f16}: lane l = (l % 16, l / 16) holds A[m][4j..4j+3],
// B[4j..4j+3][n] and D[4j..4j+3][n].
template <class VA, class VC>
inline VC mfma_16x16x16(int dt, VA a, VA b, VC c, int line) {
    static_assert(sizeof(VA) == 8 && sizeof(VC) == 16, "16x16x16: 4 x 16-bit A/B, 4 x fp32 C/D");
    XOp op{};
    op.kind = X_MFMA;
    op.dt = dt;
    op.bytes = 8;
    op.p0 = 16;  // K
    op.line = line;
    memcpy(op.a, &a, 8);
    memcpy(op.b, &b, 8);
    memcpy(op.c, &c, 16);
    cross_lane(op);
    VC d;
    memcpy(&d, op.d, 16);
    return d;
}

float bf16_bits_to_f32(uint32_t h);
float f16_bits_to_f32(uint32_t h);

// v_dot2_f32_{bf16,f16}: c + a.lo * b.lo + a.hi * b.hi (products exact in fp32; one
// rounding of the sum, done here in double).
template <class V2>
inline float dot2(int dt, V2 a, V2 b, float c) {
    static_assert(sizeof(V2) == 4, "two 16-bit elements");
    uint32_t ua, ub;
    memcpy(&ua, &a, 4);
    memcpy(&ub, &b, 4);
    auto cvt = dt == 0 ? bf16_bits_to_f32 : f16_bits_to_f32;
    const double s = (double)cvt(ua & 0xffff) * cvt(ub & 0xffff) + (double)cvt(ua >> 16) * cvt(ub >> 16) + c;
    return (float)s;
}

// v_perm_b32: byte i of the result is selector byte i applied to {a, b} (b = bytes 0-3).
inline uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
    const uint64_t x = ((uint64_t)a << 32) | b;
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        const uint32_t s = (sel >> (8 * i)) & 0xff;
        uint32_t byte;
        if (s < 8) byte = (uint32_t)(x >> (8 * s)) & 0xff;
        else if (s == 12) byte = 0;
        else if (s > 12) byte = 0xff;
        else fatal("v_perm_b32 sign-extension selector %u is not emulated", s);
        r |= byte << (8 * i);
    }
    return r;
}

// ------------------------------------------------------------------ atomics (fibers never interleave inside one)
template <class T, class U>
inline T atomic_fetch_add(T *p, U v) {
    const T o = *p;
    *p = (T)(o + (T)v);
    return o;
}
template <class T>
inline T atomic_load(T *p) { return *p; }
template <class T, class U>
inline void atomic_store(T *p, U v) { *p = (T)v; }
template <class T, class U>
inline bool atomic_cas(T *p, T *expected, U desired) {
    if (*p == *expected) {
        *p = (T)desired;
        return true;
    }
    *expected = *p;
    return false;
}

// ------------------------------------------------------------------ launches
using Body = void (*)(void *);
void run_grid(const char *name, dim3 grid, dim3 block, size_t dynamic_lds, Body body, void *ctx);

template <class... P, class... A>
inline void launch(const char *name, void (*k)(P...), dim3 grid, dim3 block, size_t dyn, A &&...args) {
    using Tup = std::tuple<std::decay_t<P>...>;
    Tup t(static_cast<std::decay_t<P>>(args)...);
    struct Ctx {
        void (*k)(P...);
        Tup *t;
    } ctx{k, &t};
    run_grid(name, grid, block, dyn, [](void *p) {
        Ctx *c = static_cast<Ctx *>(p);
        std::apply(c->k, *c->t);
    }, &ctx);
}

}  // namespace emu

#define threadIdx (::emu::thread_idx())
#define blockIdx (::emu::block_idx())
#define blockDim (::emu::block_dim())
#define gridDim (::emu::grid_dim())

// ------------------------------------------------------------------ builtins
#define __shfl(v, l, w) ::emu::xlane(::emu::X_SHFL, (v), (l), (w), __LINE__)
#define __shfl_xor(v, m, w) ::emu::xlane(::emu::X_SHFL_XOR, (v), (m), (w), __LINE__)
#define __shfl_up(v, d, w) ::emu::xlane(::emu::X_SHFL_UP, (v), (d), (w), __LINE__)
#define __ballot(p) ::emu::ballot((p), __LINE__)
#define __popcll(x) __builtin_popcountll(x)
#define __syncthreads() ::emu::barrier(__LINE__)
#define __builtin_amdgcn_s_barrier() ::emu::barrier(__LINE__)
#define __builtin_amdgcn_wave_barrier() ::emu::wave_barrier(__LINE__)
#define __builtin_amdgcn_fence(...) ((void)0)
#define __builtin_amdgcn_s_sleep(n) ::emu::sleep_yield()
#define __builtin_amdgcn_s_setprio(n) ((void)0)
#define __builtin_amdgcn_sched_barrier(n) ((void)0)
#define __builtin_amdgcn_readfirstlane(x) ::emu::readfirstlane((int)(x), __LINE__)
#define __builtin_amdgcn_readlane(x, l) ::emu::readlane((int)(x), (l), __LINE__)
#define __builtin_amdgcn_update_dpp(o, s, c, rm, bm, bc) ::emu::update_dpp((o), (s), (c), (rm), (bm), (bc), __LINE__)
#define __builtin_amdgcn_mov_dpp(s, c, rm, bm, bc) ::emu::update_dpp((int)0xDEADBEEF, (s), (c), (rm), (bm), (bc), __LINE__)
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, x, y, z) ::emu::mfma_16x16x32(0, (a), (b), (c), __LINE__)
#define __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, x, y, z) ::emu::mfma_16x16x32(1, (a), (b), (c), __LINE__)
#define __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, x, y, z) ::emu::mfma_16x16x16(0, (a), (b), (c), __LINE__)
#define __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, x, y, z) ::emu::mfma_16x16x16(1, (a), (b), (c), __LINE__)
#define __builtin_amdgcn_fdot2_f32_bf16(a, b, c, clamp) ::emu::dot2(0, (a), (b), (c))
#define __builtin_amdgcn_fdot2(a, b, c, clamp) ::emu::dot2(1, (a), (b), (c))
#define __builtin_amdgcn_perm(a, b, s) ::emu::perm((a), (b), (s))
#define __builtin_amdgcn_exp2f(x) exp2f(x)
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define __builtin_amdgcn_kernarg_segment_ptr() (::emu::fatal("kernarg_segment_ptr is not emulated"), (void *)nullptr)
#define __hip_atomic_fetch_add(p, v, o, s) ::emu::atomic_fetch_add((p), (v))
#define __hip_atomic_load(p, o, s) ::emu::atomic_load((p))
#define __hip_atomic_store(p, v, o, s) ::emu::atomic_store((p), (v))
#define __hip_atomic_compare_exchange_strong(p, e, d, o1, o2, s) ::emu::atomic_cas((p), (e), (d))
#define atomicAdd(p, v) ::emu::atomic_fetch_add((p), (v))

// ------------------------------------------------------------------ host runtime
typedef enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorLaunchFailure = 719,
} hipError_t;
typedef struct ihipStream_t *hipStream_t;
typedef enum hipFuncAttribute { hipFuncAttributeMaxDynamicSharedMemorySize = 8 } hipFuncAttribute;
typedef enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 63 } hipDeviceAttribute_t;

hipError_t hipGetLastError();
hipError_t hipPeekAtLastError();
const char *hipGetErrorString(hipError_t e);
hipError_t hipFuncSetAttribute(const void *f, hipFuncAttribute attr, int value);
hipError_t hipGetDevice(int *dev);
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t attr, int dev);
hipError_t hipMemsetAsync(void *p, int value, size_t bytes, hipStream_t s);
// Occupancy: the executor runs every workgroup, so any positive count is in bounds; a
// small one makes strided kernels walk several rows per workgroup.
template <class F>
inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int *blocks, F, int, size_t) {
    *blocks = 1;
    return hipSuccess;
}

#define HIP_SYMBOL(x) (&(x))
template <class T>
inline hipError_t hipGetSymbolAddress(void **p, T *sym) {
    *p = (void *)sym;
    return hipSuccess;
}

#define hipLaunchKernelGGL(k, grid, block, dyn, stream, ...) \
    ::emu::launch(#k, k, dim3(grid), dim3(block), (size_t)(dyn), __VA_ARGS__)
