// Fiber scheduler, cross-lane evaluation and launches of the CPU executor (emu.h).
#include "emu.h"

#include <sys/mman.h>
#include <unistd.h>

#include <cstdarg>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#endif
#endif
#ifdef EMU_ASAN
#include <sanitizer/asan_interface.h>
#include <sanitizer/common_interface_defs.h>
#endif

// Context switch (x86-64 System V): saves the callee-saved registers, MXCSR and the x87
// control word on the current stack, stores the stack pointer to *save, loads `load`.
extern "C" void emu_swap(void **save, void *load);
extern "C" void emu_trampoline();
asm(R"(
    .text
    .globl emu_swap
    .type emu_swap, @function
emu_swap:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    subq $8, %rsp
    stmxcsr (%rsp)
    fnstcw 4(%rsp)
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    ldmxcsr (%rsp)
    fldcw 4(%rsp)
    addq $8, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size emu_swap, .-emu_swap

    .globl emu_trampoline
    .type emu_trampoline, @function
emu_trampoline:
    movq %r12, %rdi
    callq *%r13
    ud2
    .size emu_trampoline, .-emu_trampoline
)");

namespace emu {
namespace {

enum State { READY, AT_XLANE, AT_BARRIER, DONE };

constexpr size_t kStackBytes = 512 * 1024;
constexpr int kWave = 64;

struct Thread {
    void *sp = nullptr;
    char *stack = nullptr;  // mapping, lowest page is a guard
    Idx3 tid{0, 0, 0};
    int linear = 0;
    State state = READY;
    XOp *op = nullptr;
    int barrier_line = 0;
    void *fake_stack = nullptr;
};

struct Block {
    const char *kernel = nullptr;
    Idx3 bidx{0, 0, 0}, bdim{1, 1, 1}, gdim{1, 1, 1};
    std::vector<Thread> threads;
    Body body = nullptr;
    void *ctx = nullptr;
    char *lds = nullptr;
};

Thread *g_cur = nullptr;
Block *g_block = nullptr;
void *g_sched_sp = nullptr;
const void *g_sched_bottom = nullptr;
size_t g_sched_size = 0;
void *g_sched_fake = nullptr;
hipError_t g_last = hipSuccess;
int g_cus = 256;
std::vector<char *> g_stack_pool;

char *take_stack() {
    if (!g_stack_pool.empty()) {
        char *s = g_stack_pool.back();
        g_stack_pool.pop_back();
        return s;
    }
    const size_t page = (size_t)sysconf(_SC_PAGESIZE);
    void *m = mmap(nullptr, kStackBytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (m == MAP_FAILED) fatal("mmap of a fiber stack failed");
    mprotect(m, page, PROT_NONE);
    return static_cast<char *>(m);
}

void give_stack(char *s) { g_stack_pool.push_back(s); }

void describe_current() {
    if (g_block)
        fprintf(stderr, "[emu] kernel %s, workgroup (%u,%u,%u), thread %d (wave %d, lane %d)\n", g_block->kernel,
                g_block->bidx.x, g_block->bidx.y, g_block->bidx.z, g_cur ? g_cur->linear : -1,
                g_cur ? g_cur->linear / kWave : -1, g_cur ? g_cur->linear % kWave : -1);
}

#ifdef EMU_ASAN
void asan_death() { describe_current(); }
struct AsanHook {
    AsanHook() { __asan_set_death_callback(asan_death); }
} g_asan_hook;
#endif

extern "C" void emu_fiber_main(Thread *t) {
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(nullptr, &g_sched_bottom, &g_sched_size);
#endif
    (void)t;
    g_block->body(g_block->ctx);
    g_cur->state = DONE;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(nullptr, g_sched_bottom, g_sched_size);
#endif
    void *dead;
    emu_swap(&dead, g_sched_sp);
    __builtin_unreachable();
}

void init_fiber(Thread &t) {
    t.stack = take_stack();
    char *top = t.stack + kStackBytes;
    uintptr_t sp0 = ((uintptr_t)top - 64) & ~(uintptr_t)15;
    uint64_t *s = reinterpret_cast<uint64_t *>(sp0);
    s[-1] = (uint64_t)(uintptr_t)&emu_trampoline;  // return address of the first switch
    s[-2] = 0;                                     // rbp
    s[-3] = 0;                                     // rbx
    s[-4] = (uint64_t)(uintptr_t)&t;               // r12: argument
    s[-5] = (uint64_t)(uintptr_t)&emu_fiber_main;  // r13: entry
    s[-6] = 0;                                     // r14
    s[-7] = 0;                                     // r15
    uint32_t *ctl = reinterpret_cast<uint32_t *>(&s[-8]);
    ctl[0] = 0x1F80;  // MXCSR
    ctl[1] = 0x037F;  // x87 control word
    t.sp = &s[-8];
}

void run_fiber(Thread &t) {
    g_cur = &t;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(&g_sched_fake, t.stack, kStackBytes);
#endif
    emu_swap(&g_sched_sp, t.sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(g_sched_fake, nullptr, nullptr);
#endif
    g_cur = nullptr;
}

// Called on a fiber: back to the scheduler until it resumes this fiber.
void suspend() {
    Thread *t = g_cur;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(&t->fake_stack, g_sched_bottom, g_sched_size);
#endif
    emu_swap(&t->sp, g_sched_sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(t->fake_stack, &g_sched_bottom, &g_sched_size);
#endif
    g_cur = t;
}

const char *kind_name(int k) {
    switch (k) {
        case X_SHFL: return "shfl";
        case X_SHFL_XOR: return "shfl_xor";
        case X_SHFL_UP: return "shfl_up";
        case X_READLANE: return "readlane";
        case X_READFIRST: return "readfirstlane";
        case X_BALLOT: return "ballot";
        case X_DPP: return "dpp";
        case X_MFMA: return "mfma";
        case X_WAVE_BARRIER: return "wave_barrier";
    }
    return "?";
}

// DPP source lane of `lane` for control `ctrl`, or -1 when the source is out of range.
int dpp_source(int lane, int ctrl) {
    const int row = lane & ~15, in = lane & 15;
    if (ctrl >= 0x000 && ctrl <= 0x0ff) return (lane & ~3) | ((ctrl >> (2 * (lane & 3))) & 3);
    if (ctrl >= 0x101 && ctrl <= 0x10f) {  // row_shl: lane i reads i + n
        const int n = ctrl - 0x100;
        return in + n < 16 ? lane + n : -1;
    }
    if (ctrl >= 0x111 && ctrl <= 0x11f) {  // row_shr: lane i reads i - n
        const int n = ctrl - 0x110;
        return in >= n ? lane - n : -1;
    }
    if (ctrl >= 0x121 && ctrl <= 0x12f) {  // row_ror: lane i reads (i - n) mod 16
        const int n = ctrl - 0x120;
        return row | ((in - n) & 15);
    }
    if (ctrl == 0x140) return row | (15 - in);                    // row_mirror
    if (ctrl == 0x141) return (lane & ~7) | (7 - (lane & 7));     // row_half_mirror
    if (ctrl >= 0x150 && ctrl <= 0x15f) return row | (ctrl - 0x150);  // row_newbcast
    fatal("DPP control 0x%x is not emulated", ctrl);
}

float cvt16(int dt, uint32_t h) { return dt == 0 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h); }

void resolve_wave(Block &b, int w0, int w1) {
    XOp *ops[kWave] = {};
    int first = -1, kind = 0, line = 0;
    for (int i = w0; i < w1; ++i) {
        Thread &t = b.threads[i];
        if (t.state != AT_XLANE) continue;
        ops[i - w0] = t.op;
        if (first < 0) {
            first = i - w0;
            kind = t.op->kind;
            line = t.op->line;
        } else if (t.op->kind != kind || t.op->line != line) {
            describe_current();
            fatal("kernel %s workgroup %u: lanes of wave %d meet at different cross-lane ops (%s line %d, %s line %d)",
                  b.kernel, b.bidx.x, w0 / kWave, kind_name(kind), line, kind_name(t.op->kind), t.op->line);
        }
    }
    if (first < 0) return;
    auto active = [&](int l) { return l >= 0 && l < kWave && ops[l] != nullptr; };
    auto need = [&](int l, int dst) {
        if (!active(l))
            fatal("kernel %s workgroup %u wave %d lane %d: %s (line %d) reads lane %d, which is not active", b.kernel,
                  b.bidx.x, w0 / kWave, dst, kind_name(kind), line, l);
        return ops[l]->v;
    };
    const uint64_t mask32 = ops[first]->bytes == 8 ? ~0ull : 0xffffffffull;
    if (kind == X_MFMA) {
        for (int l = 0; l < kWave; ++l)
            if (!active(l)) fatal("kernel %s: MFMA (line %d) with inactive lane %d", b.kernel, line, l);
        const int K = ops[first]->p0, per = K / 4;  // k elements per lane group: 8 (K 32) or 4 (K 16)
        for (int l = 0; l < kWave; ++l) {
            const int n = l & 15, j = l >> 4;
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * j + i;
                double acc = ops[l]->c[i];
                for (int k = 0; k < K; ++k) {
                    const XOp &A = *ops[m + 16 * (k / per)], &B = *ops[n + 16 * (k / per)];
                    const int e = k % per;
                    const float av = cvt16(ops[l]->dt, (A.a[e >> 1] >> (16 * (e & 1))) & 0xffff);
                    const float bv = cvt16(ops[l]->dt, (B.b[e >> 1] >> (16 * (e & 1))) & 0xffff);
                    acc += (double)av * bv;
                }
                ops[l]->d[i] = (float)acc;
            }
        }
    } else {
        uint64_t res[kWave];
        for (int l = 0; l < kWave; ++l) {
            if (!active(l)) continue;
            XOp &o = *ops[l];
            switch (kind) {
                case X_SHFL: {
                    const int wdt = o.p1, base = l & ~(wdt - 1);
                    res[l] = need(base + (o.p0 & (wdt - 1)), l);
                    break;
                }
                case X_SHFL_XOR: {
                    const int wdt = o.p1, idx = l ^ o.p0;
                    res[l] = need(idx >= ((l + wdt) & ~(wdt - 1)) ? l : idx, l);
                    break;
                }
                case X_SHFL_UP: {
                    const int wdt = o.p1, idx = l - o.p0;
                    res[l] = need(idx < (l & ~(wdt - 1)) ? l : idx, l);
                    break;
                }
                case X_READLANE:
                    res[l] = need(o.p0 & 63, l);
                    break;
                case X_READFIRST:
                    res[l] = ops[first]->v;
                    break;
                case X_BALLOT: {
                    uint64_t m = 0;
                    for (int s = 0; s < kWave; ++s)
                        if (active(s) && ops[s]->v) m |= 1ull << s;
                    res[l] = m;
                    break;
                }
                case X_DPP: {
                    const int s = dpp_source(l, o.p0);
                    if (s >= 0 && active(s)) res[l] = ops[s]->v;
                    else if (s >= 0 && o.p2 == 0 && ops[l]->old == 0xDEADBEEFull)
                        fatal("kernel %s: DPP (line %d) lane %d reads inactive lane %d with no old value", b.kernel,
                              line, l, s);
                    else res[l] = o.p2 ? 0 : o.old;
                    break;
                }
                case X_WAVE_BARRIER:
                    res[l] = 0;
                    break;
                default:
                    fatal("unknown cross-lane op %d", kind);
            }
        }
        for (int l = 0; l < kWave; ++l)
            if (active(l)) ops[l]->r = res[l] & mask32;
    }
    for (int i = w0; i < w1; ++i)
        if (b.threads[i].state == AT_XLANE) b.threads[i].state = READY;
}

void run_block(Block &b) {
    const int n = (int)b.threads.size();
    for (int i = 0; i < n; ++i) {
        Thread &t = b.threads[i];
        t.linear = i;
        t.tid = Idx3{(unsigned)(i % b.bdim.x), (unsigned)((i / b.bdim.x) % b.bdim.y),
                     (unsigned)(i / (b.bdim.x * b.bdim.y))};
        t.state = READY;
        init_fiber(t);
    }
    long idle_rounds = 0;
    for (;;) {
        bool any_ready = false;
        for (auto &t : b.threads)
            if (t.state == READY) run_fiber(t);
        bool progress = false;
        for (int w0 = 0; w0 < n; w0 += kWave) {
            const int w1 = min(w0 + kWave, n);
            bool ready = false, xl = false;
            for (int i = w0; i < w1; ++i) {
                ready |= b.threads[i].state == READY;
                xl |= b.threads[i].state == AT_XLANE;
            }
            any_ready |= ready;
            if (!ready && xl) {
                resolve_wave(b, w0, w1);
                progress = true;
            }
        }
        if (progress) {
            idle_rounds = 0;
            continue;
        }
        if (any_ready) {  // spinning fibers only (s_sleep)
            if (++idle_rounds > 20000000) fatal("kernel %s workgroup %u: no progress (spin-wait never ends)", b.kernel,
                                                b.bidx.x);
            continue;
        }
        int live = 0, at_barrier = 0;
        for (auto &t : b.threads) {
            live += t.state != DONE;
            at_barrier += t.state == AT_BARRIER;
        }
        if (live == 0) break;
        if (at_barrier == live) {
            for (auto &t : b.threads)
                if (t.state == AT_BARRIER) t.state = READY;
            idle_rounds = 0;
            continue;
        }
        fatal("kernel %s workgroup %u: deadlock", b.kernel, b.bidx.x);
    }
    for (auto &t : b.threads) give_stack(t.stack);
}

}  // namespace

const Idx3 &thread_idx() { return g_cur->tid; }
const Idx3 &block_idx() { return g_block->bidx; }
const Idx3 &block_dim() { return g_block->bdim; }
const Idx3 &grid_dim() { return g_block->gdim; }

void cross_lane(XOp &op) {
    g_cur->op = &op;
    g_cur->state = AT_XLANE;
    suspend();
}

void barrier(int line) {
    g_cur->barrier_line = line;
    g_cur->state = AT_BARRIER;
    suspend();
}

void sleep_yield() {
    g_cur->state = READY;
    suspend();
}

void *dynamic_lds() { return g_block->lds; }

void fatal(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    fprintf(stderr, "[emu] fatal: ");
    vfprintf(stderr, fmt, ap);
    fprintf(stderr, "\n");
    va_end(ap);
    describe_current();
    fflush(stderr);
    abort();
}

float bf16_bits_to_f32(uint32_t h) { return __uint_as_float((h & 0xffff) << 16); }

float f16_bits_to_f32(uint32_t h) {
    const uint16_t b = (uint16_t)h;
    _Float16 x;
    memcpy(&x, &b, 2);
    return (float)x;
}

// Launch order of the workgroups: EMU_ORDER=reverse runs them last to first (the
// dynamic schedules then hand the claims to other workers).
static bool reverse_order() {
    static int r = [] {
        const char *e = getenv("EMU_ORDER");
        return e && !strcmp(e, "reverse") ? 1 : 0;
    }();
    return r != 0;
}

void run_grid(const char *name, dim3 grid, dim3 block, size_t dynamic_lds, Body body, void *ctx) {
    if (g_cur) fatal("launch from device code");
    const long nthreads = (long)block.x * block.y * block.z;
    if (nthreads <= 0 || nthreads > 1024) {
        g_last = hipErrorInvalidValue;
        return;
    }
    if (dynamic_lds > 160 * 1024) {
        g_last = hipErrorInvalidValue;
        return;
    }
    const long nblocks = (long)grid.x * grid.y * grid.z;
    for (long q = 0; q < nblocks; ++q) {
        const long id = reverse_order() ? nblocks - 1 - q : q;
        Block b;
        b.kernel = name;
        b.bidx = Idx3{(unsigned)(id % grid.x), (unsigned)((id / grid.x) % grid.y), (unsigned)(id / ((long)grid.x * grid.y))};
        b.bdim = Idx3{block.x, block.y, block.z};
        b.gdim = Idx3{grid.x, grid.y, grid.z};
        b.threads.resize(nthreads);
        b.body = body;
        b.ctx = ctx;
        b.lds = dynamic_lds ? static_cast<char *>(malloc(dynamic_lds)) : nullptr;
        if (b.lds) memset(b.lds, 0xA5, dynamic_lds);  // LDS holds garbage when a workgroup starts
        g_block = &b;
        run_block(b);
        g_block = nullptr;
        free(b.lds);
    }
}

}  // namespace emu

// ------------------------------------------------------------------ host runtime
hipError_t hipGetLastError() {
    const hipError_t e = emu::g_last;
    emu::g_last = hipSuccess;
    return e;
}
hipError_t hipPeekAtLastError() { return emu::g_last; }
const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "emulated launch error"; }
hipError_t hipFuncSetAttribute(const void *, hipFuncAttribute, int value) {
    return value <= 160 * 1024 ? hipSuccess : hipErrorInvalidValue;
}
hipError_t hipGetDevice(int *dev) {
    *dev = 0;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t attr, int) {
    if (attr != hipDeviceAttributeMultiprocessorCount) return hipErrorInvalidValue;
    *v = emu::g_cus;
    return hipSuccess;
}
hipError_t hipMemsetAsync(void *p, int value, size_t bytes, hipStream_t) {
    memset(p, value, bytes);
    return hipSuccess;
}

// C entry points of the executor itself (used by the Python driver).
extern "C" {
void *emu_alloc(size_t bytes) {
    void *p = malloc(bytes ? bytes : 1);
    if (p) memset(p, 0xA5, bytes);  // device memory from hipMalloc holds garbage
    return p;
}
void emu_free(void *p) { free(p); }
void emu_set_cus(int n) { emu::g_cus = n; }
}
