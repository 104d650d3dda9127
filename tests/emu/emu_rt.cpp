// CPU emulation of the HIP execution model for the library's own kernels
// (test infrastructure, see include/hip/hip_runtime.h here).
//
// A launch runs its workgroups one after the other.  Each GPU thread of a
// workgroup is a coroutine with its own stack; the scheduler runs every
// runnable thread until it blocks:
//   - at __syncthreads (a workgroup barrier: released when every thread
//     that has not returned is waiting there, all at the same call site);
//   - at a wave-wide builtin (released when every live lane of its 64-lane
//     wave waits either there or at a barrier: the builtin runs over the
//     lanes that reached it, as the SIMD runs it inside a branch with the
//     other lanes masked off; the results are computed from those lanes'
//     inputs at once).
// Lanes of one wave at different builtins, a lane-to-lane read from a
// masked lane, or threads at different barriers stop the run with the call
// sites.  Dynamic LDS is a malloc'd block of exactly the launch's size, so
// an AddressSanitizer build reports LDS accesses past it; device memory is
// malloc'd too.  Every 8-byte word of a launch's arguments that points into
// host memory -- the live part of the host thread's stack, or
// (AddressSanitizer build) a heap block that is not a hipMalloc allocation --
// stops the run: on the GPU the kernel's access through it would be a
// memory fault (the library uses no pinned or managed host memory).  The
// build fills every local with a byte pattern before use, so padding bytes
// between arguments hold that pattern, never a stale address.  With EMU_STATS set, each launch prints its barrier
// releases, wave builtin rounds and coroutine resumes; EMU_ORDER, EMU_LANES
// and EMU_BLOCKS change the order in which waves and lanes run between
// synchronization points and the order of a launch's workgroups (see below).
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <time.h>

#include <algorithm>
#include <chrono>
#include <iterator>
#include <map>
#include <mutex>
#include <vector>

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#endif
#endif
#include <pthread.h>
#ifdef EMU_ASAN
extern "C" const void* __sanitizer_get_allocated_begin(const void* p);
extern "C" void __sanitizer_start_switch_fiber(void** fake_stack_save, const void* bottom, size_t size);
extern "C" void __sanitizer_finish_switch_fiber(void* fake_stack_save, const void** bottom_old, size_t* size_old);
#endif

extern "C" void emu_swap(void** save_sp, void* load_sp);

namespace emu {

namespace {

constexpr size_t STACK_BYTES = 512 * 1024;
constexpr int MAX_THREADS = 1024;

enum State { RUN, BAR, WOP, DONE };

struct Thread {
    ThreadView v;
    State st = RUN;
    void* sp = nullptr;
    char* stack = nullptr;
    int op = 0;
    uint64_t val = 0;
    int64_t arg = 0, width = 64;
    uint64_t res = 0;
    void* fake = nullptr;
    const char* file = nullptr;  // source location of the barrier or wave builtin it waits at
    int line = 0;
};

struct Launch {
    Body body = nullptr;
    void* closure = nullptr;
    char* lds = nullptr;
    size_t lds_bytes = 0;
    int nthreads = 0;
};

std::vector<char*> g_stacks;
Thread g_th[MAX_THREADS];
Thread* g_cur = nullptr;
Launch g_launch;
void* g_sched_sp = nullptr;
void* g_sched_fake = nullptr;
const void* g_sched_bottom = nullptr;
size_t g_sched_size = 0;
hipError_t g_last = hipSuccess;
std::mutex g_mu;  // one launch at a time

[[noreturn]] void die(const char* what, const Thread* t) {
    if (t)
        fprintf(stderr, "[emu] %s (thread %u,%u,%u of block %u,%u,%u, lane %d, op %d, at %s:%d)\n", what, t->v.tid.x,
                t->v.tid.y, t->v.tid.z, t->v.bid.x, t->v.bid.y, t->v.bid.z, t->v.lane, t->op,
                t->file ? t->file : "?", t->line);
    else
        fprintf(stderr, "[emu] %s\n", what);
    fflush(stderr);
    abort();
}

char* stack_of(int i) {
    while ((int)g_stacks.size() <= i) {
        void* p = mmap(nullptr, STACK_BYTES, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
        if (p == MAP_FAILED) die("cannot map a coroutine stack", nullptr);
        g_stacks.push_back((char*)p);
    }
    return g_stacks[i];
}

// switch from the running thread back to the scheduler
void to_scheduler() {
    Thread* t = g_cur;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(&t->fake, g_sched_bottom, g_sched_size);
#endif
    emu_swap(&t->sp, g_sched_sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(t->fake, nullptr, nullptr);
#endif
}

void entry() {
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(nullptr, &g_sched_bottom, &g_sched_size);
#endif
    g_launch.body(g_launch.closure);
    g_cur->st = DONE;
    Thread* t = g_cur;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(nullptr, g_sched_bottom, g_sched_size);
#endif
    emu_swap(&t->sp, g_sched_sp);
    die("a finished coroutine was resumed", t);
}

void resume(Thread& t) {
    g_cur = &t;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(&g_sched_fake, t.stack, STACK_BYTES);
#endif
    emu_swap(&g_sched_sp, t.sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(g_sched_fake, &g_sched_bottom, &g_sched_size);
#endif
    g_cur = nullptr;
}

void init_thread(Thread& t, int i) {
    t.stack = stack_of(i);
    // initial frame: six callee-saved registers, then the return address
    // emu_swap's `ret` takes (entry), then a dummy slot so that entry starts
    // with the stack aligned as after a call
    uint64_t* top = (uint64_t*)(t.stack + STACK_BYTES);
    uint64_t* sp = top - 8;
    for (int k = 0; k < 6; ++k) sp[k] = 0;
    sp[6] = (uint64_t)(void*)&entry;
    sp[7] = 0;
    t.sp = sp;
    t.st = RUN;
    t.op = 0;
}

uint64_t dpp_src(int ctrl, int lane) {
    if (ctrl <= 0xFF) {  // quad_perm
        const int q = lane & ~3, k = lane & 3;
        return (uint64_t)(q + ((ctrl >> (2 * k)) & 3));
    }
    if (ctrl == 0x140) return (uint64_t)((lane & ~15) + (15 - (lane & 15)));  // row_mirror
    if (ctrl == 0x141) return (uint64_t)((lane & ~7) + (7 - (lane & 7)));     // row_half_mirror
    die("unsupported DPP control", nullptr);
}

// Resolves one wave's builtin over its active lanes: the lanes waiting at it
// (all live lanes, or a subset whose other lanes wait further on at a
// barrier, as the hardware runs a builtin inside a branch with the other
// lanes masked off).  The active lanes must wait at one builtin at one
// source location; a ballot counts only active lanes, readfirstlane reads
// the first one, and a lane-to-lane read (shuffle, readlane, DPP) from an
// inactive lane stops the run.
void resolve(int w0, int n) {
    Thread* L = &g_th[w0];
    int first = -1, op = 0;
    for (int l = 0; l < n; ++l) {
        if (L[l].st != WOP) continue;
        if (first < 0) {
            first = l;
            op = L[l].op;
        } else if (L[l].op != op || L[l].line != L[first].line || L[l].file != L[first].file) {
            fprintf(stderr, "[emu]   lane %d waits at %s:%d, lane %d at %s:%d\n", first,
                    L[first].file ? L[first].file : "?", L[first].line, l, L[l].file ? L[l].file : "?", L[l].line);
            die("lanes of one wave wait at different wave builtins", &L[l]);
        }
    }
    uint64_t act = 0;  // the active set, taken before any lane is released
    for (int l = 0; l < n; ++l)
        if (L[l].st == WOP) act |= 1ull << l;
    auto active = [&](int l) { return l >= 0 && l < n && ((act >> l) & 1u); };
    uint64_t ballot = 0;
    if (op == W_BALLOT)
        for (int l = 0; l < n; ++l)
            if (active(l) && L[l].val) ballot |= 1ull << l;
    for (int l = 0; l < n; ++l) {
        Thread& t = L[l];
        if (!active(l)) continue;
        const int width = (int)t.width;
        const int base = l & ~(width - 1), off = l & (width - 1);
        int src = l;
        switch (op) {
            case W_READFIRST: src = first; break;
            case W_READLANE: src = (int)t.arg; break;
            case W_BALLOT: break;
            case W_SHFL: src = base + (int)(t.arg & (width - 1)); break;
            case W_SHFL_UP: src = off >= t.arg ? l - (int)t.arg : l; break;
            case W_SHFL_DOWN: src = off + t.arg < width ? l + (int)t.arg : l; break;
            case W_SHFL_XOR: src = base + ((off ^ (int)t.arg) & (width - 1)); break;
            case W_DPP: src = (int)dpp_src((int)t.arg, l); break;
            default: die("unknown wave builtin", &t);
        }
        if (op != W_BALLOT && src >= 0 && src < n && L[src].st != DONE && !active(src))
            die("a wave builtin reads a lane that does not take part in it", &t);
        if (op == W_BALLOT) t.res = ballot;
        else t.res = active(src) ? L[src].val : t.val;
        t.st = RUN;
    }
}

// Counts of one launch for EMU_STATS: barrier releases and wave builtin
// resolutions (per workgroup / per wave), and coroutine resumes.
struct Stats {
    uint64_t blocks = 0, barriers = 0, wave_ops = 0, resumes = 0;
};
Stats g_stats;
const bool g_print_stats = getenv("EMU_STATS") != nullptr;

// Order in which the waves of a workgroup run between synchronization
// points (EMU_ORDER): "forward" (default), "reverse", or "shuffle" (a new
// random order every round, seeded by EMU_SEED).  Lanes of a wave keep their
// order.  Kernels whose waves communicate only across barriers give the
// same results in every order; a missing barrier shows as a difference.
enum Order { FORWARD, REVERSE, SHUFFLE };
const Order g_order = [] {
    const char* e = getenv("EMU_ORDER");
    if (!e || !strcmp(e, "forward")) return FORWARD;
    if (!strcmp(e, "reverse")) return REVERSE;
    if (!strcmp(e, "shuffle")) return SHUFFLE;
    fprintf(stderr, "[emu] EMU_ORDER must be forward, reverse or shuffle\n");
    abort();
}();
// EMU_FILL: the byte that fresh LDS and fresh device allocations hold
// (default 0xCD for LDS, 0xAB for device memory).  A kernel that reads
// memory it never wrote gives results that change with it.
const int g_fill = [] {
    const char* e = getenv("EMU_FILL");
    return e ? (int)(strtol(e, nullptr, 0) & 0xff) : -1;
}();

// EMU_BLOCKS: the order of a launch's workgroups, as EMU_ORDER ("forward",
// "reverse", "shuffle").
const Order g_blocks = [] {
    const char* e = getenv("EMU_BLOCKS");
    if (!e || !strcmp(e, "forward")) return FORWARD;
    if (!strcmp(e, "reverse")) return REVERSE;
    if (!strcmp(e, "shuffle")) return SHUFFLE;
    fprintf(stderr, "[emu] EMU_BLOCKS must be forward, reverse or shuffle\n");
    abort();
}();
// EMU_LANES=reverse runs the lanes of each wave from the last to the first
// between synchronization points.
const bool g_lanes_reversed = [] {
    const char* e = getenv("EMU_LANES");
    return e && !strcmp(e, "reverse");
}();
uint64_t g_rng = [] {
    const char* e = getenv("EMU_SEED");
    return e ? strtoull(e, nullptr, 10) * 0x9e3779b97f4a7c15ull + 1 : 0x2545F4914F6CDD1Dull;
}();
uint32_t next_rand() {  // xorshift64*
    g_rng ^= g_rng >> 12;
    g_rng ^= g_rng << 25;
    g_rng ^= g_rng >> 27;
    return (uint32_t)((g_rng * 0x2545F4914F6CDD1Dull) >> 32);
}

void run_block(dim3 bid, dim3 grid, dim3 block) {
    const int n = g_launch.nthreads;
    for (int i = 0; i < n; ++i) {
        Thread& t = g_th[i];
        init_thread(t, i);
        t.v.tid = Idx{(uint32_t)(i % block.x), (uint32_t)((i / block.x) % block.y), (uint32_t)(i / (block.x * block.y))};
        t.v.bid = Idx{bid.x, bid.y, bid.z};
        t.v.bdim = Idx{block.x, block.y, block.z};
        t.v.gdim = Idx{grid.x, grid.y, grid.z};
        t.v.lane = i & 63;
    }
    ++g_stats.blocks;
    const int nw = (n + 63) / 64;
    int worder[MAX_THREADS / 64];
    for (int w = 0; w < nw; ++w) worder[w] = g_order == REVERSE ? nw - 1 - w : w;
    for (;;) {
        if (g_order == SHUFFLE)
            for (int w = nw - 1; w > 0; --w) std::swap(worder[w], worder[next_rand() % (uint32_t)(w + 1)]);
        for (int wi = 0; wi < nw; ++wi) {
            const int b = worder[wi] * 64, e = std::min(n, b + 64);
            for (int k = 0; k < e - b; ++k) {
                const int i = g_lanes_reversed ? e - 1 - k : b + k;
                if (g_th[i].st == RUN) {
                    resume(g_th[i]);
                    ++g_stats.resumes;
                }
            }
        }
        bool moved = false;
        for (int w0 = 0; w0 < n; w0 += 64) {
            const int wn = std::min(64, n - w0);
            int live = 0, wop = 0;
            for (int l = 0; l < wn; ++l) {
                const State s = g_th[w0 + l].st;
                live += s != DONE;
                wop += s == WOP;
            }
            if (wop == 0) continue;
            // every live lane now waits at a builtin or a barrier; those at
            // a barrier are the lanes a branch left out of the builtin
            resolve(w0, wn);
            ++g_stats.wave_ops;
            moved = true;
        }
        if (moved) continue;
        int live = 0, bar = 0;
        for (int i = 0; i < n; ++i) {
            live += g_th[i].st != DONE;
            bar += g_th[i].st == BAR;
        }
        if (live == 0) break;
        if (bar != live) die("deadlock: no thread can run", nullptr);
        // one barrier releases the workgroup: every waiting thread must be
        // at the same __syncthreads
        const Thread* b0 = nullptr;
        for (int i = 0; i < n; ++i) {
            const Thread& t = g_th[i];
            if (t.st != BAR) continue;
            if (!b0) {
                b0 = &t;
            } else if (t.line != b0->line || t.file != b0->file) {
                fprintf(stderr, "[emu]   a thread waits at %s:%d, another at %s:%d\n", b0->file ? b0->file : "?",
                        b0->line, t.file ? t.file : "?", t.line);
                die("threads of a workgroup wait at different barriers", &t);
            }
        }
        for (int i = 0; i < n; ++i)
            if (g_th[i].st == BAR) g_th[i].st = RUN;
        ++g_stats.barriers;
    }
}

}  // namespace

const ThreadView& view() {
    if (!g_cur) die("thread index read outside a kernel", nullptr);
    return g_cur->v;
}

char* lds_base() {
    if (!g_cur) die("LDS used outside a kernel", nullptr);
    return g_launch.lds;
}

void barrier(const char* file, int line) {
    if (!g_cur) die("__syncthreads outside a kernel", nullptr);
    g_cur->file = file;
    g_cur->line = line;
    g_cur->st = BAR;
    to_scheduler();
}

uint64_t wave(int op, uint64_t v, int64_t arg, int64_t width, const char* file, int line) {
    if (!g_cur) die("wave builtin outside a kernel", nullptr);
    Thread* t = g_cur;
    t->file = file;
    t->line = line;
    t->op = op;
    t->val = v;
    t->arg = arg;
    t->width = width;
    t->st = WOP;
    to_scheduler();
    return t->res;
}

void check_kernel_args(const char* name, const void* args, size_t bytes);

void launch_raw(const void*, const char* name, dim3 grid, dim3 block, size_t lds, hipStream_t, Body body,
                void* closure, const void* args, size_t args_bytes) {
    check_kernel_args(name, args, args_bytes);
    std::lock_guard<std::mutex> lk(g_mu);
    const uint64_t nt = (uint64_t)block.x * block.y * block.z;
    if (nt == 0 || nt > MAX_THREADS || grid.x == 0 || grid.y == 0 || grid.z == 0) {
        g_last = hipErrorInvalidValue;
        return;
    }
    // the dispatch packet counts work-items per dimension in 32 bits, and
    // HIP reports 65,536 as the largest y and z grid
    if ((uint64_t)grid.x * block.x > 0xffffffffull || (uint64_t)grid.y * block.y > 0xffffffffull ||
        (uint64_t)grid.z * block.z > 0xffffffffull || grid.y > 65536u || grid.z > 65536u) {
        fprintf(stderr, "emu: kernel %s: grid %ux%ux%u of %ux%ux%u threads is past the dispatch limits\n",
                name ? name : "?", grid.x, grid.y, grid.z, block.x, block.y, block.z);
        abort();
    }
    if (lds > 160 * 1024) {
        g_last = hipErrorInvalidValue;
        return;
    }
    g_launch.body = body;
    g_launch.closure = closure;
    g_launch.nthreads = (int)nt;
    g_launch.lds_bytes = lds;
    // workgroups in grid order, or reversed / shuffled (EMU_BLOCKS)
    const uint64_t nb = (uint64_t)grid.x * grid.y * grid.z;
    std::vector<uint64_t> bo;
    if (g_blocks != FORWARD) {
        bo.resize(nb);
        for (uint64_t b = 0; b < nb; ++b) bo[b] = g_blocks == REVERSE ? nb - 1 - b : b;
        if (g_blocks == SHUFFLE)
            for (uint64_t b = nb - 1; b > 0; --b)
                std::swap(bo[b], bo[((uint64_t)next_rand() << 32 | next_rand()) % (b + 1)]);
    }
    for (uint64_t k = 0; k < nb; ++k) {
        const uint64_t b = bo.empty() ? k : bo[k];
        const uint32_t x = (uint32_t)(b % grid.x), y = (uint32_t)(b / grid.x % grid.y),
                       z = (uint32_t)(b / ((uint64_t)grid.x * grid.y));
        // exactly the launch's dynamic LDS (at least one byte), filled with a
        // pattern so that reads of uncleared LDS show
        g_launch.lds = (char*)malloc(lds ? lds : 1);
        memset(g_launch.lds, g_fill >= 0 ? g_fill : 0xCD, lds ? lds : 1);
        run_block(dim3(x, y, z), grid, block);
        free(g_launch.lds);
        g_launch.lds = nullptr;
    }
    if (g_print_stats) {
        fprintf(stderr, "[emu-stats] %s grid %ux%ux%u block %llu: %llu barriers, %llu wave-op rounds, %llu resumes\n",
                name, grid.x, grid.y, grid.z, (unsigned long long)nt, (unsigned long long)g_stats.barriers,
                (unsigned long long)g_stats.wave_ops, (unsigned long long)g_stats.resumes);
    }
    g_stats = Stats();
}

}  // namespace emu

// ---- runtime API -----------------------------------------------------------
struct emu_stream {
    int id;
};
struct emu_event {
    double t;
};

static double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// Live hipMalloc allocations (base -> bytes), so that pointers outside them
// can be reported as host memory when the driver asks for that (or the
// environment sets EMU_TRACK_HOST, for programs that know nothing of the
// emulation).
static std::map<uintptr_t, size_t> g_allocs;
static bool g_track_host = getenv("EMU_TRACK_HOST") != nullptr;
extern "C" void emu_track_host_memory(int on) { g_track_host = on != 0; }

hipError_t hipMalloc(void** p, size_t n) {
    if (!p) return hipErrorInvalidValue;
    *p = malloc(n ? n : 1);
    if (!*p) return emu::g_last = hipErrorOutOfMemory;
    memset(*p, emu::g_fill >= 0 ? emu::g_fill : 0xAB, n ? n : 1);  // device memory starts with garbage
    g_allocs[(uintptr_t)*p] = n ? n : 1;
    return hipSuccess;
}
hipError_t hipFree(void* p) {
    g_allocs.erase((uintptr_t)p);
    free(p);
    return hipSuccess;
}
namespace emu {

long long knob(const char* name, long long dflt) {
    const char* e = getenv(name);
    return e && *e ? strtoll(e, nullptr, 0) : dflt;
}

// True when p lies in a live hipMalloc allocation or one past its end.
static bool in_device_alloc(uintptr_t p) {
    auto it = g_allocs.upper_bound(p);
    if (it == g_allocs.begin()) return false;
    --it;
    return p <= it->first + it->second;
}

// The launch's arguments as stored for the kernel (8-byte words at 8-byte
// offsets): a word pointing into the host thread's stack, or into a host
// heap block (AddressSanitizer build), stops the run.
void check_kernel_args(const char* name, const void* args, size_t bytes) {
    static uintptr_t stack_lo = 0, stack_hi = 0;
    if (!stack_hi) {
        pthread_attr_t at;
        void* base = nullptr;
        size_t size = 0;
        if (pthread_getattr_np(pthread_self(), &at) == 0) {
            pthread_attr_getstack(&at, &base, &size);
            pthread_attr_destroy(&at);
        }
        stack_lo = (uintptr_t)base;
        stack_hi = stack_lo + size;
    }
    // the live part of the stack: from this frame up to the stack's top
    const uintptr_t live_lo = (uintptr_t)__builtin_frame_address(0);
    for (size_t o = 0; o + 8 <= bytes; o += 8) {
        uintptr_t w;
        memcpy(&w, (const char*)args + o, 8);
        if (w < 4096 || in_device_alloc(w)) continue;
        const char* what = nullptr;
        if (w >= live_lo && w < stack_hi && w >= stack_lo) what = "the host stack";
#ifdef EMU_ASAN
        else if (const void* b = __sanitizer_get_allocated_begin((const void*)w))
            if (!in_device_alloc((uintptr_t)b)) what = "host heap memory";
#endif
        if (what) {
            fprintf(stderr, "emu: kernel %s: argument bytes %zu..%zu point into %s (%p), not device memory\n",
                    name ? name : "?", o, o + 7, what, (void*)w);
            abort();
        }
    }
}

}  // namespace emu

// A device of MI355X's 288 GiB whose free memory is that less the live
// hipMalloc allocations.
hipError_t hipMemGetInfo(size_t* free_b, size_t* total_b) {
    const size_t total = (size_t)288 << 30;
    size_t used = 0;
    for (const auto& a : g_allocs) used += a.second;
    if (free_b) *free_b = used < total ? total - used : 0;
    if (total_b) *total_b = total;
    return hipSuccess;
}
hipError_t hipMemcpy(void* d, const void* s, size_t n, hipMemcpyKind) {
    if (n) memmove(d, s, n);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind k, hipStream_t) { return hipMemcpy(d, s, n, k); }
hipError_t hipMemset(void* d, int v, size_t n) {
    if (n) memset(d, v, n);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* d, int v, size_t n, hipStream_t) { return hipMemset(d, v, n); }
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) {
    *s = new emu_stream{1};
    return hipSuccess;
}
hipError_t hipStreamCreate(hipStream_t* s) { return hipStreamCreateWithFlags(s, 0); }
hipError_t hipStreamDestroy(hipStream_t s) {
    delete s;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipDeviceSynchronize() { return hipSuccess; }
hipError_t hipEventCreate(hipEvent_t* e) {
    *e = new emu_event{0.0};
    return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t e) {
    delete e;
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t e, hipStream_t) {
    e->t = now_ms();
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t a, hipEvent_t b) {
    *ms = (float)(b->t - a->t);
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipGetDeviceCount(int* n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int) {
    switch (a) {
        case hipDeviceAttributeMaxSharedMemoryPerBlock: *v = 160 * 1024; return hipSuccess;  // gfx950
        case hipDeviceAttributeMultiprocessorCount: *v = 256; return hipSuccess;
    }
    return hipErrorInvalidValue;
}
hipError_t hipPointerGetAttributes(hipPointerAttribute_t* a, const void* p) {
    // every pointer is "device" memory in the emulation, unless host memory
    // is tracked: then only pointers into hipMalloc allocations are
    memset(a, 0, sizeof(*a));
    a->type = hipMemoryTypeDevice;
    a->devicePointer = (void*)p;
    if (g_track_host) {
        auto it = g_allocs.upper_bound((uintptr_t)p);
        const bool dev = it != g_allocs.begin() && (uintptr_t)p < std::prev(it)->first + std::prev(it)->second;
        if (!dev) {
            a->type = hipMemoryTypeHost;
            a->devicePointer = nullptr;
            a->hostPointer = (void*)p;
        }
    }
    return hipSuccess;
}
hipError_t hipFuncSetAttribute(const void*, hipFuncAttribute, int v) {
    return v <= 160 * 1024 ? hipSuccess : hipErrorInvalidValue;
}
hipError_t hipGetLastError() {
    hipError_t e = emu::g_last;
    emu::g_last = hipSuccess;
    return e;
}
hipError_t hipPeekAtLastError() { return emu::g_last; }
const char* hipGetErrorString(hipError_t e) {
    switch (e) {
        case hipSuccess: return "hipSuccess";
        case hipErrorInvalidValue: return "hipErrorInvalidValue";
        case hipErrorOutOfMemory: return "hipErrorOutOfMemory";
        default: return "hipError (emulation)";
    }
}
hipError_t hipGetSymbolAddress(void** p, const void* sym) {
    *p = (void*)sym;
    return hipSuccess;
}
