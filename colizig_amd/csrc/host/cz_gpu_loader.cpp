// cz_gpu_loader.cpp - host-side loader of libcolizig_hip.so: the Linux
// counterpart of colizig's src/backend/gpu.zig, which loads the backend with
// LoadLibraryA/GetProcAddress on Windows only (gpu.zig:72-109) and is a stub
// elsewhere (gpu.zig:74-77).
//
// Same behaviour: best-effort init that writes one line to `err` and leaves
// the backend unavailable on any failure (library missing, a symbol missing,
// init rc != 0); calls serialised by a spinlock (gpu.zig:55-62); matmul
// returns false so the caller runs its CPU path (gpu.zig:175-190).  The
// MoE-level extension symbols are optional: missing ones only clear
// czgpu_has_moe().
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

namespace {

typedef int (*InitFn)(void);
typedef void (*ShutdownFn)(void);
typedef const char *(*NameFn)(void);
typedef void (*SetBudgetFn)(uint64_t);
typedef void (*StatsFn)(uint64_t *, uint64_t *, uint64_t *, uint64_t *);
typedef int (*MatmulFp8Fn)(float *, const float *, const unsigned char *, const float *, int, int, int, uint64_t);
typedef int (*MoeForwardFn)(uint32_t, const float *, int, float *, uint32_t *, float *);

void *handle = nullptr;
bool ready = false;
bool has_moe = false;
char name_buf[160];

ShutdownFn f_shutdown;
MatmulFp8Fn f_matmul_fp8;
SetBudgetFn f_set_budget;
StatsFn f_stats;
MoeForwardFn f_moe_forward;

std::atomic_flag call_lock = ATOMIC_FLAG_INIT;
struct Lock {
    Lock() { while (call_lock.test_and_set(std::memory_order_acquire)) {} }
    ~Lock() { call_lock.clear(std::memory_order_release); }
};

void put(char *err, size_t n, const char *msg) {
    if (err && n) snprintf(err, n, "%s", msg);
}

int fail(char *err, size_t n, const char *missing) {
    char b[256];
    snprintf(b, sizeof b, "--cuda: %s missing from libcolizig_hip.so - using CPU\n", missing);
    put(err, n, b);
    dlclose(handle);
    handle = nullptr;
    return 0;
}

template <typename T>
bool sym(T *out, const char *name) {
    *out = (T)dlsym(handle, name);
    return *out != nullptr;
}

}  // namespace

extern "C" {

// gpu.zig:72-109 init.  Returns 1 when the backend is up, 0 when the engine
// stays on the CPU; `err` receives the one-line report.
int czgpu_init(const char *lib_path, char *err, size_t errlen) {
    if (ready) return 1;
    handle = dlopen(lib_path ? lib_path : "libcolizig_hip.so", RTLD_NOW | RTLD_LOCAL);
    if (!handle) {
        put(err, errlen, "--cuda: libcolizig_hip.so not found - using CPU\n");
        return 0;
    }
    InitFn init_fn;
    NameFn name_fn;
    ShutdownFn shutdown_fn;
    MatmulFp8Fn matmul_fn;
    SetBudgetFn budget_fn;
    StatsFn stats_fn;
    if (!sym(&init_fn, "colizig_cuda_init")) return fail(err, errlen, "colizig_cuda_init");
    if (!sym(&name_fn, "colizig_cuda_device_name")) return fail(err, errlen, "colizig_cuda_device_name");
    if (!sym(&shutdown_fn, "colizig_cuda_shutdown")) return fail(err, errlen, "colizig_cuda_shutdown");
    if (!sym(&matmul_fn, "colizig_cuda_matmul_fp8")) return fail(err, errlen, "colizig_cuda_matmul_fp8");
    if (!sym(&budget_fn, "colizig_cuda_set_vram_budget")) return fail(err, errlen, "colizig_cuda_set_vram_budget");
    if (!sym(&stats_fn, "colizig_cuda_stats")) return fail(err, errlen, "colizig_cuda_stats");

    const int rc = init_fn();
    if (rc != 0) {
        char b[256];
        snprintf(b, sizeof b, "--cuda: no usable GPU device (colizig_cuda_init rc=%d) - using CPU\n", rc);
        put(err, errlen, b);
        dlclose(handle);
        handle = nullptr;
        return 0;
    }
    snprintf(name_buf, sizeof name_buf, "%s", name_fn());
    f_shutdown = shutdown_fn;
    f_matmul_fp8 = matmul_fn;
    f_set_budget = budget_fn;
    f_stats = stats_fn;
    has_moe = sym(&f_moe_forward, "colizig_hip_moe_forward");
    ready = true;
    char b[256];
    snprintf(b, sizeof b, "--cuda: GPU backend up - %s\n", name_buf);
    put(err, errlen, b);
    return 1;
}

// gpu.zig:116-122
void czgpu_deinit(void) {
    if (!ready) return;
    f_shutdown();
    if (handle) dlclose(handle);
    handle = nullptr;
    ready = false;
    has_moe = false;
}

int czgpu_available(void) { return ready ? 1 : 0; }   // gpu.zig:124-126
int czgpu_has_moe(void) { return has_moe ? 1 : 0; }
const char *czgpu_device_name(void) { return ready ? name_buf : ""; }  // gpu.zig:150-152

// gpu.zig:156-158
void czgpu_set_vram_budget(uint64_t bytes) {
    if (ready) f_set_budget(bytes);
}

// gpu.zig:160-170: one status line; returns its length (0 when unavailable)
int czgpu_stats_line(char *buf, size_t n) {
    if (!ready || !buf || !n) return 0;
    uint64_t hits = 0, misses = 0, up_mib = 0, resident = 0;
    f_stats(&hits, &misses, &up_mib, &resident);
    const uint64_t total = hits + misses;
    const double pct = total == 0 ? 0.0 : 100.0 * (double)hits / (double)total;
    return snprintf(buf, n, "  cuda: %llu matmuls  VRAM cache %.1f%% hit (%llu resident experts)  %llu MiB pushed H2D\n",
                    (unsigned long long)total, pct, (unsigned long long)resident, (unsigned long long)up_mib);
}

// gpu.zig:175-190: true (1) when the GPU handled the matmul; false (0) ->
// the caller runs the CPU path.
int czgpu_matmul_fp8(float *y, const float *x, const unsigned char *w, const float *scales, size_t S, size_t I,
                     size_t O, uint64_t key) {
    if (!ready) return 0;
    Lock lk;
    const int rc = f_matmul_fp8(y, x, w, scales, (int)S, (int)I, (int)O, key);
    return rc == 0 ? 1 : 0;
}

// MoE-level dispatch (optional symbol): true when the GPU ran moe.forward.
int czgpu_moe_forward(uint32_t layer, const float *x, size_t S, float *out, uint32_t *idx, float *gates) {
    if (!ready || !has_moe) return 0;
    Lock lk;
    return f_moe_forward(layer, x, (int)S, out, idx, gates) == 0 ? 1 : 0;
}

}  // extern "C"
