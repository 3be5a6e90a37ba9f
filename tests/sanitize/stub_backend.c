/* A host-only stand-in for libcolizig_hip.so with the six symbols the
 * engine-side loader binds (src/backend/gpu.zig:84-89), for the loader's
 * sanitizer build: STUB_INIT_RC is what colizig_cuda_init returns, and
 * STUB_DROP_MATMUL leaves colizig_cuda_matmul_fp8 out.  The "matmul" writes
 * y[s][o] = s + o and succeeds. */
#include <stddef.h>
#include <stdint.h>

#ifndef STUB_INIT_RC
#define STUB_INIT_RC 0
#endif

static uint64_t calls;

int colizig_cuda_init(void) { return STUB_INIT_RC; }
const char *colizig_cuda_device_name(void) { return "host stub backend"; }
void colizig_cuda_shutdown(void) {}
void colizig_cuda_set_vram_budget(uint64_t bytes) { (void)bytes; }
void colizig_cuda_stats(uint64_t *hits, uint64_t *misses, uint64_t *uploaded_mib, uint64_t *resident) {
    if (hits) *hits = calls;
    if (misses) *misses = 1;
    if (uploaded_mib) *uploaded_mib = 2;
    if (resident) *resident = 3;
}
#ifndef STUB_DROP_MATMUL
int colizig_cuda_matmul_fp8(float *y, const float *x, const unsigned char *w, const float *scales, int S, int I,
                            int O, uint64_t key) {
    (void)x; (void)w; (void)scales; (void)I; (void)key;
    for (int s = 0; s < S; ++s)
        for (int o = 0; o < O; ++o) y[(size_t)s * O + o] = (float)(s + o);
    ++calls;
    return 0;
}
#endif
