/*
 * cz_oracle_audit.c - exhaustive checks of the oracle's f32 exp against the
 * correctly rounded exp.  TEST INFRASTRUCTURE ONLY (part of the oracle).
 *
 * For each f32 input x the correctly rounded result is taken from the x87
 * long double expl (64-bit significand): its rounding to f32 is the correct
 * one unless expl's value lies within a few long-double ulps of an f32
 * rounding midpoint, which is counted as "ambiguous" and left out.
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include "cz_oracle.h"

typedef float (*czo_f32fn)(float);

typedef struct {
    uint64_t lo, hi; /* bit-pattern range [lo, hi) */
    czo_f32fn fn;
    uint64_t checked, ambiguous, mismatches, max_ulp;
    uint32_t first_bad;
} audit_job;

static int32_t ordered(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    return i < 0 ? (int32_t)0x80000000 - i : i;
}

static void *audit_run(void *p) {
    audit_job *j = (audit_job *)p;
    for (uint64_t u = j->lo; u < j->hi; ++u) {
        const uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        if (x != x) continue;
        const long double y = expl((long double)x);
        const float f = (float)y;
        const float got = j->fn(x);
        j->checked++;
        if (isfinite(f) && f > 0) {
            const long double fl = nextafterf(f, 0.0f), fh = nextafterf(f, INFINITY);
            const long double m1 = ((long double)f + fl) / 2, m2 = ((long double)f + fh) / 2;
            const long double tol = fabsl(y) * 0x1p-60L;
            if (fabsl(y - m1) < tol || fabsl(y - m2) < tol) {
                j->ambiguous++;
                continue;
            }
        }
        if (got != f && !(got == 0 && f == 0)) {
            if (j->mismatches == 0) j->first_bad = b;
            j->mismatches++;
            int64_t d = (int64_t)ordered(got) - (int64_t)ordered(f);
            if (d < 0) d = -d;
            if ((uint64_t)d > j->max_ulp) j->max_ulp = (uint64_t)d;
        }
    }
    return NULL;
}

/* Audits fn over the f32 bit patterns [lo, hi) with `threads` threads.
 * out[0..4] = checked, ambiguous, mismatches, max_ulp, first_bad_bits. */
void czo_exp_audit(czo_f32fn fn, uint64_t lo, uint64_t hi, uint32_t threads, uint64_t *out) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    audit_job jobs[64];
    pthread_t th[64];
    const uint64_t n = hi - lo, step = (n + threads - 1) / threads;
    for (uint32_t t = 0; t < threads; ++t) {
        memset(&jobs[t], 0, sizeof jobs[t]);
        jobs[t].lo = lo + t * step < hi ? lo + t * step : hi;
        jobs[t].hi = lo + (t + 1) * step < hi ? lo + (t + 1) * step : hi;
        jobs[t].fn = fn;
        pthread_create(&th[t], NULL, audit_run, &jobs[t]);
    }
    memset(out, 0, 5 * sizeof(uint64_t));
    out[4] = 0xffffffffu;
    for (uint32_t t = 0; t < threads; ++t) {
        pthread_join(th[t], NULL);
        out[0] += jobs[t].checked;
        out[1] += jobs[t].ambiguous;
        if (jobs[t].mismatches && out[2] == 0) out[4] = jobs[t].first_bad;
        out[2] += jobs[t].mismatches;
        if (jobs[t].max_ulp > out[3]) out[3] = jobs[t].max_ulp;
    }
}

/* Bitwise comparison of two f32 functions over [lo, hi): returns the number
 * of inputs (NaN inputs skipped) whose outputs differ in any bit. */
typedef struct {
    uint64_t lo, hi;
    czo_f32fn a, b;
    uint64_t diff;
    uint32_t first;
} cmp_job;

static void *cmp_run(void *p) {
    cmp_job *j = (cmp_job *)p;
    for (uint64_t u = j->lo; u < j->hi; ++u) {
        const uint32_t bb = (uint32_t)u;
        float x;
        memcpy(&x, &bb, 4);
        if (x != x) continue;
        const float ra = j->a(x), rb = j->b(x);
        uint32_t ia, ib;
        memcpy(&ia, &ra, 4);
        memcpy(&ib, &rb, 4);
        if (ia != ib) {
            if (!j->diff) j->first = bb;
            j->diff++;
        }
    }
    return NULL;
}

uint64_t czo_f32fn_compare(czo_f32fn a, czo_f32fn b, uint64_t lo, uint64_t hi, uint32_t threads,
                           uint32_t *first_diff) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    cmp_job jobs[64];
    pthread_t th[64];
    const uint64_t n = hi - lo, step = (n + threads - 1) / threads;
    for (uint32_t t = 0; t < threads; ++t) {
        memset(&jobs[t], 0, sizeof jobs[t]);
        jobs[t].lo = lo + t * step < hi ? lo + t * step : hi;
        jobs[t].hi = lo + (t + 1) * step < hi ? lo + (t + 1) * step : hi;
        jobs[t].a = a;
        jobs[t].b = b;
        pthread_create(&th[t], NULL, cmp_run, &jobs[t]);
    }
    uint64_t tot = 0;
    if (first_diff) *first_diff = 0xffffffffu;
    for (uint32_t t = 0; t < threads; ++t) {
        pthread_join(th[t], NULL);
        if (jobs[t].diff && tot == 0 && first_diff) *first_diff = jobs[t].first;
        tot += jobs[t].diff;
    }
    return tot;
}
