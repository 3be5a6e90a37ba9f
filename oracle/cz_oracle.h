/*
 * cz_oracle.h - CPU restatement of colizig's block-FP8 MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the oracle the HIP library is checked
 * against; it is never linked into, loaded by or called from the product
 * library.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg use it, and only as the reference results / the timed CPU baseline.
 *
 * Every function restates one function of the reference (Zig 0.16 sources,
 * which cannot be compiled here: no zig toolchain) with the same operation
 * order, citing the reference file:line it follows.  The SIMD width of the
 * reference (`std.simd.suggestVectorLength`) is fixed at L = 8 lanes, the
 * value on the reference's AVX2 development machine (docs/OPS.md:25-27).
 *
 * Parity pins (what checks each function against something other than
 * itself) are listed in the header comment of cz_oracle.c.
 */
#ifndef CZ_ORACLE_H
#define CZ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CZO_BLOCK 128u /* fp8.zig:13 */
#define CZO_LANES 8u   /* fp8.zig:68, matmul.zig:15 on AVX2 */

/* moe.zig:23-46 `Dims` */
typedef struct czo_dims {
    uint32_t hidden;
    uint32_t experts;
    uint32_t topk;
    uint32_t inter;
    uint32_t shared_inter; /* 0 = no shared expert */
    uint32_t norm_topk;    /* bool */
} czo_dims;

/* moe.zig:50-100 `Fp8Matrix`: row-major [rows, cols] E4M3 bytes plus
 * [nblk(rows), nblk(cols)] f32 block scales. */
typedef struct czo_fp8mat {
    const uint8_t *w;
    const float *s;
    uint32_t rows;
    uint32_t cols;
} czo_fp8mat;

/* moe.zig:102-117 `Expert` */
typedef struct czo_expert {
    czo_fp8mat gate; /* [inter, hidden] */
    czo_fp8mat up;   /* [inter, hidden] */
    czo_fp8mat down; /* [hidden, inter] */
} czo_expert;

/* moe.zig:297-338 `Layer`.  The reference's shared expert is a resident
 * NativeMatrix (f32/bf16); the Qwen4-Exp-style configuration stores it as
 * block-FP8, so here it is an Fp8Matrix evaluated with the same S==1 fused
 * kernel as the routed experts (fp8.zig:137-160). */
typedef struct czo_layer {
    czo_dims d;
    const float *router;       /* [experts, hidden] f32 */
    const czo_expert *experts; /* [experts] */
    czo_fp8mat sh_gate_proj;   /* [shared_inter, hidden] */
    czo_fp8mat sh_up_proj;     /* [shared_inter, hidden] */
    czo_fp8mat sh_down_proj;   /* [hidden, shared_inter] */
    const float *sh_gate;      /* [hidden] f32 */
    const float *router_bias;  /* [experts] added to each logit, or NULL (the reference: none) */
    /* A NativeMatrix shared expert (moe.zig:300-303: f32 rows, or BF16 rows
     * widened exactly, since dotBf16 is dotF32's order on the widened values,
     * matmul.zig:60-110): when set, used instead of the block-FP8 one. */
    const float *sh_native_gate;  /* [shared_inter, hidden] */
    const float *sh_native_up;    /* [shared_inter, hidden] */
    const float *sh_native_down;  /* [hidden, shared_inter] */
} czo_layer;

/* ---- fp8.zig ---------------------------------------------------------- */
size_t czo_nblk(size_t x);                            /* fp8.zig:19-21 */
float czo_e4m3_decode(uint8_t b);                     /* fp8.zig:40-51 */
const float *czo_e4m3_lut(void);                      /* fp8.zig:33-38 */
void czo_decode_lane(const uint8_t *bytes, float sc, float *out8); /* fp8.zig:80-106 */
void czo_dequant_row(float *out, const uint8_t *w, const float *scale_row, size_t n); /* :123-130 */
void czo_dequant_matrix(float *out, const uint8_t *w, const float *scales, size_t rows, size_t cols);
float czo_dot_fp8_row(const float *x, const uint8_t *w, const float *scale_row, size_t n); /* :137-160 */
float czo_dot_fp8_row_scalar(const float *x, const uint8_t *w, const float *scale_row, size_t n);
void czo_matmul_fp8(float *y, const float *x, const uint8_t *w, const float *scales,
                    size_t S, size_t I, size_t O); /* fp8.zig:215-257 */

/* ---- matmul.zig --------------------------------------------------------- */
float czo_dot_f32(const float *a, const float *b, size_t n);        /* matmul.zig:60-82 */
float czo_dot_f32_scalar(const float *a, const float *b, size_t n);
void czo_matmul_f32(float *y, const float *x, const float *w, size_t S, size_t I, size_t O); /* :21-33 */

/* ---- activation.zig ----------------------------------------------------- */
float czo_expf(float x); /* stands in for Zig's f32 @exp; see cz_oracle.c */
void czo_expf_array(const float *in, float *out, size_t n);
float czo_sigmoid(float x); /* activation.zig:9-16 */
float czo_silu(float x);    /* activation.zig:18-20 */

/* ---- moe.zig ------------------------------------------------------------ */
/* route (moe.zig:435-463): idx[K], gates[K]; logits_out (nullable) receives
 * the E post-exp values v_e = exp(l_e - max) that the top-k scans. */
void czo_route(const czo_layer *L, const float *xs, uint32_t *idx, float *gates, float *logits_out);
/* router logits only (tensors.zig:114-119 -> matmul.zig:21-33) */
void czo_router_logits(const czo_layer *L, const float *xs, float *logits);
/* moe.forward (moe.zig:409-426): S==1 -> forwardDense, S>1 -> forwardGrouped.
 * r_idx/r_gate (nullable) receive [S*K] routing.  Returns 0, or -1 on OOM. */
int czo_moe_forward(const czo_layer *L, const float *x, size_t S, float *out,
                    uint32_t *r_idx, float *r_gate);
/* forwardDense on every token (the S==1 path applied per token), for the
 * "grouped prefill ~= per-token dense" property (moe.zig:720-728). */
int czo_moe_forward_dense_each(const czo_layer *L, const float *x, size_t S, float *out,
                               uint32_t *r_idx, float *r_gate);

/* ---- parallel.zig ------------------------------------------------------- */
void czo_parallel_enable(uint32_t max_tasks); /* parallel.zig:23-26 (0 -> CPU count) */
void czo_parallel_disable(void);
uint32_t czo_parallel_max_tasks(void);
/* Chunk boundaries `chunks` would use (parallel.zig:50-76): writes up to
 * max_out [lo,hi) pairs; returns the number of chunks (1 when serial). */
uint32_t czo_chunk_bounds(size_t n, size_t work, uint32_t *lo_hi, uint32_t max_out);

/* ---- ExpertCache (moe.zig:121-249): LRU policy simulation ---------------- */
typedef struct czo_cache_stats {
    uint64_t hits, misses, loads, evictions, prefetch_hits, prefetch_wasted;
} czo_cache_stats;
/* Replays `n` demand gets of expert ids through an LRU of `cap` slots,
 * writing the slot each get landed in; returns resident count at the end. */
uint32_t czo_cache_replay(uint32_t cap, const uint32_t *ids, size_t n, int32_t *slot_out,
                          czo_cache_stats *st);

/* The same cache over (layer, expert) keys for every streamed layer, as one
 * pool of `nslots` slots (the library's HBM expert pool), replaying a log of
 * ops of 4 words (op, layer, expert, result):
 *   0 begin a layer's gets: the slots the previous layer pinned are free to
 *     evict again;
 *   1 get (moe.zig:221-240): a hit touches the LRU clock and consumes a
 *     prefetch mark; a miss fills a victim; the slot is pinned;
 *   2 prefetch (moe.zig:244-248): a no-op when resident, else a fill marked
 *     prefetched; dropped when every slot is pinned;
 *   3 warm fill into the first free slot (expert_usage.zig:137-160);
 *   4 every slot freed.
 * Victim (moe.zig:183-197): the first empty slot, else the least recently
 * used slot not pinned by the layer in flight; evicting a prefetched slot
 * counts as wasted.  Writes each op's result in the log's encoding (get:
 * slot | 0x80000000 on a hit; prefetch: slot, 0xfffffffe resident,
 * 0xffffffff dropped; warm: slot; others 0) to res_out; returns the number
 * of resident entries at the end, or -1 when a get finds every slot pinned. */
typedef struct czo_pool_stats {
    uint64_t hits, misses, loads, evictions, prefetch_issued, prefetch_hits, prefetch_wasted;
} czo_pool_stats;
int64_t czo_pool_replay(uint32_t nslots, const uint32_t *ops, size_t n, uint32_t *res_out, czo_pool_stats *st);

/* ---- the decode chain (qwen3moe/model.zig:228-232 around the MoE block) -- */
/* rmsnorm.zig:32-40 `rms` with a unit weight: f64 sum of squares, mean
 * rounded to f32, r = 1/sqrt(mean + eps) in f32, out = x * r. */
void czo_rms_unit(float *out, const float *x, size_t n, float eps);
/* x <- x + moe(rms(x)) for one layer (S rows).  xn (nullable) gets the
 * router input. */
int czo_chain_layer(const czo_layer *L, float *x, size_t S, float eps, float *xn_out,
                    uint32_t *r_idx, float *r_gate);

#ifdef __cplusplus
}
#endif
#endif
