/*
 * colizig_hip.h - C-ABI of libcolizig_hip.so, the MI355X (gfx950) block-FP8
 * MoE expert path for colizig.
 *
 * Plain C types only (pointers, sizes, ints).  Two groups of entry points:
 *
 *  1. The six symbols colizig's engine already resolves by name
 *     (src/backend/gpu.zig:84-89) with the exact signatures of its extern fn
 *     types (src/backend/gpu.zig:20-34), replacing the CUDA DLL
 *     (src/backend/cuda/colizig_cuda.cu:171-284).  Same return codes, same
 *     ownership (caller-owned host pointers valid for the call), same
 *     MXCSR save/restore at every entry.
 *
 *  2. Optional MoE-level extensions (colizig_hip_*).  A loader that finds any
 *     of them missing keeps using group 1 only, the loader's existing rule
 *     (gpu.zig:84-89).  Same error convention: 0 ok, negative = the caller
 *     falls back to its CPU path.
 *
 * Not thread-safe across calls on one process (one global context, as the
 * CUDA DLL): the caller serialises, as gpu.zig:55-62 does.
 */
#ifndef COLIZIG_HIP_H
#define COLIZIG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* 1. the existing backend ABI                                              */
/* ------------------------------------------------------------------------ */

/* Replaces colizig_cuda.cu:171-187 (InitFn, gpu.zig:20).  Idempotent.
 * 0 ok; -1 no device; -2 set-device failed; -3 device query failed;
 * -4 device constant setup failed. */
int colizig_cuda_init(void);

/* Replaces colizig_cuda.cu:189-191 (NameFn, gpu.zig:22).  "" before init;
 * library-owned static buffer. */
const char *colizig_cuda_device_name(void);

/* Replaces colizig_cuda.cu:195-202 (SetBudgetFn, gpu.zig:23).  Bytes of HBM
 * the keyed weight cache may hold; 0 disables it.  Clamped to
 * free - free/8.  No-op before init. */
void colizig_cuda_set_vram_budget(uint64_t bytes);

/* Replaces colizig_cuda.cu:204-209 (StatsFn, gpu.zig:24).  NULL-tolerant. */
void colizig_cuda_stats(uint64_t *hits, uint64_t *misses, uint64_t *uploaded_mib, uint64_t *resident);

/* Replaces colizig_cuda.cu:211-224 (ShutdownFn, gpu.zig:21).  Frees every
 * device allocation (also the MoE layers below) and resets the context;
 * safe when not initialised. */
void colizig_cuda_shutdown(void);

/* Replaces colizig_cuda.cu:228-284 (MatmulFp8Fn, gpu.zig:25-34), called from
 * src/ops/fp8.zig:182.  Synchronous:
 *   y[S,O] = x[S,I] @ (e4m3(w[O,I]) * scales[o/128, i/128])^T
 * w row-major [O,I] E4M3 (OCP e4m3fn), scales row-major
 * [ceil(O/128), ceil(I/128)] f32.  key 0 = upload w every call; non-zero =
 * keep w in the HBM cache under that key (fp8 key scheme moe.zig:97-99).
 * 0 ok; -1 bad args / not initialised; -2 device alloc; -3 H2D copy;
 * -4 launch; -5 D2H copy / kernel fault. */
int colizig_cuda_matmul_fp8(float *y, const float *x, const unsigned char *w, const float *scales, int S, int I,
                            int O, uint64_t key);

/* Device-resident form of the keyed matmul above for the FP8 attention
 * projections (src/qwen3moe/attn.zig:206-208 q/k/v, :260 o, keyed by
 * attnKey, attn.zig:47-50) and any other Fp8Matrix at decode.
 * colizig_hip_matrix_load puts w/scales under `key` in the same HBM cache
 * (synchronous upload; the budget of colizig_cuda_set_vram_budget must be
 * set: -8 otherwise); a later load or host matmul may evict the slot, so
 * finish device calls that read a slot before loading what may replace it.
 * colizig_hip_matmul_fp8_dev: y_dev[S,O] = x_dev[S,I] @ (e4m3(w) *
 * scales)^T with the matrix resident under key, asynchronous on `stream`
 * (NULL = the library's stream); x_dev, y_dev 16-byte aligned.  -7 key not
 * resident; -1 bad args or a shape other than the resident one; -4 launch. */
int colizig_hip_matrix_load(uint64_t key, const unsigned char *w, const float *scales, int I, int O);
int colizig_hip_matmul_fp8_dev(float *y_dev, const float *x_dev, int S, int I, int O, uint64_t key, void *stream);

/* Several keyed FP8 matrices of one row width I on the same input rows x_dev
 * [S][I] in one launch: y_devs[m] [S][Os[m]] = x . dequant(W_keys[m])^T,
 * each bit-identical to colizig_hip_matmul_fp8_dev of that key alone.  For a
 * caller that has a layer's q, k and v projections together (the reference
 * makes them three matmulFp8Keyed calls, qwen3moe/attn.zig:206-208): one
 * launch instead of three; the 1 MiB k and v matrices are launch-bound on
 * their own.  n in 1..4, every key resident as FP8 [Os[m]][I].  Returns 0,
 * -1 bad arguments or a key resident with another shape or type, -7 a key
 * not resident, -4 launch failed.  No counterpart in the reference. */
int colizig_hip_matmul_fp8_dev_multi(int n, float *const *y_devs, const uint64_t *keys, const int *Os,
                                     const float *x_dev, int S, int I, void *stream);

/* BF16 rows (lm_head and the other BF16 NativeMatrix GEMVs: dotBf16,
 * src/ops/matmul.zig:84-110; tensors.zig's NativeMatrix(bf16).matmul) on
 * device activations: colizig_hip_matrix_load_bf16 puts w [O][I] (BF16 bits)
 * under `key` in the same HBM cache; colizig_hip_matmul_bf16_dev computes
 * y_dev[S,O] with every dot in dotBf16's operation order (bit-identical to
 * the reference), asynchronous on `stream`.  I = 32 * {8,16,32,64,96,128}.
 * Return codes as for the FP8 pair; a key loaded as the other type is -1. */
int colizig_hip_matrix_load_bf16(uint64_t key, const uint16_t *w, int I, int O);
int colizig_hip_matmul_bf16_dev(float *y_dev, const float *x_dev, int S, int I, int O, uint64_t key, void *stream);

/* ------------------------------------------------------------------------ */
/* 2. MoE-level extensions                                                   */
/* ------------------------------------------------------------------------ */

/* Mirrors src/qwen38/moe.zig:23-46 `Dims` (shape contract of one layer). */
typedef struct colizig_dims {
    uint32_t hidden;       /* H */
    uint32_t experts;      /* E */
    uint32_t topk;         /* K */
    uint32_t inter;        /* I, routed moe_intermediate */
    uint32_t shared_inter; /* SI, 0 = no shared expert */
    uint32_t norm_topk;    /* renormalise gates over the top-k */
} colizig_dims;

/* Bit-exact dequantisation hook (fp8.zig:123-130 semantics: one f32
 * multiply e4m3(b) * scale, the same arithmetic the GEMV kernels use in
 * registers).  Host pointers: out[rows*cols] f32, w[rows*cols] E4M3,
 * scales[ceil(rows/128)*ceil(cols/128)].  No counterpart in the reference:
 * it exists so the dequantised weights can be compared bit for bit. */
int colizig_hip_dequant_fp8(float *out, const unsigned char *w, const float *scales, int rows, int cols);

/* Registers one MoE layer: replaces Layer.load (moe.zig:306-328).
 * router[E*H] f32 (the reference's `gate.weight`, moe.zig:316) is copied
 * into HBM.  Re-registering a layer frees its previous weights.  Experts
 * start absent; forward fails with -6 until every expert is loaded. */
int colizig_hip_layer_init(uint32_t layer, const colizig_dims *dims, const float *router);

/* Copies expert `expert` of `layer` into its HBM slot: replaces loadExpert
 * (moe.zig:251-292) + ExpertCache.fill (moe.zig:199-217).  gate/up are
 * [I,H] E4M3 with [ceil(I/128), ceil(H/128)] scales, down is [H,I] with
 * [ceil(H/128), ceil(I/128)] scales. */
int colizig_hip_expert_load(uint32_t layer, uint32_t expert, const unsigned char *gate_w, const float *gate_s,
                            const unsigned char *up_w, const float *up_s, const unsigned char *down_w,
                            const float *down_s);

/* Shared expert of a layer (moe.zig:300-303, 319-325), block-FP8:
 * gate/up [SI,H], down [H,SI], sh_gate[H] f32 (shared_expert_gate.weight). */
/* NativeMatrix weights (src/model/tensors.zig:65-120), as the reference
 * loads a router or shared expert stored in f32 or BF16.
 * colizig_hip_layer_set_router_bf16: the router as BF16 bits [E][H] (replaces
 * the f32 one; logits in dotBf16's order, matmul.zig:84-110, bit for bit).
 * colizig_hip_layer_set_shared_native: the shared expert's gate, up [SI][H]
 * and down [H][SI] rows as f32 (dtype 0) or BF16 bits (dtype 1), evaluated
 * with dotF32 / dotBf16 rows (moe.zig:300-303, 316-325, 467-479), plus
 * sh_gate [H] f32; replaces a block-FP8 shared expert.  Such a layer runs
 * the three-kernel decode and its shared-expert GEMVs (not the one-launch
 * decode) and is not served by colizig_hip_moe_forward_dev_noalloc.
 * -1 bad args / no shared expert in the dims; -2 alloc; -3 copy. */
int colizig_hip_layer_set_router_bf16(uint32_t layer, const uint16_t *router);
int colizig_hip_layer_set_shared_native(uint32_t layer, int dtype, const void *gate, const void *up,
                                        const void *down, const float *sh_gate);

int colizig_hip_layer_set_shared(uint32_t layer, const unsigned char *gate_w, const float *gate_s,
                                 const unsigned char *up_w, const float *up_s, const unsigned char *down_w,
                                 const float *down_s, const float *sh_gate);

/* Optional per-expert router bias: logits[e] = dot(router[e], x) + bias[e]
 * (one f32 add after the dot).  bias[E] f32, NULL clears it.  No counterpart
 * in the reference, whose route has no bias term (moe.zig:435-463): a
 * workload-shaping hook that skews routing (e.g. Zipf-distributed expert
 * popularity) for prefill and streaming-tier benchmarks. */
int colizig_hip_layer_set_router_bias(uint32_t layer, const float *bias);

/* moe.forward (moe.zig:409-426) on host pointers, synchronous:
 * out[S*H] = MoE(x[S*H]).  routed_idx[S*K] / routed_gates[S*K] (nullable)
 * receive each token's top-k expert ids and gates in selection order.
 * S = 1..15 runs the decode kernels (one GEMV per token and slot, combine in
 * top-k order, as forwardDense); S >= 16 with H, I, SI multiples of 128 runs
 * the grouped regime (forwardGrouped, moe.zig:597-665): dispatch of the S*K
 * slots into per-expert row lists, grouped MFMA GEMMs, combine with the
 * shared expert first and the experts in ascending id order.
 * 0 ok; -1 bad args; -2 alloc; -3 H2D; -4 launch; -5 D2H/fault;
 * -6 layer not registered or experts missing. */
int colizig_hip_moe_forward(uint32_t layer, const float *x, int S, float *out, uint32_t *routed_idx,
                            float *routed_gates);

/* Same on device pointers, asynchronous on `stream` (a hipStream_t; NULL =
 * the library's stream).  Pointers must stay valid until the stream
 * reaches the end of this work.  Activation buffers (x_dev, out_dev, and
 * x_dev of the chain and stream entry points below) must be 16-byte
 * aligned, as hipMalloc returns them; -1 otherwise. */
int colizig_hip_moe_forward_dev(uint32_t layer, const float *x_dev, int S, float *out_dev, uint32_t *idx_dev,
                                float *gates_dev, void *stream);

/* No counterpart in the reference.  colizig_hip_moe_forward_dev for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): same arguments, same
 * kernels, same results, bit for bit.  Its scratch (normalised rows, logits,
 * routing, expert hidden rows) lives in a static 4 MiB device array per GPU,
 * held until the process ends; nothing is allocated or freed.  Serves the
 * decode regime of resident layers: -1 with a message for a streamed layer,
 * for S that takes the grouped regime, or when
 * S*(H + E + 2K + 1 + K*I + SI) floats (each part rounded up to 256 bytes)
 * exceed 4 MiB.  Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, two threads' streams) race. */
int colizig_hip_moe_forward_dev_noalloc(uint32_t layer, const float *x_dev, int S, float *out_dev,
                                        uint32_t *idx_dev, float *gates_dev, void *stream);

/* Decode chain over layers [layer0, layer0+nlayers) on device memory:
 *   x <- x + MoE_l(rmsnorm(x)),  rmsnorm(x)_i = x_i / sqrt(mean(x^2) + eps)
 * (unit-weight RMSNorm; the residual stream the MoE blocks sit in,
 * qwen3moe/model.zig:228-231).  x_dev[S*H] is updated in place.  Optional
 * per-layer traces (device pointers, NULL = off): xn_trace[nlayers*S*H] the
 * router inputs, idx_trace/gates_trace[nlayers*S*K] the routing.
 * Asynchronous on `stream` (NULL = library stream). */
int colizig_hip_chain_decode(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps, float *xn_trace,
                             uint32_t *idx_trace, float *gates_trace, void *stream);

/* Captures colizig_hip_chain_decode (traces off) into a HIP graph and
 * returns a handle (>0) for colizig_hip_graph_launch; <0 on error.  The graph
 * holds the layers' device buffers: colizig_hip_graph_launch returns -1
 * (launching nothing) once a captured layer has been re-registered, had its
 * router bias added or removed, or been switched to streaming. */
int64_t colizig_hip_chain_graph_create(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps);
int colizig_hip_graph_launch(int64_t handle, void *stream);
void colizig_hip_graph_destroy(int64_t handle);

/* Per-kernel timing: one chain step (x_dev advances as in
 * colizig_hip_chain_decode), then for each of the router, gate/up and down
 * kernels a HIP graph of `reps` passes over the layers launching only that
 * kernel is replayed between two events on the library stream.  us_out[3]
 * receives each kernel's mean duration per launch in microseconds. */
int colizig_hip_chain_kernel_times(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps, int reps,
                                   float *us_out);

/* One-launch-per-layer decode.  colizig_hip_chain_decode and its graph run
 * a batch-1 chain of resident layers as one kernel per layer (plus one final
 * residual add per chain) when the device has 8 XCDs x 32 CUs and every layer
 * has no shared expert, hidden 512, 1024 or 2048, at most 128 experts, K at
 * most 32, I a multiple of 128 and K*I/1024 in {1, 2, 4, 6, 8} (the Qwen3-30B-A3B shape
 * and config 1 qualify); otherwise the three-kernel decode.  Results are the same within the 1e-3 bar, routing
 * bit-identical.  colizig_hip_set_fused_decode(0) turns it off (returns the
 * previous setting); colizig_hip_fused_decode_active says whether a chain
 * would take it.  Its kernels exchange data between workgroups with bounded
 * waits: a wait that runs out makes the next colizig_hip_sync return -5 (the
 * step's results are then invalid).  colizig_hip_chain_fused_times: per
 * layer launch and final-kernel mean durations (us_out[2]) from replayed
 * graphs of `reps` steps, x_dev advancing.  No counterpart in the reference. */
int colizig_hip_set_fused_decode(int enable);

/* Predicted experts in the one-launch decode (mode 1, the default): each
 * layer's kernel also takes the next layer's top-k of its router logits on
 * this layer's router input, and the next kernel requests those experts'
 * rows before its own routing is known; a slot whose predicted expert was
 * not picked loads the picked one after the routing.  Routing, gates and
 * outputs are those of the layer's own routing either way.  0 turns it off;
 * 2 and 3 spoil the prediction on purpose (no slot keeps its prediction;
 * slot 0 does not) to exercise the late loads.  Returns the previous mode,
 * -1 for a mode outside 0..3.  No counterpart in the reference. */
int colizig_hip_set_fused_predict(int mode);

/* Counts since the last call: out[0] slots that had a predicted expert,
 * out[1] of them whose predicted expert was picked; then zeroes them.  0, or
 * -1 before any one-launch decode ran.  No counterpart in the reference. */
int colizig_hip_fused_predict_stats(uint64_t *out);

/* The one-launch decode's placement check: 1 when the census at init found
 * each of the 8 XCDs running exactly one workgroup of each rank 0..31 of a
 * 256-workgroup launch (the layout its exchanges inside an XCD need), 0
 * otherwise (every chain then takes the three-kernel decode), -1 before
 * init.  No counterpart in the reference. */
int colizig_hip_fused_placement(void);

/* Test hook of the one-launch decode's failure path: from the next chain on,
 * the layer at chain position pos (0-based; -1 turns the hook off) polls for
 * a tag no layer writes.  Its bounded waits give up after 20 ms, its kernel
 * finishes with what it read, and the next colizig_hip_sync returns -5 with
 * a message (the step's results are invalid).  Returns the previous
 * position.  No counterpart in the reference. */
int colizig_hip_set_fused_fault(int pos);

/* The grouped regime's GEMMs (prefill, batch decode) on FP8 MFMA
 * (v_mfma_scale_f32_32x32x64_f8f6f4: E4M3 weights as they are, the A rows as
 * three E4M3 terms with E8M0 exponents per 32 columns; the default) when
 * enable != 0, or on f16 MFMA (E4M3 weights widened exactly, A rows as f16
 * hi + lo); returns the previous setting.  Outputs stay within the 1e-3
 * relative L2 bar either way: over a 48-layer Qwen3-30B-A3B prefill chain
 * (512 tokens, 64 checked against the oracle's own chain) the residual
 * stream is within 4.8e-5 (FP8) and 7.9e-7 (f16), and routing is bit-exact
 * at every layer in both modes.  FP8 runs about 2% faster. */
int colizig_hip_set_prefill_fp8(int enable);
int colizig_hip_fused_decode_active(uint32_t layer0, uint32_t nlayers, int S);
int colizig_hip_chain_fused_times(uint32_t layer0, uint32_t nlayers, float *x_dev, float eps, int reps,
                                  float *us_out);

/* ---- streaming tier: experts in pinned host memory, cached in HBM -------
 * ExpertCache (moe.zig:121-249) + loadExpert redesigned for one GPU: one HBM
 * pool of fixed-size expert slots shared by every streamed layer, a global
 * LRU over (layer, expert) that spares the slots of the layer in flight,
 * fills by hipMemcpyAsync from pinned host memory on a side stream that the
 * compute stream waits for.  Prefetches go through a bounded priority queue
 * (Scheduler, src/runtime/io.zig:58-140): at one token the next streamed
 * layer's routing is predicted on the device from the current layer's
 * router input (MEDIUM), and the experts a layer routed for the previous
 * token (LastTokenPredictor, predict.zig:29-90) are queued LOW; they fill
 * while the current layer's expert kernels run. */

/* Creates the pool: floor(cap_bytes / slot) slots for experts of shape
 * (dims->hidden, dims->inter); a slot holds [3*I*H weight bytes | 3*nblk(I)*
 * nblk(H) f32 scales], rounded up to 16 bytes.  -1 when the pool would hold
 * fewer than top-k experts or one is configured already.
 * colizig_hip_stream_pool_free: unregisters every streamed layer, frees the
 * pool and zeroes its counters (a new pool may then be created). */
int colizig_hip_stream_pool_init(const colizig_dims *dims, uint64_t cap_bytes);
int colizig_hip_stream_pool_free(void);

/* Makes a registered layer stream its experts from host memory: host_ew /
 * host_es hold all E experts in the HBM slab layout (expert e at e*3*I*H
 * bytes: gate | up | down; scales at e*3*nblk(I)*nblk(H) floats), pinned
 * (colizig_hip_host_alloc), caller-owned, valid until the layer is
 * re-registered or the context shut down.  The layer's own HBM expert slab
 * is released. */
int colizig_hip_layer_stream_from_host(uint32_t layer, const unsigned char *host_ew, const float *host_es);

/* The same with one pinned slab of E experts, expert e at e * P bytes with P
 * = 3*I*H + 12*nblk(I)*nblk(H): gate | up | down weights, then their scales
 * (f32), so that a fill is one copy.  -1 when P is not a multiple of 16. */
int colizig_hip_layer_stream_from_host_packed(uint32_t layer, const unsigned char *host_slab);

/* colizig_hip_chain_decode over layers some of which stream: per streamed
 * layer the routing is read back to the host, misses are filled, the next
 * streamed layer's predicted experts are prefetched, then the expert kernels
 * run.  Returns after the last layer is enqueued (the host waits once per
 * streamed layer for its routing).  colizig_hip_moe_forward and
 * colizig_hip_moe_forward_dev accept streamed layers the same way; the
 * plain chain, its graph and the read-back hooks refuse them (-1). */
int colizig_hip_stream_decode(uint32_t layer0, uint32_t nlayers, float *x_dev, int S, float eps);

/* Routed-selection counters of every registered layer (bumpUsage,
 * src/qwen38/moe.zig:428-432, into ExpertUsage rows, expert_usage.zig:
 * 39-45): the routing kernels add one per pick of each token with integer
 * vector atomics.  colizig_hip_usage_read: counts[l * experts + e] for
 * layers layer0 .. layer0 + nlayers - 1 (zeros for a layer not registered
 * or of another expert count); waits for the library stream.
 * colizig_hip_usage_reset: every layer's counters to zero.  -1 bad args. */
int colizig_hip_usage_read(uint32_t layer0, uint32_t nlayers, uint32_t experts, uint64_t *counts);
int colizig_hip_usage_reset(void);

/* Learned priors for the streaming tier (src/runtime/expert_usage.zig:
 * ExpertUsage counts, :21-75; warmCaches, :137-180).
 * colizig_hip_stream_usage: the same counters as colizig_hip_usage_read.
 * colizig_hip_stream_warm: fills the pool's free slots with the streamed
 * (layer, expert) pairs of non-zero count, hottest first (one pool across
 * layers: the global top, where the reference warms each layer's cache with
 * its own top); complete on return; returns the number warmed (>= 0).
 * colizig_hip_stream_evict_all: every slot freed (counters and counts kept).
 * -1 bad args / no pool; -3 copy error. */
int colizig_hip_stream_usage(uint32_t layer0, uint32_t nlayers, uint32_t experts, uint64_t *counts);
int colizig_hip_stream_warm(uint32_t layer0, uint32_t nlayers, uint32_t experts, const uint64_t *counts);
int colizig_hip_stream_evict_all(void);

/* Pool counters, out[0..n) (n <= 27): hits, misses, loads, evictions,
 * prefetch_issued, prefetch_hits, prefetch_wasted (CacheStats,
 * moe.zig:121-139), bytes_h2d, slots, resident entries; next-layer
 * prediction: ids predicted, ids correct; last-token prediction: predicted,
 * correct (predict.zig:19-27); scheduler (io.zig:38-52): submitted, deduped,
 * upgraded, rejected_full, serviced HIGH / MEDIUM / LOW, cancelled,
 * queue_peak; token-level prediction: predicted, correct; layers run in
 * speculative runs, runs stopped by a pick without a slot. */
int colizig_hip_stream_stats(uint64_t *out, int n);
/* Opens a new statistics window: every counter above restarts at 0 (the
 * scheduler's queue peak at the queue's current length), and a prefetch
 * counts as a hit or as wasted only in the window that issued it.  The
 * pool's contents, LRU order and predictions are kept.  0, or -1 without a
 * pool.  No counterpart in the reference. */
int colizig_hip_stream_stats_reset(void);

/* Routing prediction for prefetch at one token: bit 0, the next streamed
 * layer's routing from the current layer's router input (its router and
 * routing kernels run once more on that input); bit 1, every later streamed
 * layer's from the chain's first streamed layer's router input (one router
 * launch over those layers, one routing launch).  Bit 2 (with bit 1, every
 * layer after the first streamed, f32 routers): the host leaves the
 * per-layer path.  After the first layer's prediction is serviced, every
 * later layer's slot map (all its resident experts) and its three kernels
 * are enqueued at once.  A layer that picks an expert without a slot stops
 * the rest of the run through a device word; that layer goes through the
 * per-layer path, and a new run starts after it.  The layers that ran are
 * then accounted in order (LRU touches, op log, counters, prediction
 * scores), as the per-layer path does.  Default 6.  Returns the previous
 * mode, -1 for a mode outside 0..7. */
int colizig_hip_stream_set_predict(int mode);

/* Op log of the pool's policy (test hook).  colizig_hip_stream_log(1) clears
 * and starts it, (0) stops it.  colizig_hip_stream_log_read copies up to
 * max_ops ops of 4 words (op, layer, expert, result) and returns the count
 * held.  op 0 = a layer's gets begin (its pins replace the previous layer's),
 * 1 = demand get (result: slot, | 0x80000000 on a hit), 2 = prefetch
 * (result: slot filled, 0xfffffffe already resident, 0xffffffff every slot
 * pinned: dropped), 3 = warm fill of a free slot (result: slot), 4 = every
 * slot freed. */
int colizig_hip_stream_log(int enable);
int64_t colizig_hip_stream_log_read(uint32_t *out, uint64_t max_ops);

/* The streaming tier's policy objects on their own: host code, no device
 * and no colizig_cuda_init needed.
 * Scheduler (io.zig:58-140) of expert keys (layer, id): create with a
 * capacity; submit (prio 0 HIGH, 1 MEDIUM, 2 LOW) returns 1 accepted (a
 * queued key is deduplicated and takes the stronger priority), 0 refused
 * (full); next returns 1 and the strongest-priority key (FIFO within a
 * priority), 0 when empty; cancel / has return 1 or 0; stats out[0..n)
 * (n <= 10): submitted, deduped, upgraded, rejected_full, serviced HIGH /
 * MEDIUM / LOW, cancelled, queue_peak, queued.
 * LastTokenPredictor (predict.zig:29-90): record(layer, ids) scores the
 * previous prediction of that layer and keeps the first topk ids; predict
 * copies them (returns how many); stats: ids predicted, ids correct.
 * -1 on an unknown handle or bad arguments. */
int64_t colizig_hip_sched_create(uint32_t capacity);
void colizig_hip_sched_destroy(int64_t h);
int colizig_hip_sched_submit(int64_t h, uint32_t layer, uint32_t id, int prio);
int colizig_hip_sched_next(int64_t h, uint32_t *layer, uint32_t *id);
int colizig_hip_sched_cancel(int64_t h, uint32_t layer, uint32_t id);
int colizig_hip_sched_has(int64_t h, uint32_t layer, uint32_t id);
int colizig_hip_sched_stats(int64_t h, uint64_t *out, int n);
int64_t colizig_hip_predictor_create(uint32_t topk);
void colizig_hip_predictor_destroy(int64_t h);
int colizig_hip_predictor_record(int64_t h, uint32_t layer, const uint32_t *ids, uint32_t n);
int colizig_hip_predictor_predict(int64_t h, uint32_t layer, uint32_t *out, uint32_t max);
int colizig_hip_predictor_stats(int64_t h, uint64_t *predicted, uint64_t *correct);
/* predictScored (predict.zig:61-72): the prediction of `layer` as at most
 * max (<= 64) rows, each with the predictor's accuracy so far as its
 * confidence (at least 0.1) and an expected use distance of 1; returns the
 * rows written, or -1 for an unknown handle. */
typedef struct colizig_prefetch_prediction {
    uint32_t layer;
    uint32_t expert;
    float confidence;
    uint32_t expected_use_distance;
} colizig_prefetch_prediction;
int colizig_hip_predictor_predict_scored(int64_t h, uint32_t layer, colizig_prefetch_prediction *out, uint32_t max);

/* ---- HBM plan (budget.plan, src/runtime/budget.zig:59-264, for HBM) ------
 * Where a model's MoE bytes go on one GPU: every layer keeps its router (f32
 * [E][H]), its shared expert and sigmoid gate, its routed-selection counters
 * and slot map resident; the routed experts are either all resident (when
 * they fit) or streamed through one HBM pool of expert slots shared by every
 * layer (the reference's per-layer cache cap, as one budget).  Host code:
 * with hbm_budget = 0 the budget is the device's free memory less an eighth
 * (the colizig_cuda_set_vram_budget clamp, needs colizig_cuda_init);
 * max_tokens sizes the forward's scratch. */
typedef struct colizig_hbm_plan {
    uint64_t hbm_budget;         /* bytes the plan may use */
    uint64_t per_expert_bytes;   /* one routed expert: weights + scales (one pool slot) */
    uint64_t per_layer_fixed;    /* router + shared expert + sh_gate + counters + slot map */
    uint64_t scratch;            /* the forward's scratch for max_tokens tokens */
    uint64_t fixed_resident;     /* layers * per_layer_fixed + scratch */
    uint64_t expert_bytes;       /* experts resident, or the pool */
    uint64_t total;              /* fixed_resident + expert_bytes */
    uint32_t all_resident;       /* 1: every expert resident, no streaming */
    uint32_t pool_slots;         /* streamed: expert slots of the pool */
    uint32_t expert_cap;         /* streamed: pool_slots / layers (the average cap per layer) */
    uint32_t ladder_cap;         /* the largest cap_ladder entry <= expert_cap (budget.zig:62), 0 below it */
    uint32_t fits;               /* 0: not even top-k slots fit after the fixed bytes */
    char reason[128];            /* "" when it fits */
} colizig_hbm_plan;
int colizig_hip_plan_hbm(const colizig_dims *dims, uint32_t layers, uint64_t hbm_budget, uint32_t max_tokens,
                         colizig_hbm_plan *out);

/* Bytes the forward's scratch holds now (grow-only; the plan's `scratch` for
 * max_tokens counts what a forward of that many tokens allocates in the
 * active prefill mode).  0, or -1 before init.  No counterpart in the
 * reference. */
int colizig_hip_work_bytes(uint64_t *out);

/* Pinned host memory for the host expert slabs. */
void *colizig_hip_host_alloc(uint64_t bytes);
void colizig_hip_host_free(void *p);

/* Fills a registered layer (router, every expert, shared expert) with
 * seeded synthetic weights directly in HBM: router and sh_gate f32
 * N(0, std_router); expert matrices N(0, std_w) quantised per 128x128 block
 * to E4M3 (RNE, saturating) with scale = amax/448 (1 for an all-zero
 * block).  A workload generator for benchmarks and tests, no counterpart in
 * the reference (its fixtures come from tools/gen_tiny_fixture.zig). */
int colizig_hip_layer_synth(uint32_t layer, uint64_t seed, float std_w, float std_router);

/* Copies a registered expert / the router / the shared expert back to host
 * memory (same layouts as the load calls); for checking and baselines. */
int colizig_hip_expert_read(uint32_t layer, uint32_t expert, unsigned char *gate_w, float *gate_s,
                            unsigned char *up_w, float *up_s, unsigned char *down_w, float *down_s);
int colizig_hip_router_read(uint32_t layer, float *router);
/* The whole expert slab of a layer in its HBM layout: ew[E * 3*I*H] bytes
 * (expert e: gate | up | down) and es[E * 3*nblk(I)*nblk(H)] scales. */
int colizig_hip_expert_slab_read(uint32_t layer, unsigned char *ew, float *es);
int colizig_hip_shared_read(uint32_t layer, unsigned char *gate_w, float *gate_s, unsigned char *up_w,
                            float *up_s, unsigned char *down_w, float *down_s, float *sh_gate);

/* Device-side f32 exp used by the router softmax and SiLU, evaluated on the
 * GPU for n inputs (host pointers); and the same function run on the host.
 * Test hooks for the router's bit-exactness. */
int colizig_hip_expf_dev(const float *in, float *out, int n);
float colizig_hip_expf_host(float x);

/* Small device-memory / stream / event helpers so callers without a GPU
 * framework can drive the *_dev entry points. */
void *colizig_hip_malloc(uint64_t bytes);
void colizig_hip_free(void *p);
int colizig_hip_memcpy_htod(void *dst, const void *src, uint64_t bytes);
int colizig_hip_memcpy_dtoh(void *dst, const void *src, uint64_t bytes);
int colizig_hip_memset(void *dst, int value, uint64_t bytes);
void *colizig_hip_stream(void); /* the library's stream */
int colizig_hip_sync(void);     /* synchronise the library's stream; -5 when a one-launch decode step
                                   since the last call reported an error */
/* Events on the library stream: create returns a handle; record puts it on
 * `stream` (NULL = library stream); elapsed_ms waits for `b`. */
int64_t colizig_hip_event_create(void);
int colizig_hip_event_record(int64_t ev, void *stream);
float colizig_hip_event_elapsed_ms(int64_t a, int64_t b);
void colizig_hip_event_destroy(int64_t ev);

/* Last error message of the library (static buffer). */
const char *colizig_hip_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
