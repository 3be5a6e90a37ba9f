// cz_kernels.h - gfx950 kernels of the block-FP8 MoE expert path.
//
// HBM layout of one registered layer (LayerDev):
//   router  f32 [E][H]
//   experts one slab, expert e at e*ew_stride bytes: gate [I][H] | up [I][H] |
//           down [H][I] E4M3 (row-major, as the checkpoint stores them)
//   scales  one slab, expert e at e*es_stride floats: gate [nbI][nbH] |
//           up [nbI][nbH] | down [nbH][nbI]
//   shared  gate [SI][H] | up [SI][H] | down [H][SI] E4M3, scales likewise,
//           sh_gate f32 [H]
// Decode regime (S tokens, 1..32): three launches per layer
//   k_router_*  logits only, in the reference's dotF32 operation order (one
//               half-wave per expert row, every row element loaded before the
//               FMA chains run); optional unit-weight RMSNorm of the input
//   k_up_*      prologue: one wave turns the token's logits into top-k ids and
//               gates (softmax, strict '>' scan, f64 gates) in LDS; then
//               h[slot][r] = silu(Wg[r].x) * (Wu[r].x) for the block's rows,
//               128-bit loads, E4M3 decoded in registers, wave reduction; the
//               shared expert's rows and its sigmoid gate ride in the same grid
//   k_down_*    out[t][d] = xres + sum_z g_z (Wd_z[d] . h_z) + sgate Wsd[d].h_sh,
//               one wave per output row, all K experts' row loads in flight at
//               once; the weighted combine is fused into the GEMV in top-k order
#pragma once

#include "cz_device.h"

#define CZ_SEL_ARGS 8  // selected experts whose pool slots can travel in the kernel arguments

struct LayerDev {
    uint32_t H, E, K, I, SI, norm_topk;
    // a streamed layer's selected experts and their pool slots, sel[i] =
    // expert | slot << 16 (sel_n > 0: used instead of slot_map, no slot-map
    // upload).  Kept in the arguments' first 64 bytes, which every kernel
    // reads at entry.
    uint32_t sel_n;
    uint32_t sel[CZ_SEL_ARGS];
    uint32_t nbH, nbI, nbSI;
    const float *router;   // [E][H]
    const uint8_t *ew;     // expert weight slab
    const float *es;       // expert scale slab
    uint64_t ew_stride;    // bytes per expert = 3*I*H
    uint64_t es_stride;    // floats per expert = 3*nbI*nbH
    const uint8_t *sw;     // shared weights (gate|up|down) or null
    const float *ss;       // shared scales (gate|up|down)
    const float *sh_gate;  // [H]
    const float *router_bias;  // [E] added to each logit, or null (workload shaping only)
    const int32_t *slot_map;   // [E] HBM pool slot of each expert (layers streamed from
                               // host memory; ew/es then point at the pool), or null
    unsigned long long *usage; // [E] routed-selection counters (bumpUsage, moe.zig:428-432), or null
    const uint16_t *router_bf16;  // [E][H] BF16 router (NativeMatrix bf16), or null: `router` is f32
};

// bumpUsage (moe.zig:428-432): one count per pick of a token (all K of them,
// a repeated pick counted again), by integer vector atomics (order-free).
__device__ inline void cz_bump_usage(unsigned long long *usage, uint32_t E, uint32_t e) {
    if (usage && e < E) atomicAdd(usage + e, 1ull);
}

// Slot of expert e in ew/es: e itself for a resident layer, the pool slot for
// a streamed one (the host makes every selected expert resident before the
// layer's expert kernels run; a negative entry, or an expert missing from the
// argument table, maps to a valid slot so that a read stays in bounds).
__device__ inline uint64_t cz_slot(const LayerDev &L, uint32_t e) {
    if (L.sel_n) {  // e is one of the sel_n selected experts (else the first one's slot)
        uint32_t s = L.sel[0] >> 16;
#pragma unroll
        for (uint32_t i = 1; i < CZ_SEL_ARGS; ++i) s = (i < L.sel_n && (L.sel[i] & 0xffffu) == e) ? L.sel[i] >> 16 : s;
        return s;
    }
    return L.slot_map ? (uint64_t)max(L.slot_map[e], 0) : (uint64_t)e;
}

// Shared-expert gate pre-activation x . sh_gate of one token by one wave
// (moe.zig:475-477): lane l sums x[i] * g[i] for i = l, l + 64, ... in
// increasing order (terms past H are not added), then the DPP wave sum.  The
// loads of 16 terms per lane are in flight at once.
__device__ inline float cz_sgate_dot(const float *__restrict__ x, const float *__restrict__ g, uint32_t H,
                                     uint32_t lane) {
    float d = 0.0f;
    for (uint32_t i0 = 0; i0 < H; i0 += 64 * 16) {
        float xv[16], gv[16];
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) {
            const uint32_t i = min(i0 + 64 * q + lane, H - 1);  // clamped: in bounds
            xv[q] = x[i];
            gv[q] = g[i];
        }
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) {
            const float prod = xv[q] * gv[q];
            const float dn = d + prod;
            d = i0 + 64 * q + lane < H ? dn : d;
        }
    }
    return cz_wave_sum_dpp(d);
}

#define CZ_ROUTER_TT 4    // most tokens per router tile
#define CZ_MAX_E 1024     // experts supported by the top-k wave
#define CZ_MAX_K 64

// Scratch and routing buffers one layer's three kernels share.
struct StepArgs {
    LayerDev L;
    const float *x;        // [S][H] router input (rms = 0) or raw residual (rms = 1)
    float *xn;             // [S][H] router input, written by router block 0 when rms = 1
    float *logits;         // [S][E]
    uint32_t *idx;         // [S][K] top-k ids in selection order
    float *gates;          // [S][K]
    float *sgate;          // [S] shared-expert sigmoid gate
    float *h;              // [S*K][I] gated products of the routed experts
    float *hs;             // [S][SI] gated products of the shared expert
    const float *xres;     // [S][H] residual added to the output (nullable)
    float *out;            // [S][H]
    uint32_t *idx_trace;   // nullable [S][K]
    float *gates_trace;    // nullable [S][K]
    float *xn_trace;       // nullable [S][H]
    _Float16 *xh, *xl;     // nullable [S][H]: k_rms_rows also writes xn as f16 hi + lo (xn ~= hi + lo)
    uint8_t *xq, *xe;      // nullable: k_rms_rows_wg also writes xn as three E4M3 terms [3][S][H] with
                           // E8M0 exponents per 32 columns [3][S][H/32] (cz_q3_scale), the FP8-MFMA A rows
    // nullable: k_router_fast at S = 1, E <= 128 also routes the token in its
    // last workgroup (route_count: a zeroed device counter it leaves zeroed)
    // and writes the picks to host_idx, then host_seq to host_flag
    uint32_t *route_count, *host_idx, *host_flag;
    uint32_t host_seq;
    // nullable: a streamed token run with the host off the per-layer path.
    // Every kernel of a layer exits at once while the word is nonzero; the
    // gate/up kernel stores stop_code there when one of the token's picks
    // has no pool slot (slot_map < 0), and then neither publishes nor counts
    // the routing, so the layer and every later one leave x as it was.
    uint32_t *stop;
    uint32_t stop_code;
    uint32_t rms_ready;    // 1: the previous layer's combine already wrote xn (and its GEMM terms)
    int S;
    int tt;                // router tokens per tile (1..CZ_ROUTER_TT)
    int rms;
    float eps;
};

// A streamed token's stop word is set (an earlier layer, or this one, met a
// pick without a pool slot): the kernel does nothing.
__device__ __forceinline__ bool cz_stopped(const StepArgs &A) {
    return A.stop && __builtin_nontemporal_load(A.stop) != 0u;
}

// ---------------------------------------------------------------------------
// bit-exact dequantisation (test hook): out = e4m3(w) * scale, one multiply
// ---------------------------------------------------------------------------
__global__ void k_dequant_fp8(float *__restrict__ out, const uint8_t *__restrict__ w,
                              const float *__restrict__ scales, uint32_t rows, uint32_t cols, uint32_t nbc) {
    const uint64_t n = (uint64_t)rows * cols;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    if ((cols & 3u) == 0) {
        // four bytes per thread through v_cvt_pk_f32_fp8, as the GEMV kernels
        for (uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; q < n / 4; q += stride) {
            const uint64_t i = q * 4;
            const uint32_t r = (uint32_t)(i / cols), c = (uint32_t)(i - (uint64_t)r * cols);
            const uint32_t wd = ((const uint32_t *)w)[q];
            const float s = scales[(r / CZ_BLOCK) * nbc + c / CZ_BLOCK];
            const cz_float2 lo = cz_fp8x2_lo(wd), hi = cz_fp8x2_hi(wd);
            out[i + 0] = lo.x * s;
            out[i + 1] = lo.y * s;
            out[i + 2] = hi.x * s;
            out[i + 3] = hi.y * s;
        }
        return;
    }
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t r = (uint32_t)(i / cols), c = (uint32_t)(i - (uint64_t)r * cols);
        const float v = __builtin_amdgcn_cvt_f32_fp8((int)w[i], 0);
        out[i] = v * scales[(r / CZ_BLOCK) * nbc + c / CZ_BLOCK];
    }
}

// ---------------------------------------------------------------------------
// generic block-FP8 GEMM for the per-matmul ABI (any S, I, O):
// y[s][o] = sum_i x[s][i] * e4m3(w[o][i]) * scale[o/128][i/128]
// one wave per output row, lanes stride the columns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_gemm_fp8_generic(float *__restrict__ y, const float *__restrict__ x,
                                                          const uint8_t *__restrict__ w,
                                                          const float *__restrict__ scales, int S, int I, int O) {
    const int o = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (o >= O) return;
    const int lane = threadIdx.x & 63;
    const int nbi = (I + CZ_BLOCK - 1) / CZ_BLOCK;
    const uint8_t *wr = w + (uint64_t)o * I;
    const float *sr = scales + (uint64_t)(o / CZ_BLOCK) * nbi;
    const bool vec = (I % 4 == 0) && ((((uintptr_t)wr) & 3) == 0);
    for (int s = 0; s < S; ++s) {
        const float *xs = x + (uint64_t)s * I;
        float acc = 0.0f;
        if (vec) {
            for (int i = lane * 4; i < I; i += 256) {
                const uint32_t wd = *(const uint32_t *)(wr + i);
                const float sc = sr[i / CZ_BLOCK];
                const float x4[4] = {xs[i], xs[i + 1], xs[i + 2], xs[i + 3]};
                acc = cz_dot4_fp8(wd, sc, x4, acc);
            }
        } else {
            for (int i = lane; i < I; i += 64) {
                const float v = __builtin_amdgcn_cvt_f32_fp8((int)wr[i], 0) * sr[i / CZ_BLOCK];
                acc = __builtin_fmaf(xs[i], v, acc);
            }
        }
        acc = cz_wave_sum_dpp(acc);
        if (lane == 0) y[(uint64_t)s * O + o] = acc;
    }
}

// ---------------------------------------------------------------------------
// router logits in the reference's dotF32 order (matmul.zig:60-82): four
// accumulators x 8 lanes.  Half-wave lane j (0..31) owns chain j: it
// accumulates elements i + j of every 32-element step (matmul.zig:65-71),
// lanes 0..7 then take the 8-element steps (matmul.zig:72-76);
// total_l = ((0 + acc0_l) + acc1_l) + acc2_l) + acc3_l (matmul.zig:77-78),
// sum = sequential over l from -0 (matmul.zig:79), scalar fma tail
// (matmul.zig:80).
// ---------------------------------------------------------------------------
__device__ inline float cz_router_combine(float acc, uint32_t j, uint32_t half_base) {
    const float a1 = __shfl(acc, half_base + (j & 7) + 8, CZ_WAVE);
    const float a2 = __shfl(acc, half_base + (j & 7) + 16, CZ_WAVE);
    const float a3 = __shfl(acc, half_base + (j & 7) + 24, CZ_WAVE);
    float total = 0.0f;
    total = total + acc;  // lanes j<8 own acc0_l
    total = total + a1;
    total = total + a2;
    total = total + a3;
    float sum = -0.0f;
#pragma unroll
    for (uint32_t l = 0; l < 8; ++l) sum = sum + __shfl(total, half_base + l, CZ_WAVE);
    return sum;
}

// any n: the same order with loads inside the loop
__device__ inline float cz_router_dot(const float *__restrict__ a, const float *__restrict__ b, uint32_t n,
                                      uint32_t j, uint32_t half_base) {
    float acc = 0.0f;
    uint32_t i = 0;
    for (; i + 32 <= n; i += 32) acc = __builtin_fmaf(a[i + j], b[i + j], acc);
    for (; i + 8 <= n; i += 8)
        if (j < 8) acc = __builtin_fmaf(a[i + j], b[i + j], acc);
    float sum = cz_router_combine(acc, j, half_base);
    for (; i < n; ++i) sum = __builtin_fmaf(a[i], b[i], sum);
    return sum;
}

// Router input tile of one block into LDS: tokens t0..t0+nt-1, optionally
// RMS-normalised (rmsnorm.zig:32-40 with a unit weight, cz_rms_inv); block 0
// of the grid publishes the normalised rows.  blockDim.x == 64 (one wave).
__device__ inline void cz_router_stage_x(const StepArgs &A, float *smem, uint32_t t0, uint32_t nt) {
    const uint32_t H = A.L.H;
    for (uint32_t t = 0; t < nt; ++t) {
        const float *xs = A.x + (uint64_t)(t0 + t) * H;
        float inv = 1.0f;
        if (A.rms) {
            double ss = 0.0;
            for (uint32_t i = threadIdx.x; i < H; i += 64) {
                const double v = (double)xs[i];
                ss += v * v;
            }
            inv = cz_rms_inv(cz_wave_sum_f64(ss), H, A.eps);
        }
        const bool pub = A.rms && blockIdx.x == 0;
        for (uint32_t i = threadIdx.x; i < H; i += 64) {
            const float v = A.rms ? xs[i] * inv : xs[i];
            smem[t * H + i] = v;
            if (pub) {
                A.xn[(uint64_t)(t0 + t) * H + i] = v;
                if (A.xn_trace) A.xn_trace[(uint64_t)(t0 + t) * H + i] = v;
            }
        }
    }
}

// Fast-path staging of one token row whose NX = H/64 values per lane
// (columns lane + 64i) are in registers: optional RMS normalisation (the sum
// of squares in that order, then the DPP wave sum), the row into LDS slot t,
// and block 0's copy of the normalised row to xn (and xn_trace).
template <int NX>
__device__ __forceinline__ void cz_router_stage_row(const StepArgs &A, float *smem, uint32_t t0, uint32_t t,
                                                    float (&xv)[NX]) {
    constexpr uint32_t H = 64 * NX;
    const uint32_t lane = threadIdx.x;
    if (A.rms) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NX; ++i) ss += (double)xv[i] * (double)xv[i];
        const float inv = cz_rms_inv(cz_wave_sum_f64(ss), H, A.eps);
#pragma unroll
        for (int i = 0; i < NX; ++i) xv[i] = xv[i] * inv;
    }
#pragma unroll
    for (int i = 0; i < NX; ++i) smem[t * H + lane + 64 * i] = xv[i];
    if (A.rms && blockIdx.x == 0) {  // block-uniform
        float *xo = A.xn + (uint64_t)(t0 + t) * H + lane;
#pragma unroll
        for (int i = 0; i < NX; ++i) xo[64 * i] = xv[i];
        if (A.xn_trace) {
            float *xt = A.xn_trace + (uint64_t)(t0 + t) * H + lane;
#pragma unroll
            for (int i = 0; i < NX; ++i) xt[64 * i] = xv[i];
        }
    }
}

template <int M>
__device__ inline void cz_route_wave_m(const float *__restrict__ lg, uint32_t E, uint32_t K, uint32_t norm_topk,
                                       uint32_t *s_idx, float *s_gate, uint32_t &o_pos, uint32_t &o_id,
                                       float &o_gate);

// One wave per block, two experts per wave (one per half).  NS = H/32: every
// router element the lane needs is loaded into registers before the input
// tile is staged and the chains run.  With A.host_flag (one token, E <= 128)
// the last block to finish routes the token (the routing wave of the decode
// kernels on the logits, after an agent-scope fence on both sides of the
// block counter) and hands the picks to the host, in place of a routing
// launch.
template <int NS>
__global__ __launch_bounds__(64) void k_router_fast(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    constexpr uint32_t H = 32 * NS;
    const uint32_t E = A.L.E;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t half = lane >> 5, j = lane & 31, hb = half * 32;
    const uint32_t e = blockIdx.x * 2 + half;
    const uint32_t ec = min(e, E - 1);
    const uint32_t t0 = blockIdx.y * (uint32_t)A.tt;
    const uint32_t nt = min((uint32_t)A.tt, (uint32_t)A.S - t0);
    extern __shared__ float smem[];  // [nt][H]
    const float *wr = A.L.router + (uint64_t)ec * H + j;
    float w[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) w[i] = wr[32 * i];
    // the first token's row is requested with the router elements (no wait
    // between them); later tokens of the tile follow one by one
    {
        float xv[NS / 2];
#pragma unroll
        for (int i = 0; i < NS / 2; ++i) xv[i] = A.x[(uint64_t)t0 * H + lane + 64 * i];
        cz_router_stage_row<NS / 2>(A, smem, t0, 0, xv);
    }
    for (uint32_t t = 1; t < nt; ++t) {
        float xv[NS / 2];
#pragma unroll
        for (int i = 0; i < NS / 2; ++i) xv[i] = A.x[(uint64_t)(t0 + t) * H + lane + 64 * i];
        cz_router_stage_row<NS / 2>(A, smem, t0, t, xv);
    }
    __syncthreads();
    // the chain's LDS reads go in batches of CB, all in flight before the
    // batch's FMAs (read one by one, each FMA waited on its read's latency)
    constexpr int CB = NS < 32 ? NS : 32;
    for (uint32_t t = 0; t < nt; ++t) {
        const float *xs = smem + t * H + j;
        float acc = 0.0f;
#pragma unroll
        for (int i0 = 0; i0 < NS; i0 += CB) {
            float xb[CB];
#pragma unroll
            for (int q = 0; q < CB; ++q) xb[q] = xs[32 * (i0 + q)];
#pragma unroll
            for (int q = 0; q < CB; ++q) acc = __builtin_fmaf(xb[q], w[i0 + q], acc);
        }
        float lg = cz_router_combine(acc, j, hb);
        if (A.L.router_bias) lg = lg + A.L.router_bias[ec];
        if (j == 0 && e < E) A.logits[(uint64_t)(t0 + t) * E + e] = lg;
    }
    if (A.host_flag) {  // uniform
        __shared__ uint32_t s_last;
        __shared__ uint32_t s_ri[CZ_MAX_K];
        __shared__ float s_rg[CZ_MAX_K];
        __threadfence();  // this block's logits are visible to the last block
        if (threadIdx.x == 0) s_last = atomicAdd(A.route_count, 1u) == gridDim.x * gridDim.y - 1u ? 1u : 0u;
        __syncthreads();
        if (s_last) {
            __threadfence();  // every block's logits are visible here
            uint32_t o_pos = 0, o_id = 0;
            float o_gate = 0.0f;
            if (E <= 64)  // the routing launch's wave for E experts (cz_route_groups)
                cz_route_wave_m<1>(A.logits, E, A.L.K, A.L.norm_topk, s_ri, s_rg, o_pos, o_id, o_gate);
            else
                cz_route_wave_m<2>(A.logits, E, A.L.K, A.L.norm_topk, s_ri, s_rg, o_pos, o_id, o_gate);
            if (lane < A.L.K) A.host_idx[o_pos] = o_id;  // in pick order
            __threadfence_system();
            if (lane == 0) {
                *A.route_count = 0u;  // for the next launch (stream order)
                __hip_atomic_store(A.host_flag, A.host_seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    }
}

// Router logits of several layers for one token (the streaming tier's
// prediction of later layers' routing from one router input): logits[l][e]
// = router_l[e] . x (+ bias_l[e]) in the decode router's dotF32 order (so
// the same input gives the same logits); one wave per two experts of one
// layer (blockIdx.y).  H % 32 == 0.
struct RouterLayersArgs {
    const float *const *router;  // [n] router of each layer, [E][H]
    const float *const *bias;    // [n] its bias [E], or null
    const float *x;              // [H]
    float *logits;               // [n][E]
    uint32_t E, H;
};

__global__ __launch_bounds__(64) void k_router_layers(RouterLayersArgs A) {
    const uint32_t l = blockIdx.y, lane = threadIdx.x & 63, half = lane >> 5, j = lane & 31;
    const uint32_t e = blockIdx.x * 2 + half, ec = min(e, A.E - 1);
    const float *wr = A.router[l] + (uint64_t)ec * A.H + j;
    const float *xr = A.x + j;
    float acc = 0.0f;
    const uint32_t n = A.H / 32;
#pragma unroll 16
    for (uint32_t i = 0; i < n; ++i) acc = __builtin_fmaf(xr[32 * i], wr[32 * i], acc);
    float lg = cz_router_combine(acc, j, half * 32);
    const float *b = A.bias[l];
    if (b) lg = lg + b[ec];
    if (j == 0 && e < A.E) A.logits[(uint64_t)l * A.E + e] = lg;
}

// Publishes `seq` to a host-memory flag after everything before it on the
// stream (system-scope release).
__global__ void k_host_signal(uint32_t *flag, uint32_t seq) {
    if (threadIdx.x == 0) {
        __threadfence_system();
        __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// Many-token router input (S > 1, rms = 1): one wave per token writes xn =
// rms(x) (rmsnorm.zig:32-40 with a unit weight: the f64 sum of the squares,
// cz_rms_inv), and, when xh / xl are given, xn split into f16 hi + lo (the
// grouped GEMM's A operand).  Rows of up to CZ_RMS_MAXB * 2048 columns stay in
// registers, loaded at once; loads past H read column H - 64 + lane and add
// +0.  Longer rows are read twice.
#define CZ_RMS_PB 32   // columns per lane per batch
#define CZ_RMS_MAXB 2  // register-resident batches

__device__ __forceinline__ void cz_rms_store(const StepArgs &A, uint64_t o, float v) {
    A.xn[o] = v;
    if (A.xn_trace) A.xn_trace[o] = v;
    if (A.xh) {
        const _Float16 hv = (_Float16)v;
        A.xh[o] = hv;
        A.xl[o] = (_Float16)(v - (float)hv);
    }
}

// Activations for the FP8-MFMA grouped GEMMs: each 32-column group of a row
// as three E4M3 terms.  Term t of a group with max |r_t| = amax: k_t = the
// least k with amax <= 448 * 2^k (clamped to [-126, 127]), q_t = e4m3(r_t *
// 2^-k_t), r_{t+1} = r_t - 2^k_t * q_t (exact: q_t rounds r_t * 2^-k_t), the
// exponent byte k_t + 127; an all-zero group has byte 0 and zero terms.
__device__ __forceinline__ uint32_t cz_f32_to_e4m3(float v) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xffu;
}

struct CzQ3 {
    float inv, sc;  // 2^-k, 2^k (0 for an all-zero group)
    uint32_t eb;    // exponent byte
};

__device__ __forceinline__ CzQ3 cz_q3_scale(float amax) {
    if (!(amax > 0.0f)) return CzQ3{0.0f, 0.0f, 0u};
    const int ef = (int)((__builtin_bit_cast(uint32_t, amax) >> 23) & 0xffu);
    int k = (ef ? ef - 127 : -127) - 8;  // floor(log2 amax) - 8 (subnormals: below -127)
    if (amax > __builtin_ldexpf(448.0f, k)) ++k;
    k = max(-126, min(k, 127));
    return CzQ3{__builtin_ldexpf(1.0f, -k), __builtin_ldexpf(1.0f, k), (uint32_t)(k + 127)};
}

// e4m3 byte of r in the group's scale, and r less what the byte represents
__device__ __forceinline__ uint32_t cz_q3_term(float &r, const CzQ3 &s) {
    const uint32_t b = s.eb ? cz_f32_to_e4m3(r * s.inv) : 0u;
    r = r - cz_fp8x2_lo(b).x * s.sc;
    return b;
}

// Four consecutive columns r[0..3] of a 32-column group spread over 8
// consecutive lanes (lane % 8 = column / 4 within the group) to three E4M3
// terms: the group's |max| goes round its 8 lanes by DPP, the lane's four
// bytes of term t go to q + t * q_plane (a 4-byte aligned word), and the
// group's exponent byte of term t to e + t * e_plane from the lead lane.  All
// 8 lanes of a group execute it together; store = false skips the stores only.
__device__ __forceinline__ void cz_q3_group4(float (&r)[4], uint8_t *q, uint64_t q_plane, uint8_t *e,
                                             uint64_t e_plane, bool lead, bool store) {
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        float am = fmaxf(fmaxf(__builtin_fabsf(r[0]), __builtin_fabsf(r[1])),
                         fmaxf(__builtin_fabsf(r[2]), __builtin_fabsf(r[3])));
        am = fmaxf(am, cz_dpp<0xB1>(am));   // lanes xor 1
        am = fmaxf(am, cz_dpp<0x4E>(am));   // xor 2
        am = fmaxf(am, cz_dpp<0x141>(am));  // the mirror within 8: every lane of the 8
        const CzQ3 sc = cz_q3_scale(am);
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) word |= cz_q3_term(r[j], sc) << (8 * j);
        if (store) {
            *reinterpret_cast<uint32_t *>(q + t * q_plane) = word;
            if (lead) e[t * e_plane] = (uint8_t)sc.eb;
        }
    }
}

// One workgroup of 256 threads per token row (H % 256 == 0, H <= 1024 Q):
// the row is requested at once as 128-bit loads (Q per thread) and staged in
// LDS; wave 0 forms the f64 sum of squares (cz_rms_inv), every thread then
// writes its 4-column groups of xn (and xn_trace) and of the f16 split.  With
// a shared expert, wave 1 also forms its gate sigmoid(xn . sh_gate) in
// cz_sgate_dot's order (lane l: columns l, l + 64, ... increasing, then the
// DPP wave sum), its sh_gate elements requested with the row.
// The RMS rows of token `t` from its row v (thread tid holds float4 tid +
// 256 k): the row staged in LDS, the sum of squares by one wave in the decode
// order, then xn (and its f16 split or E4M3 terms, the shared-expert gate)
// written for A's layer.  Shared by k_rms_rows_wg and the combine that forms
// the next layer's rows (k_combine_rms).
template <int Q>
__device__ __forceinline__ void cz_rms_row_tail(const StepArgs &A, uint32_t t, float4 (&v)[Q], float *s_row,
                                                float *s_inv_p) {
    const uint32_t H = A.L.H, n4 = H / 4, tid = threadIdx.x, nq = H / 64;
    const uint64_t row = (uint64_t)t * H;
    const bool gate = A.L.SI != 0 && (tid >> 6) == 1;  // wave-uniform
    float g[16 * Q];
    if (gate) {
#pragma unroll
        for (uint32_t i = 0; i < 16 * Q; ++i) g[i] = A.L.sh_gate[(tid & 63) + 64 * min(i, nq - 1)];  // clamped
    }
    float &s_inv = *s_inv_p;
#pragma unroll
    for (uint32_t k = 0; k < Q; ++k)
        if (tid + 256 * k < n4) reinterpret_cast<float4 *>(s_row)[tid + 256 * k] = v[k];
    __syncthreads();
    if (tid < 64) {
        float a[16 * Q];
#pragma unroll
        for (uint32_t i = 0; i < 16 * Q; ++i) a[i] = s_row[tid + 64 * min(i, nq - 1)];
        double ss = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < 16 * Q; ++i) ss += i < nq ? (double)a[i] * (double)a[i] : 0.0;  // past H: + 0
        ss = cz_wave_sum_f64(ss);
        if (tid == 0) s_inv = cz_rms_inv(ss, H, A.eps);
    }
    __syncthreads();
    const float inv = s_inv;
    if (gate) {
        const uint32_t l = tid & 63;
        float d = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < 16 * Q; ++i) {
            const float y = s_row[l + 64 * min(i, nq - 1)] * inv;  // the xn value of column l + 64i
            const float prod = y * g[i];
            const float dn = d + prod;
            d = i < nq ? dn : d;
        }
        d = cz_wave_sum_dpp(d);
        if (l == 0) A.sgate[t] = cz_sigmoid(d);
    }
    typedef _Float16 cz_half4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (uint32_t k = 0; k < Q; ++k) {
        const uint32_t q = tid + 256 * k;
        if (q >= n4) break;
        const float4 y = make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv);
        reinterpret_cast<float4 *>(A.xn + row)[q] = y;
        if (A.xn_trace) reinterpret_cast<float4 *>(A.xn_trace + row)[q] = y;
        if (A.xh) {
            const cz_half4 hi = {(_Float16)y.x, (_Float16)y.y, (_Float16)y.z, (_Float16)y.w};
            const cz_half4 lo = {(_Float16)(y.x - (float)hi[0]), (_Float16)(y.y - (float)hi[1]),
                                 (_Float16)(y.z - (float)hi[2]), (_Float16)(y.w - (float)hi[3])};
            reinterpret_cast<cz_half4 *>(A.xh + row)[q] = hi;
            reinterpret_cast<cz_half4 *>(A.xl + row)[q] = lo;
        }
        if (A.xq) {  // the group of 32 columns is 8 consecutive lanes (H % 32 == 0: whole groups active)
            float r[4] = {y.x, y.y, y.z, y.w};
            cz_q3_group4(r, A.xq + row + 4 * q, (uint64_t)A.S * H, A.xe + (uint64_t)t * (H / 32) + q / 8,
                         (uint64_t)A.S * (H / 32), (q & 7u) == 0, true);
        }
    }
}

template <int Q>
__global__ __launch_bounds__(256) void k_rms_rows_wg(StepArgs A) {
    __shared__ __align__(16) float s_row[Q * 1024];
    __shared__ float s_inv;
    const uint32_t n4 = A.L.H / 4, tid = threadIdx.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(A.x + (uint64_t)blockIdx.x * A.L.H);
    float4 v[Q];
#pragma unroll
    for (uint32_t k = 0; k < Q; ++k) v[k] = x4[min(tid + 256 * k, n4 - 1)];  // clamped: in bounds
    cz_rms_row_tail<Q>(A, blockIdx.x, v, s_row, &s_inv);
}

// Rows longer than the workgroup form holds: one wave per token.
__global__ __launch_bounds__(256) void k_rms_rows(StepArgs A) {
    const uint32_t H = A.L.H;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4 + wave;
    if (t >= (uint32_t)A.S) return;  // wave-uniform
    const float *xs = A.x + (uint64_t)t * H;
    const uint64_t row = (uint64_t)t * H;
    const uint32_t nb = (H + 64 * CZ_RMS_PB - 1) / (64 * CZ_RMS_PB);
    double ss = 0.0;
    if (nb <= CZ_RMS_MAXB) {
        float v[CZ_RMS_MAXB][CZ_RMS_PB];
#pragma unroll
        for (uint32_t b = 0; b < CZ_RMS_MAXB; ++b)
            if (b < nb) {
#pragma unroll
                for (uint32_t q = 0; q < CZ_RMS_PB; ++q) v[b][q] = xs[min(64 * (CZ_RMS_PB * b + q), H - 64) + lane];
            }
#pragma unroll
        for (uint32_t b = 0; b < CZ_RMS_MAXB; ++b)
            if (b < nb) {
#pragma unroll
                for (uint32_t q = 0; q < CZ_RMS_PB; ++q)
                    ss += 64 * (CZ_RMS_PB * b + q) < H ? (double)v[b][q] * (double)v[b][q] : 0.0;
            }
        const float inv = cz_rms_inv(cz_wave_sum_f64(ss), H, A.eps);
#pragma unroll
        for (uint32_t b = 0; b < CZ_RMS_MAXB; ++b)
            if (b < nb) {
#pragma unroll
                for (uint32_t q = 0; q < CZ_RMS_PB; ++q) {
                    const uint32_t i = 64 * (CZ_RMS_PB * b + q) + lane;
                    if (i < H) cz_rms_store(A, row + i, v[b][q] * inv);
                }
            }
        return;
    }
    for (uint32_t i0 = 0; i0 < H; i0 += 64 * CZ_RMS_PB) {
        float v[CZ_RMS_PB];
#pragma unroll
        for (uint32_t q = 0; q < CZ_RMS_PB; ++q) v[q] = xs[min(i0 + 64 * q, H - 64) + lane];
#pragma unroll
        for (uint32_t q = 0; q < CZ_RMS_PB; ++q) ss += i0 + 64 * q < H ? (double)v[q] * (double)v[q] : 0.0;
    }
    const float inv = cz_rms_inv(cz_wave_sum_f64(ss), H, A.eps);
    for (uint32_t i = lane; i < H; i += 64) cz_rms_store(A, row + i, xs[i] * inv);
}

// Many-token router (S > 1): a workgroup of CZ_RT_TG x 256 threads computes
// CZ_RT_EXP experts x TOK tokens (TOK = 16, 8 or 4: fewer tokens per
// workgroup for small batches, so the grid still covers the CUs).  Thread (token group g, half-wave hw
// of its 256, lane j) owns experts 2hw, 2hw + 1 of the tile and tokens
// [g*NTT, (g+1)*NTT); lane j is chain j: it accumulates columns j, j + 32, ...
// in increasing order, exactly as the one-token kernel, so logits are
// bit-identical to the decode router's.  The router elements come from
// HBM/L2 into registers (a ring of CZ_RT_RING chunk sets, CZ_RT_RING - 1
// 256-column chunks ahead); the input chunk goes through LDS (two buffers,
// one barrier per chunk), and each LDS value feeds two FMAs.  The half-wave
// combine (cz_router_combine's additions, same order) reads the 32 chain sums
// from LDS, one thread per logit.  Input: xn when rms = 1 (k_rms_rows ran
// first), else x.  H % 256 == 0.
#define CZ_RT_EXP 16
#define CZ_RT_TG 2       // token groups (256 threads each)
#define CZ_RT_ACC_LD 36  // floats per (expert, token) row of chain sums (16 B aligned, b128 conflict-free)
#define CZ_RT_RING 4     // register sets of chunk operands in flight

template <int TOK, bool TM>
__global__ __launch_bounds__(256 * CZ_RT_TG) void k_router_tiled(StepArgs A) {
    constexpr uint32_t NTT = TOK / CZ_RT_TG;  // tokens per thread
    const LayerDev &L = A.L;
    const uint32_t H = L.H, E = L.E;
    const uint32_t tid = threadIdx.x, col = tid & 255, g = tid >> 8, hw = col >> 5, j = col & 31;
    // block b runs on XCD b % 8.  TM (more tokens than experts): grid (token
    // tiles, expert groups), so each XCD takes every eighth token tile with
    // all the expert groups and its L2 fetches its tokens' rows and the
    // router once; else grid (expert groups, token tiles), so each XCD's L2
    // fetches an eighth of the router and all the rows
    const uint32_t eg = TM ? blockIdx.y : blockIdx.x, tg = TM ? blockIdx.x : blockIdx.y;
    const uint32_t ea = min(eg * CZ_RT_EXP + 2 * hw, E - 1), eb = min(eg * CZ_RT_EXP + 2 * hw + 1, E - 1);
    const uint32_t t0 = tg * TOK;
    const uint32_t nt = min((uint32_t)TOK, (uint32_t)A.S - t0);
    constexpr uint32_t XBUF = 2 * TOK * 256, ACCN = CZ_RT_EXP * TOK * CZ_RT_ACC_LD;
    __shared__ __align__(16) float s_buf[XBUF > ACCN ? XBUF : ACCN];
    const float *src = A.rms ? A.xn : A.x;
    const float *wa = L.router + (uint64_t)ea * H + j, *wb = L.router + (uint64_t)eb * H + j;
    // this thread stages column `col` of tokens g*NTT .. g*NTT + NTT - 1 (clamped to nt - 1)
    const float *xcol = src + (uint64_t)t0 * H + col;
    float acc[2][NTT];
#pragma unroll
    for (uint32_t t = 0; t < NTT; ++t) acc[0][t] = acc[1][t] = 0.0f;
    float w[CZ_RT_RING][2][8], xv[CZ_RT_RING][NTT];
    const uint32_t nch = H / 256;
    auto load_chunk = [&](uint32_t r, uint32_t c) {
        const uint32_t c0 = min(c, nch - 1) * 256;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w[r][0][i] = wa[c0 + 32 * i];
            w[r][1][i] = wb[c0 + 32 * i];
        }
#pragma unroll
        for (uint32_t t = 0; t < NTT; ++t) xv[r][t] = xcol[(uint64_t)min(g * NTT + t, nt - 1) * H + c0];
    };
#pragma unroll
    for (uint32_t r = 0; r + 1 < CZ_RT_RING; ++r) load_chunk(r, r);
    for (uint32_t cb = 0; cb < nch; cb += CZ_RT_RING) {
#pragma unroll
        for (uint32_t r = 0; r < CZ_RT_RING; ++r) {
            const uint32_t c = cb + r;
            if (c < nch) {  // uniform
                float *sx = s_buf + (c & 1) * (TOK * 256);
#pragma unroll
                for (uint32_t t = 0; t < NTT; ++t) sx[(g * NTT + t) * 256 + col] = xv[r][t];
                float wc[2][8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    wc[0][i] = w[r][0][i];
                    wc[1][i] = w[r][1][i];
                }
                if (c + CZ_RT_RING - 1 < nch) load_chunk((r + CZ_RT_RING - 1) % CZ_RT_RING, c + CZ_RT_RING - 1);
                __syncthreads();
                const float *sxg = sx + g * NTT * 256 + j;
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (uint32_t t = 0; t < NTT; ++t) {
                        const float xval = sxg[t * 256 + 32 * i];
                        acc[0][t] = __builtin_fmaf(xval, wc[0][i], acc[0][t]);
                        acc[1][t] = __builtin_fmaf(xval, wc[1][i], acc[1][t]);
                    }
            }
        }
    }
    __syncthreads();  // every thread is done with the input buffers
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (uint32_t t = 0; t < NTT; ++t)
            s_buf[((2 * hw + m) * TOK + g * NTT + t) * CZ_RT_ACC_LD + j] = acc[m][t];
    __syncthreads();
    if (tid >= CZ_RT_EXP * TOK) return;
    // thread (expert el = tid / 16, token t = tid % 16): total_l = ((0 + a_l)
    // + a_{l+8}) + a_{l+16}) + a_{l+24}, sum = -0 + total_0 + ... + total_7
    const uint32_t el = tid / TOK, t = tid % TOK;
    const float4 *row = (const float4 *)(s_buf + (el * TOK + t) * CZ_RT_ACC_LD);
    float a[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 v = row[q];
        a[4 * q] = v.x;
        a[4 * q + 1] = v.y;
        a[4 * q + 2] = v.z;
        a[4 * q + 3] = v.w;
    }
    float sum = -0.0f;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        float total = 0.0f;
        total = total + a[l];
        total = total + a[l + 8];
        total = total + a[l + 16];
        total = total + a[l + 24];
        sum = sum + total;
    }
    const uint32_t e = eg * CZ_RT_EXP + el;
    if (e < E && t < nt) {
        float lg = sum;
        if (L.router_bias) lg = lg + L.router_bias[e];
        A.logits[(uint64_t)(t0 + t) * E + e] = lg;
    }
}

__global__ __launch_bounds__(64) void k_router_generic(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    const uint32_t H = A.L.H, E = A.L.E;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t half = lane >> 5, j = lane & 31, hb = half * 32;
    const uint32_t e = blockIdx.x * 2 + half;
    const uint32_t ec = min(e, E - 1);
    const uint32_t t0 = blockIdx.y * (uint32_t)A.tt;
    const uint32_t nt = min((uint32_t)A.tt, (uint32_t)A.S - t0);
    extern __shared__ float smem[];
    cz_router_stage_x(A, smem, t0, nt);
    __syncthreads();
    const float *wr = A.L.router + (uint64_t)ec * H;
    for (uint32_t t = 0; t < nt; ++t) {
        float lg = cz_router_dot(smem + t * H, wr, H, j, hb);
        if (A.L.router_bias) lg = lg + A.L.router_bias[ec];
        if (j == 0 && e < E) A.logits[(uint64_t)(t0 + t) * E + e] = lg;
    }
}

// ---------------------------------------------------------------------------
// routing of one token by one wave (moe.zig:435-463): mx = max logit; v =
// exp(l - mx) in f32; K passes of a strict '>' scan over the unchosen from
// bv = -1 (ties to the lowest id; none left -> expert 0); top = sum of the picked v in f64 in pick order; den = norm_topk ?
// top : sum_e f64(v_e) in expert order; gate_z = f32(f64(v_z) / den).  Lane l
// holds experts l + 64m for m < M (M = ceil(E/64)); values move between lanes
// by DPP and readlane only.  Lane z < K leaves pick z in registers
// (o_pos = z, o_id, o_gate) and writes s_idx[z] / s_gate[z] (LDS), which the
// block reads after a barrier.  Must be called by a whole wave.
// cz_route_wave_regs takes the logits in the wave's registers (v[m] in lane
// l: expert l + 64m; overwritten), cz_route_wave_m reads them from lg.
// ---------------------------------------------------------------------------
template <int M>
__device__ inline void cz_route_wave_regs(float (&v)[M], uint32_t E, uint32_t K, uint32_t norm_topk,
                                          uint32_t *s_idx, float *s_gate, uint32_t &o_pos, uint32_t &o_id,
                                          float &o_gate) {
    const uint32_t lane = cz_lane();
    // moe.zig:439-440: mx = max over the logits (NaN-ignoring @max)
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < M; ++m)
        if (lane + 64 * m < E) mx = fmaxf(mx, v[m]);
    mx = cz_wave_max_dpp(mx);
    // moe.zig:441-445: v = exp(l - mx) in f32; lanes past E hold NaN, which
    // never wins a strict '>' comparison or an equality test
#pragma unroll
    for (int m = 0; m < M; ++m) v[m] = lane + 64 * m < E ? cz_expf(v[m] - mx) : __builtin_nanf("");
    double all = 0.0;
    if (!norm_topk) {
#pragma unroll
        for (int m = 0; m < M; ++m)
            for (uint32_t l = 0; l < 64; ++l)
                if (64 * m + l < E) all += (double)cz_readlane(v[m], l);
    }
    const float v0 = cz_readlane(v[0], 0);
    // moe.zig:447-460 as two wave maxima per pick: vk = bits(v) + 1 for an
    // unchosen expert with a value (v >= +0 orders like its bits; 0 = chosen,
    // NaN or past E), the largest vk is the largest value; among the experts
    // holding it the largest 0xffffffff - id is the lowest id: the strict '>'
    // scan's winner.  All vk 0: none left -> expert 0.
    uint32_t vk[M];
#pragma unroll
    for (int m = 0; m < M; ++m)
        vk[m] = (lane + 64u * m < E && v[m] == v[m]) ? __builtin_bit_cast(uint32_t, v[m]) + 1u : 0u;
    double top = 0.0;
    float my_v = 0.0f;    // lane z: value of pick z
    uint32_t my_i = 0;    // lane z: id of pick z
    for (uint32_t z = 0; z < K; ++z) {
        uint32_t lk = 0;
#pragma unroll
        for (int m = 0; m < M; ++m) lk = max(lk, vk[m]);
        const uint32_t bvk = cz_wave_max_u32(lk);  // uniform
        uint32_t ik = 0;
#pragma unroll
        for (int m = 0; m < M; ++m) ik = max(ik, (bvk != 0u && vk[m] == bvk) ? 0xffffffffu - (lane + 64u * m) : 0u);
        const uint32_t bik = cz_wave_max_u32(ik);  // uniform
        const bool none = bvk == 0u;
        const uint32_t best = none ? 0u : 0xffffffffu - bik;
        const float vb = none ? v0 : __builtin_bit_cast(float, bvk - 1u);  // v[best]
#pragma unroll
        for (int m = 0; m < M; ++m) vk[m] = lane + 64u * m == best ? 0u : vk[m];  // the winner is chosen
        top += (double)vb;  // moe.zig:459 in pick order
        if (lane == z) {
            my_v = vb;
            my_i = best;
        }
    }
    if (lane < K) {
        const double den = norm_topk ? top : all;  // moe.zig:461-462
        o_pos = lane;
        o_id = my_i;
        o_gate = (float)((double)my_v / den);
        s_idx[lane] = o_id;
        s_gate[lane] = o_gate;
    }
}

template <int M>
__device__ inline void cz_route_wave_m(const float *__restrict__ lg, uint32_t E, uint32_t K, uint32_t norm_topk,
                                       uint32_t *s_idx, float *s_gate, uint32_t &o_pos, uint32_t &o_id,
                                       float &o_gate) {
    float v[M];
#pragma unroll
    for (int m = 0; m < M; ++m) v[m] = lg[min(cz_lane() + 64 * m, E - 1)];  // clamped: in bounds
    cz_route_wave_regs<M>(v, E, K, norm_topk, s_idx, s_gate, o_pos, o_id, o_gate);
}

// expert groups of 64 a routing wave holds for E experts
__host__ __device__ constexpr int cz_route_groups(uint32_t E) {
    return E <= 64 ? 1 : E <= 128 ? 2 : E <= 256 ? 4 : E <= 512 ? 8 : 16;
}

// Work item of a gate/up block: a routed slot or a shared-expert token.
struct UpItem {
    const uint8_t *Wg, *Wu;
    const float *Sg, *Su;
    float *out;
    uint32_t rows, tok, tile;
    bool routed;
};

// Resolves block `blk` of a gate/up grid (rows_wg rows per block): routed
// blocks [0, S*K*tiles_r) route their token (wave 0) and publish the token's routing from the slot-0 tile-0
// block; shared-expert blocks follow, and their tile-0 block computes the
// token's sigmoid gate.  With xs_lds, the token's row of the router input is
// staged in LDS: every thread requests its NXR float4 of it before the
// routing and stores them after it (H/4 <= 256*NXR).
template <int M, int NXR>
__device__ inline UpItem cz_up_item(const StepArgs &A, uint32_t rows_wg, const float *xn, float4 *xs_lds = nullptr) {
    const LayerDev &L = A.L;
    __shared__ uint32_t s_idx[CZ_MAX_K];
    __shared__ float s_gate[CZ_MAX_K];
    const uint32_t wave = threadIdx.x >> 6, lane = cz_lane();
    const uint32_t tiles_r = (L.I + rows_wg - 1) / rows_wg;
    const uint32_t nslots = (uint32_t)A.S * L.K;
    uint32_t blk = blockIdx.x;
    UpItem it;
    const uint32_t n4 = L.H / 4;
    float4 xr[NXR > 0 ? NXR : 1];
#define CZ_UP_LOAD_X(tok_)                                                       \
    if (NXR > 0 && xs_lds) {                                                     \
        const float4 *src_ = (const float4 *)(xn + (uint64_t)(tok_) * L.H);      \
        _Pragma("unroll") for (int q = 0; q < NXR; ++q) {                        \
            const uint32_t i_ = threadIdx.x + 256u * q;                          \
            xr[q] = i_ < n4 ? src_[i_] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);    \
        }                                                                        \
    }
#define CZ_UP_STORE_X()                                                          \
    if (NXR > 0 && xs_lds) {                                                     \
        _Pragma("unroll") for (int q = 0; q < NXR; ++q) {                        \
            const uint32_t i_ = threadIdx.x + 256u * q;                          \
            if (i_ < n4) xs_lds[i_] = xr[q];                                     \
        }                                                                        \
    }
    if (blk < nslots * tiles_r) {
        const uint32_t slot = blk / tiles_r;
        it.tile = blk - slot * tiles_r;
        it.tok = slot / L.K;
        const uint32_t z = slot - it.tok * L.K;
        CZ_UP_LOAD_X(it.tok)
        const float *lg = A.logits + (uint64_t)it.tok * L.E;
        if (wave == 0) {
            uint32_t o_pos = 0, o_id = 0;
            float o_gate = 0.0f;
            cz_route_wave_m<M>(lg, L.E, L.K, L.norm_topk, s_idx, s_gate, o_pos, o_id, o_gate);
        }
        CZ_UP_STORE_X()
        __syncthreads();
        if (A.stop && L.slot_map) {  // block-uniform: a pick without a pool slot stops the token's run
            bool miss = false;
            for (uint32_t k = 0; k < L.K; ++k) miss = miss || L.slot_map[s_idx[k]] < 0;
            if (miss) {
                if (threadIdx.x == 0) atomicCAS(A.stop, 0u, A.stop_code);
                it.rows = 0;  // the caller's rows test ends the block
                it.tok = 0;
                it.tile = 0;
                return it;
            }
        }
        if (z == 0 && it.tile == 0 && wave == 0) {
            for (uint32_t k = lane; k < L.K; k += 64) {
                const uint64_t o = (uint64_t)it.tok * L.K + k;
                cz_bump_usage(L.usage, L.E, s_idx[k]);
                A.idx[o] = s_idx[k];
                A.gates[o] = s_gate[k];
                if (A.idx_trace) A.idx_trace[o] = s_idx[k];
                if (A.gates_trace) A.gates_trace[o] = s_gate[k];
            }
        }
        const uint32_t e = s_idx[z];
        const uint64_t sl = cz_slot(L, e);
        const uint8_t *base = L.ew + sl * L.ew_stride;
        it.Wg = base;
        it.Wu = base + (uint64_t)L.I * L.H;
        const float *sb = L.es + sl * L.es_stride;
        it.Sg = sb;
        it.Su = sb + (uint64_t)L.nbI * L.nbH;
        it.out = A.h + (uint64_t)slot * L.I;
        it.rows = L.I;
        it.routed = true;
    } else {
        blk -= nslots * tiles_r;
        const uint32_t tiles_s = (L.SI + rows_wg - 1) / rows_wg;
        it.tok = blk / tiles_s;
        it.tile = blk - it.tok * tiles_s;
        it.Wg = L.sw;
        it.Wu = L.sw + (uint64_t)L.SI * L.H;
        it.Sg = L.ss;
        it.Su = L.ss + (uint64_t)L.nbSI * L.nbH;
        it.out = A.hs + (uint64_t)it.tok * L.SI;
        it.rows = L.SI;
        it.routed = false;
        CZ_UP_LOAD_X(it.tok)
        // shared-expert gate sigmoid(x . sh_gate) (moe.zig:475-477)
        if (it.tile == 0 && wave == 0) {
            const float d = cz_sgate_dot(xn + (uint64_t)it.tok * L.H, L.sh_gate, L.H, lane);
            if (lane == 0) A.sgate[it.tok] = cz_sigmoid(d);
        }
        CZ_UP_STORE_X()
        __syncthreads();
    }
#undef CZ_UP_LOAD_X
#undef CZ_UP_STORE_X
    return it;
}

// ---------------------------------------------------------------------------
// fast-path helpers: NB bytes per lane per row
// ---------------------------------------------------------------------------
template <int NB>
__device__ inline void cz_load_row(const uint8_t *__restrict__ p, uint32_t (&d)[NB / 4]) {
    static_assert(NB % 4 == 0 && NB >= 4 && NB <= 64, "NB");
    if constexpr (NB % 16 == 0) {
#pragma unroll
        for (int q = 0; q < NB / 16; ++q) {
            const uint4 v = ((const uint4 *)p)[q];
            d[4 * q + 0] = v.x; d[4 * q + 1] = v.y; d[4 * q + 2] = v.z; d[4 * q + 3] = v.w;
        }
    } else if constexpr (NB == 8) {
        const uint2 v = *(const uint2 *)p;
        d[0] = v.x; d[1] = v.y;
    } else if constexpr (NB == 12) {
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 v = *(const u32x3 *)p;
        d[0] = v.x; d[1] = v.y; d[2] = v.z;
    } else {
#pragma unroll
        for (int q = 0; q < NB / 4; ++q) d[q] = ((const uint32_t *)p)[q];
    }
}

template <int NB>
__device__ inline void cz_load_x(const float *__restrict__ p, float (&x)[NB]) {
    static_assert(NB % 4 == 0, "NB");
#pragma unroll
    for (int q = 0; q < NB / 4; ++q) {
        const float4 v = ((const float4 *)p)[q];
        x[4 * q + 0] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
    }
}

// x[0..3] . e4m3(bytes of w), element order = byte order
__device__ inline float cz_dot4_raw(uint32_t w, const float *x4, float acc) {
    const cz_float2 lo = cz_fp8x2_lo(w);
    const cz_float2 hi = cz_fp8x2_hi(w);
    acc = __builtin_fmaf(x4[0], lo.x, acc);
    acc = __builtin_fmaf(x4[1], lo.y, acc);
    acc = __builtin_fmaf(x4[2], hi.x, acc);
    acc = __builtin_fmaf(x4[3], hi.y, acc);
    return acc;
}

// Scales a lane needs for its NB columns [col0, col0+NB) of one row: one per
// dword, read from the row's scale row before any weight is consumed.
template <int NB>
struct RowScales {
    static constexpr int N = (CZ_BLOCK % NB) == 0 ? 1 : NB / 4;
    float s[N];
};

template <int NB>
__device__ inline void cz_load_scales(const float *__restrict__ srow, uint32_t col0, RowScales<NB> &rs) {
    if constexpr (RowScales<NB>::N == 1) {
        rs.s[0] = srow[col0 / CZ_BLOCK];  // all of the lane's columns share one block
    } else {
#pragma unroll
        for (int q = 0; q < NB / 4; ++q) rs.s[q] = srow[(col0 + 4 * q) / CZ_BLOCK];
    }
}

// sum over the lane's NB columns of x * e4m3(w) * scale: the E4M3 products
// are summed per 128-column block and the block's scale is applied once to
// that partial sum.
template <int NB>
__device__ inline float cz_row_dot(const uint32_t (&d)[NB / 4], const float (&x)[NB], const RowScales<NB> &rs) {
    if constexpr (RowScales<NB>::N == 1) {
        float p = 0.0f;
#pragma unroll
        for (int q = 0; q < NB / 4; ++q) p = cz_dot4_raw(d[q], &x[4 * q], p);
        return p * rs.s[0];
    } else {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < NB / 4; ++q) {
            const float p = cz_dot4_raw(d[q], &x[4 * q], 0.0f);
            acc = __builtin_fmaf(p, rs.s[q], acc);
        }
        return acc;
    }
}

// ---------------------------------------------------------------------------
// Keyed FP8 GEMV on device-resident activations (attention projections and
// any other Fp8Matrix at decode, fp8.zig:182): y[S][O] = x[S][I] . (e4m3(W) *
// scale)^T for W [O][I] resident in HBM.  One wave per output row; lane l owns
// the row bytes [NB l, NB l + NB) (I = 64 NB, 128-bit loads); a wave takes RW
// consecutive rows, whose weights and scales are requested before the
// tokens' rows are staged in LDS, ST tokens at a time, then reused for every
// token.  Rows past O are read as row O - 1 and not stored (every wave
// reaches every barrier).
// ---------------------------------------------------------------------------
template <int NB, int ST, int RW>
__device__ __attribute__((always_inline)) inline void cz_gemv_fp8_block(
    float *__restrict__ y, const float *__restrict__ x, const uint8_t *__restrict__ w,
    const float *__restrict__ scales, uint32_t S, uint32_t O, uint32_t blk, float4 *xs) {
    constexpr uint32_t I = 64 * NB, I4 = I / 4, NQ = (ST * I4 + 255) / 256;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t r0 = (blk * 4 + wave) * RW;  // the wave's RW rows
    const uint32_t col0 = lane * NB;
    uint32_t d[RW][NB / 4];
    RowScales<NB> rs[RW];
#pragma unroll
    for (int q = 0; q < RW; ++q) {
        const uint32_t row = min(r0 + q, O - 1);
        cz_load_row<NB>(w + (uint64_t)row * I + col0, d[q]);
        cz_load_scales<NB>(scales + (uint64_t)(row / CZ_BLOCK) * ((I + CZ_BLOCK - 1) / CZ_BLOCK), col0, rs[q]);
    }
    for (uint32_t t0 = 0; t0 < S; t0 += ST) {
        const uint32_t n4 = min((uint32_t)ST, S - t0) * I4;
        const float4 *src = reinterpret_cast<const float4 *>(x + (uint64_t)t0 * I);
        float4 v[NQ];
#pragma unroll
        for (uint32_t k = 0; k < NQ; ++k) v[k] = src[min(tid + 256 * k, n4 - 1)];  // clamped: in bounds
#pragma unroll
        for (uint32_t k = 0; k < NQ; ++k)
            if (tid + 256 * k < n4) xs[tid + 256 * k] = v[k];
        __syncthreads();
        for (uint32_t t = 0; t < n4 / I4; ++t) {
            float xv[NB];
            cz_load_x<NB>(reinterpret_cast<const float *>(xs) + t * I + col0, xv);
#pragma unroll
            for (int q = 0; q < RW; ++q) {
                const float acc = cz_wave_sum_dpp(cz_row_dot<NB>(d[q], xv, rs[q]));
                if (lane == 0 && r0 + q < O) y[(uint64_t)(t0 + t) * O + r0 + q] = acc;
            }
        }
        __syncthreads();  // these tokens' readers are done before the next pass stores
    }
}

template <int NB, int ST, int RW>
__global__ __launch_bounds__(256) void k_gemv_fp8(float *__restrict__ y, const float *__restrict__ x,
                                                  const uint8_t *__restrict__ w, const float *__restrict__ scales,
                                                  uint32_t S, uint32_t O) {
    __shared__ float4 xs[ST * 16 * NB];
    cz_gemv_fp8_block<NB, ST, RW>(y, x, w, scales, S, O, blockIdx.x, xs);
}

// Several keyed matrices of one row width on the same input rows in one
// launch (the q, k and v projections of a layer): matrix m takes the
// workgroups [blk0[m], blk0[m + 1]); each workgroup runs the single-matrix
// GEMV's body on its matrix, so every output is bit-identical to a
// k_gemv_fp8 launch of that matrix alone.
#define CZ_GEMV_MULTI 4
struct GemvMulti {
    float *y[CZ_GEMV_MULTI];
    const uint8_t *w[CZ_GEMV_MULTI];
    const float *s[CZ_GEMV_MULTI];
    uint32_t O[CZ_GEMV_MULTI];
    uint32_t blk0[CZ_GEMV_MULTI + 1];
    uint32_t n;
};

template <int NB, int ST, int RW>
__global__ __launch_bounds__(256) void k_gemv_fp8_multi(GemvMulti G, const float *__restrict__ x, uint32_t S) {
    __shared__ float4 xs[ST * 16 * NB];
    uint32_t m = 0;
#pragma unroll
    for (uint32_t k = 1; k < CZ_GEMV_MULTI; ++k)
        if (k < G.n && blockIdx.x >= G.blk0[k]) m = k;
    cz_gemv_fp8_block<NB, ST, RW>(G.y[m], x, G.w[m], G.s[m], S, G.O[m], blockIdx.x - G.blk0[m], xs);
}

// ---------------------------------------------------------------------------
// NativeMatrix GEMV on device-resident activations (tensors.zig:114-119: f32
// rows through dotF32, matmul.zig:60-82; BF16 rows through dotBf16,
// matmul.zig:84-110, which is dotF32's order on the widened weights): y[S][O]
// with every dot in that order: half-wave per row as the router kernel (lane
// j = chain j over elements j + 32i, then cz_router_combine), so results are
// bit-identical to the reference's.  WPB waves per workgroup (2 WPB rows)
// share the token rows staged in LDS, ST at a time; I = 32 NS.  Rows past O
// are read as row O - 1 and not stored (every wave reaches every barrier).
// ---------------------------------------------------------------------------
__device__ inline float cz_widen(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ inline float cz_widen(float f) { return f; }

template <int NS, int WPB, typename T>
__global__ __launch_bounds__(64 * WPB) void k_gemv_native(float *__restrict__ y, const float *__restrict__ x,
                                                          const T *__restrict__ w, uint32_t S, uint32_t O) {
    constexpr uint32_t I = 32 * NS, I4 = I / 4, NT = 64 * WPB;
    constexpr uint32_t ST = I >= 8192 ? 1 : 8192 / I < 4 ? 8192 / I : 4;  // tokens per pass: <= 32 KiB of LDS
    constexpr uint32_t NQ = (ST * I4 + NT - 1) / NT;
    __shared__ float4 xs[ST * I4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t half = lane >> 5, j = lane & 31, hb = half * 32;
    const uint32_t r = blockIdx.x * 2 * WPB + 2 * wave + half;
    const uint32_t row = min(r, O - 1);
    float wv[NS];
    const T *wr = w + (uint64_t)row * I + j;
#pragma unroll
    for (int i = 0; i < NS; ++i) wv[i] = cz_widen(wr[32 * i]);
    constexpr int CB = NS < 32 ? NS : 32;
    for (uint32_t t0 = 0; t0 < S; t0 += ST) {
        const uint32_t n4 = min(ST, S - t0) * I4;
        const float4 *src = reinterpret_cast<const float4 *>(x + (uint64_t)t0 * I);
        float4 v[NQ];
#pragma unroll
        for (uint32_t k = 0; k < NQ; ++k) v[k] = src[min(tid + NT * k, n4 - 1)];  // clamped: in bounds
#pragma unroll
        for (uint32_t k = 0; k < NQ; ++k)
            if (tid + NT * k < n4) xs[tid + NT * k] = v[k];
        __syncthreads();
        for (uint32_t t = 0; t < n4 / I4; ++t) {
            const float *xr = reinterpret_cast<const float *>(xs) + t * I + j;
            float acc = 0.0f;
#pragma unroll
            for (int i0 = 0; i0 < NS; i0 += CB) {
                float xb[CB];
#pragma unroll
                for (int q = 0; q < CB; ++q) xb[q] = xr[32 * (i0 + q)];
#pragma unroll
                for (int q = 0; q < CB; ++q) acc = __builtin_fmaf(xb[q], wv[i0 + q], acc);
            }
            const float lg = cz_router_combine(acc, j, hb);
            if (j == 0 && r < O) y[(uint64_t)(t0 + t) * O + r] = lg;
        }
        __syncthreads();  // these tokens' readers are done before the next pass stores
    }
}

// Any row width: the same dot order (dotF32's tails: 8-wide steps on lanes
// j < 8, then a scalar FMA tail), the weights read per token.  One wave per
// two rows.
template <typename T>
__global__ __launch_bounds__(64) void k_gemv_native_any(float *__restrict__ y, const float *__restrict__ x,
                                                        const T *__restrict__ w, uint32_t S, uint32_t I, uint32_t O) {
    const uint32_t lane = threadIdx.x & 63, half = lane >> 5, j = lane & 31, hb = half * 32;
    const uint32_t r = blockIdx.x * 2 + half, row = min(r, O - 1);
    const T *wr = w + (uint64_t)row * I;
    for (uint32_t t = 0; t < S; ++t) {
        const float *a = x + (uint64_t)t * I;
        float acc = 0.0f;
        uint32_t i = 0;
        for (; i + 32 <= I; i += 32) acc = __builtin_fmaf(a[i + j], cz_widen(wr[i + j]), acc);
        for (; i + 8 <= I; i += 8)
            if (j < 8) acc = __builtin_fmaf(a[i + j], cz_widen(wr[i + j]), acc);
        float sum = cz_router_combine(acc, j, hb);
        for (; i < I; ++i) sum = __builtin_fmaf(a[i], cz_widen(wr[i]), sum);
        if (j == 0 && r < O) y[(uint64_t)t * O + r] = sum;
    }
}

// logits[t][e] += bias[e] (the router kernels' one f32 add after the dot)
__global__ void k_add_bias(float *__restrict__ logits, const float *__restrict__ bias, uint32_t S, uint32_t E) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (uint64_t)S * E) logits[i] = logits[i] + bias[i % E];
}

// A NativeMatrix shared expert (moe.zig:467-479): h = silu(g) * u in place
// of g, f32 (activation.zig:18-20 with the correctly rounded exp).
__global__ void k_swiglu_native(float *__restrict__ g, const float *__restrict__ u, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) g[i] = cz_silu(g[i]) * u[i];
}

// sgate_t = sigmoid(sum_d xn_t[d] * sh_gate[d]) (serial order, moe.zig:475-477),
// one wave per token.
__global__ __launch_bounds__(64) void k_shared_gate_native(float *__restrict__ sgate, const float *__restrict__ xn,
                                                           const float *__restrict__ sh_gate, uint32_t H) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63;
    const float d = cz_sgate_dot(xn + (uint64_t)t * H, sh_gate, H, lane);
    if (lane == 0) sgate[t] = cz_sigmoid(d);
}

// out[t][i] += sgate_t * shared[t][i] (moe.zig:478)
__global__ void k_shared_add_native(float *__restrict__ out, const float *__restrict__ shared,
                                    const float *__restrict__ sgate, uint32_t S, uint32_t H) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (uint64_t)S * H) {
        const float prod = sgate[i / H] * shared[i];
        out[i] = out[i] + prod;
    }
}

// ---------------------------------------------------------------------------
// gate/up + SiLU, fast path: row width H = 64*NB, RW rows per wave; weights,
// scales and the input slice are all requested before any is consumed.
// ---------------------------------------------------------------------------
template <int NB, int RW>
__device__ inline void cz_up_rows(const StepArgs &A, const UpItem &it, const float *xs_lds, uint32_t r0, uint32_t lane) {
    constexpr int ND = NB / 4;
    const LayerDev &L = A.L;
    const uint32_t col0 = lane * NB;
    uint32_t dg[RW][ND], du[RW][ND];
    RowScales<NB> sg[RW], su[RW];
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        const uint32_t rc = min(r0 + rr, it.rows - 1);
        cz_load_row<NB>(it.Wg + (uint64_t)rc * L.H + col0, dg[rr]);
        cz_load_row<NB>(it.Wu + (uint64_t)rc * L.H + col0, du[rr]);
        cz_load_scales<NB>(it.Sg + (uint64_t)(rc / CZ_BLOCK) * L.nbH, col0, sg[rr]);
        cz_load_scales<NB>(it.Su + (uint64_t)(rc / CZ_BLOCK) * L.nbH, col0, su[rr]);
    }
    __builtin_amdgcn_sched_barrier(0);  // every weight and scale load is in flight
    float xv[NB];
    cz_load_x<NB>(xs_lds + col0, xv);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
        const uint32_t r = r0 + rr;
        float ag = cz_row_dot<NB>(dg[rr], xv, sg[rr]);
        float au = cz_row_dot<NB>(du[rr], xv, su[rr]);
        ag = cz_wave_sum_dpp(ag);
        au = cz_wave_sum_dpp(au);
        if (lane == (uint32_t)rr && r < it.rows) it.out[r] = cz_silu_fast(ag) * au;
    }
}

template <int NB, int RW, int M>
__global__ __launch_bounds__(256) void k_up_fast(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    __shared__ float4 xs[NB * 16];  // the token's router input, H = 64*NB floats
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *xn = A.rms ? A.xn : A.x;
    const UpItem it = cz_up_item<M, (NB * 16 + 255) / 256>(A, 4 * RW, xn, xs);
    const uint32_t r0 = it.tile * 4 * RW + wave * RW;
    if (r0 >= it.rows) return;
    cz_up_rows<NB, RW>(A, it, (const float *)xs, r0, lane);
}

// ---------------------------------------------------------------------------
// down + weighted combine (+ shared expert, + residual), fast path: one wave
// per output row.  Lane l owns the column groups 4l + 256j (j < NJ), so every
// load instruction of a row, its h slice and its scales covers whole
// contiguous lines; group j of lane l lies in scale block 2j + l/32.  The h
// slices of the first KC experts are requested before the token's routing is
// read (they do not depend on it); the routing is read as wave-uniform values,
// so the weight addresses are scalar.  I = 256*NJ, SI = 256*NJS (NJS 0 =
// no shared expert).
// ---------------------------------------------------------------------------
template <int NJ>
__device__ inline void cz_load_h_groups(const float *__restrict__ hrow, uint32_t lane, float (&hv)[NJ][4]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const float4 v = *(const float4 *)(hrow + 4 * lane + 256 * j);
        hv[j][0] = v.x; hv[j][1] = v.y; hv[j][2] = v.z; hv[j][3] = v.w;
    }
}

template <int NJ>
__device__ inline void cz_load_w_groups(const uint8_t *__restrict__ wrow, const float *__restrict__ srow, uint32_t lane,
                                        uint32_t (&d)[NJ], float (&sc)[NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        d[j] = *(const uint32_t *)(wrow + 4 * lane + 256 * j);
        sc[j] = srow[2 * j + (lane >> 5)];
    }
}

// sum over the lane's groups of (e4m3 . h) * block scale
template <int NJ>
__device__ inline float cz_groups_dot(const uint32_t (&d)[NJ], const float (&hv)[NJ][4], const float (&sc)[NJ]) {
    float p = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) p = __builtin_fmaf(cz_dot4_raw(d[j], hv[j], 0.0f), sc[j], p);
    return p;
}

__device__ inline uint32_t cz_uniform_u32(const uint32_t *p) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)*p); }
// a wave-uniform read of memory no kernel in flight writes: through the
// constant address space, i.e. a scalar load (lgkmcnt, not vmcnt)
__device__ inline float cz_const_f32(const float *p) {
    return *(const __attribute__((address_space(4))) float *)p;
}
__device__ inline float cz_uniform_f32(const float *p) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, *p)));
}

template <int NJ, int NJS, int KC>
__device__ inline void cz_down_row(const StepArgs &A, uint32_t tok, uint32_t r, uint32_t lane) {
    const LayerDev &L = A.L;
    const uint64_t slot0 = (uint64_t)tok * L.K;
    float hv[KC][NJ][4];
#pragma unroll
    for (int c = 0; c < KC; ++c)
        cz_load_h_groups<NJ>(A.h + (slot0 + min((uint32_t)c, L.K - 1)) * L.I, lane, hv[c]);
    float acc = 0.0f;
    for (uint32_t z0 = 0; z0 < L.K; z0 += KC) {
        if (z0 > 0) {
#pragma unroll
            for (int c = 0; c < KC; ++c)
                cz_load_h_groups<NJ>(A.h + (slot0 + min(z0 + c, L.K - 1)) * L.I, lane, hv[c]);
        }
        uint32_t dd[KC][NJ];
        float sc[KC][NJ];
        float gz[KC];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const uint32_t z = min(z0 + c, L.K - 1);
            const uint32_t e = min(cz_uniform_u32(A.idx + slot0 + z), L.E - 1);
            gz[c] = cz_uniform_f32(A.gates + slot0 + z);
            const uint64_t sl = cz_slot(L, e);
            cz_load_w_groups<NJ>(L.ew + sl * L.ew_stride + 2ull * L.I * L.H + (uint64_t)r * L.I,
                                 L.es + sl * L.es_stride + 2ull * L.nbI * L.nbH + (uint64_t)(r / CZ_BLOCK) * L.nbI, lane,
                                 dd[c], sc[c]);
        }
        __builtin_amdgcn_sched_barrier(0);  // the chunk's loads are all in flight
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const float p = cz_groups_dot<NJ>(dd[c], hv[c], sc[c]);
            if (z0 + c < L.K) acc = __builtin_fmaf(gz[c], p, acc);
        }
    }
    if constexpr (NJS > 0) {
        float hs[NJS][4];
        uint32_t ds[NJS];
        float ss[NJS];
        cz_load_h_groups<NJS>(A.hs + (uint64_t)tok * L.SI, lane, hs);
        cz_load_w_groups<NJS>(L.sw + 2ull * L.SI * L.H + (uint64_t)r * L.SI,
                              L.ss + 2ull * L.nbSI * L.nbH + (uint64_t)(r / CZ_BLOCK) * L.nbSI, lane, ds, ss);
        const float sgv = cz_uniform_f32(A.sgate + tok);
        __builtin_amdgcn_sched_barrier(0);
        acc = __builtin_fmaf(sgv, cz_groups_dot<NJS>(ds, hs, ss), acc);
    }
    const float tot = cz_wave_sum_dpp(acc);
    if (lane == 0) {
        const uint64_t o = (uint64_t)tok * L.H + r;
        A.out[o] = (A.xres ? A.xres[o] : 0.0f) + tot;
    }
}

template <int NJ, int NJS, int KC>
__global__ __launch_bounds__(256) void k_down_fast(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    const LayerDev &L = A.L;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tiles_h = (L.H + 3) / 4;
    const uint32_t tok = blockIdx.x / tiles_h, tile = blockIdx.x - tok * tiles_h;
    const uint32_t r = tile * 4 + wave;
    if (r >= L.H || tok >= (uint32_t)A.S) return;
    cz_down_row<NJ, NJS, KC>(A, tok, r, lane);
}

// Down + weighted combine (+ shared expert, + residual), RR output rows per
// wave: the token's h slices are read into registers once and serve all RR
// rows, so each row costs only its weight and scale loads.  Lane l owns the
// routed columns [BPL l, BPL l + BPL) of every expert (I = 64 BPL: one 4, 8,
// 12 or 16-byte load per expert row) and the shared columns 16l + 1024q (q <
// NQ = SI/1024: one 16-byte load each).  A dword's columns lie in one
// 128-column scale block; with BPL = 12 a lane's dwords can span two blocks.
// KM = top-k (experts in pick order).
template <int BPL, int NQ, int KM, int RR>
__global__ __launch_bounds__(256) void k_down_rows(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    constexpr int ND = BPL / 4;
    static_assert(BPL == 4 || BPL == 8 || BPL == 12 || BPL == 16, "bytes per lane");
    const LayerDev &L = A.L;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tiles = (L.H + 4 * RR - 1) / (4 * RR);
    const uint32_t tok = blockIdx.x / tiles, tile = blockIdx.x - tok * tiles;
    const uint32_t r0 = (tile * 4 + wave) * RR;
    if (r0 >= L.H || tok >= (uint32_t)A.S) return;  // wave-uniform
    const uint64_t slot0 = (uint64_t)tok * KM;
    // the token's h slices (they do not depend on the routing): requested first
    float hv[KM][BPL];
#pragma unroll
    for (int z = 0; z < KM; ++z) {
        const float4 *hp = reinterpret_cast<const float4 *>(A.h + (slot0 + z) * L.I + BPL * lane);
#pragma unroll
        for (int d = 0; d < ND; ++d) {
            const float4 v = hp[d];
            hv[z][4 * d] = v.x; hv[z][4 * d + 1] = v.y; hv[z][4 * d + 2] = v.z; hv[z][4 * d + 3] = v.w;
        }
    }
    float hs[NQ > 0 ? NQ : 1][16];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const float4 *hp = reinterpret_cast<const float4 *>(A.hs + (uint64_t)tok * L.SI + 16 * lane + 1024 * q);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const float4 v = hp[d];
            hs[q][4 * d] = v.x; hs[q][4 * d + 1] = v.y; hs[q][4 * d + 2] = v.z; hs[q][4 * d + 3] = v.w;
        }
    }
    // the routing, wave-uniform: slots, gates
    uint64_t sl[KM];
    float gz[KM];
#pragma unroll
    for (int z = 0; z < KM; ++z) {
        const uint32_t e = min(cz_uniform_u32(A.idx + slot0 + z), L.E - 1);
        gz[z] = cz_uniform_f32(A.gates + slot0 + z);
        sl[z] = cz_slot(L, e);
    }
    const float sgv = NQ > 0 ? cz_uniform_f32(A.sgate + tok) : 0.0f;
    const uint32_t c0 = BPL * lane, b0 = c0 / CZ_BLOCK, b1 = min((c0 + BPL - 1) / CZ_BLOCK, L.nbI - 1);
    // every row's weights and scales in flight before any is consumed
    uint32_t wd[RR][KM][ND];
    float s0[RR][KM], s1[RR][KM];
    uint4 ws[RR][NQ > 0 ? NQ : 1];
    float ssc[RR][NQ > 0 ? NQ : 1];
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
        const uint32_t r = min(r0 + rr, L.H - 1);
#pragma unroll
        for (int z = 0; z < KM; ++z) {
            const uint8_t *wrow = L.ew + sl[z] * L.ew_stride + 2ull * L.I * L.H + (uint64_t)r * L.I + c0;
            const float *srow = L.es + sl[z] * L.es_stride + 2ull * L.nbI * L.nbH + (uint64_t)(r / CZ_BLOCK) * L.nbI;
            if constexpr (ND == 1) {
                wd[rr][z][0] = *reinterpret_cast<const uint32_t *>(wrow);
            } else if constexpr (ND == 2) {
                const uint2 v = *reinterpret_cast<const uint2 *>(wrow);
                wd[rr][z][0] = v.x; wd[rr][z][1] = v.y;
            } else if constexpr (ND == 3) {
                const uint3 v = *reinterpret_cast<const uint3 *>(wrow);
                wd[rr][z][0] = v.x; wd[rr][z][1] = v.y; wd[rr][z][2] = v.z;
            } else {
                const uint4 v = *reinterpret_cast<const uint4 *>(wrow);
                wd[rr][z][0] = v.x; wd[rr][z][1] = v.y; wd[rr][z][2] = v.z; wd[rr][z][3] = v.w;
            }
            s0[rr][z] = srow[b0];
            s1[rr][z] = BPL == 12 ? srow[b1] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            ws[rr][q] = *reinterpret_cast<const uint4 *>(L.sw + 2ull * L.SI * L.H + (uint64_t)r * L.SI + 16 * lane + 1024 * q);
            ssc[rr][q] = L.ss[2ull * L.nbSI * L.nbH + (uint64_t)(r / CZ_BLOCK) * L.nbSI + lane / 8 + 8 * q];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) {
        float acc = 0.0f;
#pragma unroll
        for (int z = 0; z < KM; ++z) {
            float p = 0.0f;
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                const float sc = (BPL == 12 && (c0 + 4 * d) / CZ_BLOCK != b0) ? s1[rr][z] : s0[rr][z];
                p = __builtin_fmaf(cz_dot4_raw(wd[rr][z][d], &hv[z][4 * d], 0.0f), sc, p);
            }
            acc = __builtin_fmaf(gz[z], p, acc);
        }
        if constexpr (NQ > 0) {
            float ps = 0.0f;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                float p = cz_dot4_raw(ws[rr][q].x, &hs[q][0], 0.0f);
                p = cz_dot4_raw(ws[rr][q].y, &hs[q][4], p);
                p = cz_dot4_raw(ws[rr][q].z, &hs[q][8], p);
                p = cz_dot4_raw(ws[rr][q].w, &hs[q][12], p);
                ps = __builtin_fmaf(p, ssc[rr][q], ps);
            }
            acc = __builtin_fmaf(sgv, ps, acc);
        }
        const float tot = cz_wave_sum_dpp(acc);
        const uint32_t r = r0 + rr;
        if (lane == 0 && r < L.H) {
            const uint64_t o = (uint64_t)tok * L.H + r;
            A.out[o] = (A.xres ? A.xres[o] : 0.0f) + tot;
        }
    }
}

// ---------------------------------------------------------------------------
// generic (any H, I, SI) forms of the two expert kernels: one wave per row,
// lanes stride single columns.  Used for shapes the fast paths do not cover.
// ---------------------------------------------------------------------------
__device__ inline float cz_dot_fp8_strided(const uint8_t *__restrict__ w, const float *__restrict__ srow,
                                           const float *__restrict__ x, uint32_t n, uint32_t lane) {
    float acc = 0.0f;
    for (uint32_t i = lane; i < n; i += 64) {
        const float v = __builtin_amdgcn_cvt_f32_fp8((int)w[i], 0) * srow[i / CZ_BLOCK];
        acc = __builtin_fmaf(x[i], v, acc);
    }
    return acc;
}

template <int M>
__global__ __launch_bounds__(256) void k_up_generic(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    const LayerDev &L = A.L;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *xn = A.rms ? A.xn : A.x;
    const UpItem it = cz_up_item<M, 0>(A, 4, xn);
    const uint32_t r = it.tile * 4 + wave;
    if (r >= it.rows) return;
    const float *xs = xn + (uint64_t)it.tok * L.H;
    float ag = cz_dot_fp8_strided(it.Wg + (uint64_t)r * L.H, it.Sg + (uint64_t)(r / CZ_BLOCK) * L.nbH, xs, L.H, lane);
    float au = cz_dot_fp8_strided(it.Wu + (uint64_t)r * L.H, it.Su + (uint64_t)(r / CZ_BLOCK) * L.nbH, xs, L.H, lane);
    ag = cz_wave_sum_dpp(ag);
    au = cz_wave_sum_dpp(au);
    if (lane == 0) it.out[r] = cz_silu_fast(ag) * au;
}

__global__ __launch_bounds__(256) void k_down_generic(StepArgs A) {
    if (cz_stopped(A)) return;  // block-uniform
    const LayerDev &L = A.L;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tiles_h = (L.H + 3) / 4;
    const uint32_t tok = blockIdx.x / tiles_h, tile = blockIdx.x - tok * tiles_h;
    const uint32_t r = tile * 4 + wave;
    if (r >= L.H || tok >= (uint32_t)A.S) return;
    float acc = 0.0f;
    for (uint32_t z = 0; z < L.K; ++z) {
        const uint32_t slot = tok * L.K + z;
        const uint32_t e = A.idx[slot];
        const uint64_t sl = cz_slot(L, e);
        const uint8_t *Wd = L.ew + sl * L.ew_stride + 2ull * L.I * L.H;
        const float *Sd = L.es + sl * L.es_stride + 2ull * L.nbI * L.nbH;
        const float p = cz_dot_fp8_strided(Wd + (uint64_t)r * L.I, Sd + (uint64_t)(r / CZ_BLOCK) * L.nbI,
                                           A.h + (uint64_t)slot * L.I, L.I, lane);
        acc = __builtin_fmaf(A.gates[slot], p, acc);
    }
    if (L.SI != 0) {
        const uint8_t *Wd = L.sw + 2ull * L.SI * L.H;
        const float *Sd = L.ss + 2ull * L.nbSI * L.nbH;
        const float p = cz_dot_fp8_strided(Wd + (uint64_t)r * L.SI, Sd + (uint64_t)(r / CZ_BLOCK) * L.nbSI,
                                           A.hs + (uint64_t)tok * L.SI, L.SI, lane);
        acc = __builtin_fmaf(A.sgate[tok], p, acc);
    }
    acc = cz_wave_sum_dpp(acc);
    if (lane == 0) {
        const uint64_t o = (uint64_t)tok * L.H + r;
        A.out[o] = (A.xres ? A.xres[o] : 0.0f) + acc;
    }
}

// ---------------------------------------------------------------------------
// synthetic weights (workload generator)
// ---------------------------------------------------------------------------
__device__ inline uint64_t cz_mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// standard normal from a 64-bit counter (Box-Muller on two 24-bit uniforms)
__device__ inline float cz_normal(uint64_t seed, uint64_t ctr) {
    const uint64_t r = cz_mix64(seed ^ cz_mix64(ctr));
    const float u1 = ((float)(uint32_t)(r >> 40) + 0.5f) * 0x1p-24f;
    const float u2 = (float)(uint32_t)((r >> 16) & 0xffffffu) * 0x1p-24f;
    return sqrtf(-2.0f * __logf(u1)) * __cosf(6.28318530718f * u2);
}

// f32 normals: out[i] = std * N(0,1)
__global__ void k_synth_f32(float *out, uint64_t n, uint64_t seed, float stdv) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = stdv * cz_normal(seed, i);
}
