// cz_fused.h - batch-1 decode of a chain of MoE layers with one launch per
// layer (forwardDense, moe.zig:481-539, inside qwen3moe/model.zig:228-232's
// x <- x + moe(rms(x))).
//
// The grid is 256 workgroups, one per CU.  The dispatcher hands workgroups
// to the 8 XCDs round robin, starting where the previous launch left off, so
// workgroup b runs on XCD (b + c) % 8 for a launch-wide c: a workgroup takes
// its XCD from HW_REG_XCC_ID and its rank among that XCD's 32 from b / 8.  Every XCD
// computes the whole router (1 MiB at the Qwen3-30B-A3B shape, mostly served
// from the memory-side cache after the first XCD's read) and the whole
// routing, then works on its eighth of the layer's expert work: the K selected
// experts' rows form K*I (slot, row) pairs in 128-row blocks, and XCD x owns
// every eighth block from block x (CR = K*I/8 pairs).  It computes their gated
// products h (gate/up rows) and then their contribution to every output row
// (the matching down-matrix columns), so all XCDs read the same number of
// weight bytes.  The gate/up rows of the experts predicted for the layer are
// requested first of all (the previous layer's kernel predicts them from its
// own router input); the routing then confirms or replaces each slot's
// expert.  Data moves between the workgroups of one XCD through that
// XCD's L2: values are stored as 64-bit (tag, f32) words with plain stores
// and read after an L1 invalidate (buffer_inv sc0) with plain loads, polled
// until every word carries this step's tag.  The tag is (run << 10 | layer
// position + 1), run being a counter the chain's last kernel advances, so a
// word left by an earlier layer or step (or the zeroed buffer) never matches.
// Across XCDs data moves only at kernel boundaries: each XCD writes its
// partial output rows, and the next layer's kernel (or the final one) adds the
// eight partials to the residual stream.
//
// Per workgroup (512 threads: four control waves, four weight waves; the
// kernel's comment has the details): the control waves load the residual,
// partials and router rows, form rms (f64 sum of squares, cz_rms_inv) and xn,
// and the workgroup's E/32 router rows' logits in dotF32 order
// (bit-identical to the reference); the weight waves then request the
// predicted experts' gate/up and down rows (96 KB + 48 KB at the
// Qwen3-30B-A3B shape: the first gate/up row at once, the rest once wave 0
// has polled the logits); control wave 0 takes the XCD's logits and routes
// (moe.zig:435-463's strict '>' scan restated), matches the slots to the
// picks and hands them over; the weight waves load what the prediction
// missed, form the gated products of the XCD, and its down partial of 64
// output rows.  XCD 0's control waves predict the next layer's experts.
// Every wait is bounded by the wall clock: one that runs out sets a word in
// host memory (the host reports it) and the kernel finishes with whatever it
// read, so no wave waits forever.
#pragma once

#include "cz_kernels.h"

#define CZ_NXCD 8
#define CZ_WPX 32                       // workgroups per XCD
#define CZ_FWG (CZ_NXCD * CZ_WPX)       // workgroups per layer launch
#define CZ_FEPW 4                       // router rows per workgroup (E <= 128)
#define CZ_FPOLL_TICKS 2000000ll        // poll limit: 20 ms of the 100 MHz wall clock
#ifndef CZ_PRED_EARLY
#define CZ_PRED_EARLY 1                 // predicted gate/up rows a weight wave requests before the logit poll
#endif

// error bits (host word)
#define CZ_FERR_TIMEOUT 1u

struct FusedArgs {
    LayerDev L;
    const float *rin;             // [H] residual stream before the previous layer's output
    const float *pin;             // [8][H] previous layer's per-XCD partial outputs (zeros before the first)
    uint32_t has_pin;             // 0: the first layer (x = rin exactly)
    float *rout;                  // [H] this layer's input x (written by workgroup 0); null: not kept
    float *pout;                  // [8][H] this layer's per-XCD partial outputs
    unsigned long long *lgx;      // [8][E] tagged logits, one copy per XCD
    unsigned long long *hx;       // [K*I] tagged gated products (XCD x owns [x*CR, (x+1)*CR))
    const uint32_t *run;          // chain-run counter (tag high bits)
    uint32_t *err;                // host-coherent error word
    float *xn_trace;              // nullable [H]
    uint32_t *idx_trace;          // nullable [K]
    float *gates_trace;           // nullable [K]
    uint32_t pos;                 // layer position in the chain, < 1023 (tag low bits)
    float eps;
    const uint32_t *pred_in;      // [K] this layer's predicted experts (kernels with SPEC)
    uint32_t *pred_out;           // nullable [K] the next layer's predicted experts
    unsigned long long *lgpx;     // [E] tagged next-layer logits (XCD 0's exchange)
    const float *rnext;           // [E][H] the next layer's router (with pred_out)
    const float *rbias_next;      // nullable [E] its bias
    uint32_t pred_mode;           // test hooks: 0 as computed, 1 no slot matched, 2 slot 0 unmatched
    unsigned long long *pstat;    // [2] slots predicted, slots whose prediction was picked
    uint32_t poll_mask;           // ~0u; test hook: ~1023u makes this layer's polls wait for a tag
                                  // no layer writes (a written tag's low 10 bits are never 0)
    uint32_t *stop;               // nullable: a speculative run's stop word (streamed layers, slot maps)
    uint32_t stop_code;           // this layer's code in it (run position + 1)
};

typedef float cz_f4 __attribute__((ext_vector_type(4)));

__device__ inline unsigned long long cz_tagged(uint32_t tag, float v) {
    return ((unsigned long long)tag << 32) | __builtin_bit_cast(uint32_t, v);
}

__device__ inline void cz_ferr(uint32_t *err, uint32_t bit) {
    __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Reads n tagged words of this XCD (written by its workgroups since the last
// kernel boundary): word i (i = lane + 64 q, q < NQ) -> out[q]; polls until
// every word the wave reads carries `tag` or the limit runs out.  Wave-level:
// the wave's own loop, no workgroup barrier.
template <int NQ>
__device__ inline void cz_poll_tagged(const unsigned long long *p, uint32_t n, uint32_t tag, float (&out)[NQ],
                                      uint32_t *err) {
    const uint32_t lane = cz_lane();
    const long long t0 = wall_clock64();
    for (;;) {
        asm volatile("buffer_inv sc0" ::: "memory");  // this CU's L1 holds nothing stale of p
        // every word requested before the first is waited for (relaxed
        // atomic loads: one round trip per poll, not one per word)
        unsigned long long v[NQ];
#pragma unroll
        for (int q = 0; q < NQ; ++q)
            v[q] = __hip_atomic_load(p + min(lane + 64u * q, n - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        bool ok = true;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            out[q] = __builtin_bit_cast(float, (uint32_t)v[q]);
            ok = ok && (uint32_t)(v[q] >> 32) == tag;
        }
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) return;  // wave-uniform
        if (wall_clock64() - t0 > CZ_FPOLL_TICKS) {           // a scalar clock: the same in every lane
            if (lane == 0) cz_ferr(err, CZ_FERR_TIMEOUT);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Waits until the LDS word *p reaches target (another wave of the workgroup
// advances it), bounded by the wall clock like the polls.
__device__ inline void cz_lds_wait(const uint32_t *p, uint32_t target, uint32_t *err) {
    const long long t0 = wall_clock64();
    while (__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if (wall_clock64() - t0 > CZ_FPOLL_TICKS) {
            if (cz_lane() == 0) cz_ferr(err, CZ_FERR_TIMEOUT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
}

// Top-k of E <= 128 logits held by one wave (lane l: experts l and l + 64), by
// value then lower id, K passes of two wave maxima; lane z < K returns pick z.
// The predicted experts only: any order-preserving choice serves, this one
// picks what the routing's strict '>' scan picks on the same logits (exp is
// monotonic) except where exp rounds two logits to one value.
__device__ inline uint32_t cz_topk_wave(const float (&lg)[2], uint32_t E, uint32_t K) {
    const uint32_t lane = cz_lane();
    uint32_t vk[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t e = lane + 64u * m, b = __builtin_bit_cast(uint32_t, lg[m]);
        const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // orders like the float
        vk[m] = (e < E && lg[m] == lg[m]) ? max(ord, 1u) : 0u;
    }
    uint32_t mine = 0;
    for (uint32_t z = 0; z < K; ++z) {
        const uint32_t bvk = cz_wave_max_u32(max(vk[0], vk[1]));
        uint32_t ik = 0;
#pragma unroll
        for (int m = 0; m < 2; ++m) ik = max(ik, (bvk != 0u && vk[m] == bvk) ? 0xffffffffu - (lane + 64u * m) : 0u);
        const uint32_t bik = cz_wave_max_u32(ik);
        const uint32_t best = bvk == 0u ? 0u : 0xffffffffu - bik;
#pragma unroll
        for (int m = 0; m < 2; ++m) vk[m] = lane + 64u * m == best ? 0u : vk[m];
        if (lane == z) mine = best;
    }
    return mine;
}

// NB = H/64 bytes per lane of a gate/up row; RW = gate/up rows per wave
// (CR = 128 RW pairs per XCD).  SPEC: the layer has predicted experts.
//
// Waves 0-3 of a workgroup (the control waves) compute the RMS, the router
// rows, the exchange of logits and the routing; waves 4-7 (the weight waves)
// request and use the expert weights.  A wave's vector loads complete in the
// order they were issued, so a wave that has the layer's weights in flight
// cannot poll the exchange without waiting for all of them: the two roles
// need waves of their own.  The weight waves also wait for the control
// waves' first loads (the router input in LDS) before they request anything,
// and the control waves issue at a higher priority: the CU's memory pipeline
// is shared, and the control waves' loads are on the critical path.  Both
// workgroup barriers come before the weight waves' requests (a wave stalled
// issuing loads would hold one up); after them control wave 0 routes alone
// and hands the slots to the weight waves through an LDS stage word.
//
// Pairs: the K*I (slot, row) pairs form 8 RW blocks of 128 rows (block g is
// rows 128 (g % NBI) .. + 127 of slot g / NBI, NBI = I/128), and XCD x owns
// blocks x + 8 t (t < RW): a slot's blocks lie on different XCDs, so a slot
// whose expert changes touches the XCDs evenly.  Weight wave q of workgroup
// w owns row w * 4 + q of each of the XCD's RW blocks (its row r in block
// t = r), and the XCD's gated products sit block by block (t * 128 + row).
//
// Gate/up rows: lane l reads the 16-byte pieces 1024 q + 16 l of the row
// (q < NB/16; for H = 512 the 8 bytes 8 l), so every load instruction covers
// whole lines.  Down: a weight wave owns DR = min(8, NB/2) output rows per
// pass over NB/16 passes (at least one), 8 lanes per row; lane j of a row
// reads the 16 columns 16 j of the XCD's block t (one 128-column scale block,
// one line of the row); the row's sum is taken over its 8 lanes.
//
// Predicted experts (SPEC): the previous layer's kernel left this layer's
// top-k on its own router input in pred_in; the weight waves request the
// gate/up and down rows of those experts as soon as the router input is
// ready, so the weights stream while the control waves compute the router
// and the routing: CZ_PRED_EARLY gate/up rows at once, the others (and the
// down rows) once wave 0 has polled the XCD's logits (an LDS word), so that
// the poll's round trip does not wait behind the whole request in the CU's
// memory pipeline.  Each slot then keeps its predicted expert if the routing picked
// it (matched once per pick), and a slot whose prediction missed gets a
// picked expert that no slot predicted and loads its rows again.  The
// routing itself, the gates and the usage counters are the layer's own; the
// prediction only decides which weights are requested early.  Without SPEC
// every slot loads after the routing.  XCD 0's control waves predict the next
// layer's experts (its router rows on this layer's router input) once their
// routing is done, off the weight waves' path.
// STOP: a speculative run of streamed layers (A.stop and slot maps set); the
// resident chain's kernels are built without it.
template <int NB, int RW, bool SPEC, bool STOP = false>
__global__ __launch_bounds__(512) void k_layer_fused(FusedArgs A) {
    constexpr uint32_t H = 64 * NB, H4 = H / 4;
    constexpr uint32_t QX = (H4 + 255) / 256;                    // float4 of a row per thread
    constexpr uint32_t QR = (CZ_FEPW * H4 + 255) / 256;          // float4 of the router rows per thread
    constexpr uint32_t QN = H4 / 64;                             // float4 of a router row per lane
    constexpr uint32_t CR = 128 * RW, RPW = CR / CZ_WPX;
    constexpr uint32_t OPW = H / CZ_WPX;                         // output rows per workgroup
    constexpr uint32_t DR = NB / 2 < 8 ? NB / 2 : 8;             // output rows per wave and pass
    constexpr uint32_t DP = NB / 16 > 1 ? NB / 16 : 1;           // passes
    constexpr uint32_t GB = NB >= 16 ? 16 : NB;                  // bytes per gate/up load
    constexpr uint32_t GQ = NB / GB;                             // gate/up loads per row
    constexpr uint32_t NBH = H / CZ_BLOCK;                       // scale blocks of a gate/up row
    constexpr uint32_t NSG = 2 * NBH * RW, NSQ = (NSG + 63) / 64;
    constexpr uint32_t NQH = CR / 64;                            // gated products per lane (the XCD's)
    static_assert(RPW == 4 * RW && OPW == 4 * DR * DP && OPW <= 64 && QR * 256 == CZ_FEPW * H4, "shape");
    static_assert(CZ_WPX * 4 == CZ_BLOCK && QN * 64 == H4 && NQH * 64 == CR && RW <= 64, "shape");
    const LayerDev &L = A.L;
    const uint32_t E = L.E, K = L.K, I = L.I;
    const uint32_t NBI = I / CZ_BLOCK;                           // 128-row blocks of a slot
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));
    // a speculative run that an earlier layer stopped: nothing to do (the
    // word was written before this launch, so every workgroup reads the same
    // value; this layer's own code, stored by one of its workgroups while a
    // late one starts, does not count)
    if constexpr (STOP) {
        const uint32_t sw = __builtin_nontemporal_load(A.stop);
        if (sw != 0u && sw < A.stop_code) return;  // grid-uniform
    }

    // xn, and xn and the router rows chain-major for the dotF32 chains: chain
    // j (elements j + 32 i, i < H/32) is one row of RS floats (RS = H/32 + 4
    // puts the 16-byte reads of 16 consecutive chains in distinct banks)
    constexpr uint32_t RS = H / 32 + 4;
    __shared__ __align__(16) float s_x[H];
    __shared__ __align__(16) float s_xt[32 * RS];
    __shared__ __align__(16) float s_rc[CZ_FEPW * 32 * RS];
    __shared__ __align__(16) float s_h[4][CR];              // each weight wave's copy of the XCD's gated products
    __shared__ float s_sc[4][2 * NBH * RW];                 // each weight wave's gate/up block scales
    __shared__ double s_ss[4];
    __shared__ uint32_t s_idx[CZ_MAX_K];                    // the routing: picks, gates
    __shared__ float s_gate[CZ_MAX_K];
    __shared__ uint32_t s_stage;                            // 2: slots' experts and gates are in LDS
    __shared__ uint32_t s_pe[CZ_MAX_K];                     // predicted expert of each slot
    __shared__ uint32_t s_fp[CZ_MAX_K];                     // pick position of each slot's expert
    __shared__ uint32_t s_rl;                               // slots whose rows load after the routing (bits)
    __shared__ uint32_t s_lgp;                              // 1: wave 0 has polled the XCD's logits
    __shared__ int32_t s_slot[STOP ? 128 : 1];              // STOP: the layer's slot map (E <= 128)

    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const uint32_t xcd = xcc & (CZ_NXCD - 1), w = blockIdx.x / CZ_NXCD;
    // the run counter through the scalar cache (written before this launch)
    const uint32_t tag = (*(const __attribute__((address_space(4))) uint32_t *)A.run << 10) | ((A.pos + 1u) & 1023u);
    const uint32_t ptag = tag & A.poll_mask;  // the tag this layer's polls wait for
    const uint32_t e0 = w * CZ_FEPW;
    const uint32_t ne = E > e0 ? min((uint32_t)CZ_FEPW, E - e0) : 0u;
    if (tid == 0) {
        s_stage = 0;
        s_lgp = 0;
    }

    if (wave < 4) {
        // ================= control waves (threads 0..255) =================
        // their requests go first: a higher issue priority than the weight
        // waves' (s_setprio: the order in which the CU's waves issue)
        __builtin_amdgcn_s_setprio(3);
        // ---- every load of the first phase at once: the next layer's router
        // row (XCD 0), residual, partials, router rows
        const bool pred_out = A.pred_out != nullptr && xcd == 0;  // uniform
        cz_f4 rn[QN];
        if (pred_out) {
            const cz_f4 *src = reinterpret_cast<const cz_f4 *>(A.rnext) + (uint64_t)min(e0 + wave, E - 1) * H4;
#pragma unroll
            for (uint32_t q = 0; q < QN; ++q) rn[q] = src[lane + 64 * q];
        }
        cz_f4 xv4[QX];
        cz_f4 pv[QX][CZ_NXCD];
        {
            const cz_f4 *r4 = reinterpret_cast<const cz_f4 *>(A.rin);
            const cz_f4 *p4 = reinterpret_cast<const cz_f4 *>(A.pin);
#pragma unroll
            for (uint32_t q = 0; q < QX; ++q) {
                xv4[q] = r4[min(tid + 256 * q, H4 - 1)];
#pragma unroll
                for (uint32_t x = 0; x < CZ_NXCD; ++x) pv[q][x] = p4[x * H4 + min(tid + 256 * q, H4 - 1)];
            }
        }
        int32_t sm = 0;
        if constexpr (STOP) sm = L.slot_map[min(tid, E - 1)];  // to LDS before B1
        cz_f4 rr[QR];
        {
            const cz_f4 *src = reinterpret_cast<const cz_f4 *>(L.router) + (uint64_t)min(e0, E - 1) * H4;
            const uint32_t last = ne > 0 ? ne * H4 - 1 : 0u;
#pragma unroll
            for (uint32_t q = 0; q < QR; ++q) rr[q] = src[min(tid + 256 * q, last)];  // clamped: in bounds
        }
        __builtin_amdgcn_sched_barrier(0);  // every first-phase load is in flight
        // ---- x = residual + (((p0 + p1) + ...) + p7); rms (rmsnorm.zig:32-40, unit weight)
        double ss = 0.0;
#pragma unroll
        for (uint32_t q = 0; q < QX; ++q) {
            cz_f4 v = xv4[q];
            cz_f4 o = pv[q][0];
#pragma unroll
            for (uint32_t x = 1; x < CZ_NXCD; ++x) o = o + pv[q][x];
            if (A.has_pin) v = v + o;  // uniform
            xv4[q] = v;
            if (tid + 256 * q < H4)
                ss += ((double)v.x * (double)v.x + (double)v.y * (double)v.y) +
                      ((double)v.z * (double)v.z + (double)v.w * (double)v.w);
        }
        ss = cz_wave_sum_f64_dpp(ss);
        if (lane == 0) s_ss[wave] = ss;
        if constexpr (STOP)
            if (tid < E) s_slot[tid] = sm;
        // router rows to LDS, chain-major (rows past ne are never read)
#pragma unroll
        for (uint32_t q = 0; q < QR; ++q) {
            const uint32_t f = tid + 256 * q, row = f / H4, c = 4 * (f % H4);  // elements c .. c + 3 of the row
            float *d = s_rc + (row * 32 + c % 32) * RS + c / 32;
            d[0] = rr[q].x;
            d[RS] = rr[q].y;
            d[2 * RS] = rr[q].z;
            d[3 * RS] = rr[q].w;
        }
        __syncthreads();  // B1
        const float inv = cz_rms_inv(((s_ss[0] + s_ss[1]) + s_ss[2]) + s_ss[3], H, A.eps);
#pragma unroll
        for (uint32_t q = 0; q < QX; ++q) {
            const uint32_t i = tid + 256 * q;
            if (i < H4) {
                const cz_f4 v = xv4[q];
                const cz_f4 y = v * inv;
                reinterpret_cast<cz_f4 *>(s_x)[i] = y;
                float *d = s_xt + (4 * i % 32) * RS + 4 * i / 32;
                d[0] = y.x;
                d[RS] = y.y;
                d[2 * RS] = y.z;
                d[3 * RS] = y.w;
                if (blockIdx.x == 0) {
                    if (A.rout) reinterpret_cast<cz_f4 *>(A.rout)[i] = v;
                    if (A.xn_trace) reinterpret_cast<cz_f4 *>(A.xn_trace)[i] = y;
                }
            }
        }
        __syncthreads();  // B2: xn in s_x; the weight waves start their requests
        // ---- router logits of experts e0 .. e0 + ne - 1 (dotF32 order, cz_router_combine)
        if (wave < (ne + 1) / 2) {  // half-wave hw of wave q owns expert e0 + 2 q + hw
            const uint32_t hw = lane >> 5, j = lane & 31, el = min(2 * wave + hw, ne - 1);
            const cz_f4 *xr = reinterpret_cast<const cz_f4 *>(s_xt + j * RS);
            const cz_f4 *wr = reinterpret_cast<const cz_f4 *>(s_rc + (el * 32 + j) * RS);
            float acc = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < H / 128; ++q) {  // elements j + 32 i, i = 4 q .. 4 q + 3, in order
                const cz_f4 a = xr[q], b = wr[q];
                acc = __builtin_fmaf(a.x, b.x, acc);
                acc = __builtin_fmaf(a.y, b.y, acc);
                acc = __builtin_fmaf(a.z, b.z, acc);
                acc = __builtin_fmaf(a.w, b.w, acc);
            }
            float lgt = cz_router_combine(acc, j, hw * 32);
            const uint32_t e = e0 + 2 * wave + hw;
            if (L.router_bias) lgt = lgt + L.router_bias[min(e, E - 1)];
            if (j == 0 && 2 * wave + hw < ne) A.lgx[(uint64_t)xcd * E + e] = cz_tagged(tag, lgt);
        }
        // ---- XCD 0: the next layer's logits on this router input (one row
        // per control wave), exchanged through XCD 0's L2
        if (pred_out && wave < ne) {
            float t = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < QN; ++q) {
                const cz_f4 a = reinterpret_cast<const cz_f4 *>(s_x)[lane + 64 * q];
                t = __builtin_fmaf(a.x, rn[q].x, t);
                t = __builtin_fmaf(a.y, rn[q].y, t);
                t = __builtin_fmaf(a.z, rn[q].z, t);
                t = __builtin_fmaf(a.w, rn[q].w, t);
            }
            t = cz_wave_sum_dpp(t);
            if (A.rbias_next) t = t + A.rbias_next[e0 + wave];
            if (lane == 0) A.lgpx[e0 + wave] = cz_tagged(tag, t);
        }
        if (wave != 0) return;
        // ---- wave 0: the XCD's logits, routing (moe.zig:435-463, the
        // single-wave routing of the decode kernels: no workgroup barrier)
        float lg[2] = {0.0f, 0.0f};
        cz_poll_tagged<2>(A.lgx + (uint64_t)xcd * E, E, ptag, lg, A.err);
        if (lane == 0) __hip_atomic_store(&s_lgp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint32_t o_pos = 0, o_id = 0;
        float o_gate = 0.0f;
        cz_route_wave_regs<2>(lg, E, K, L.norm_topk, s_idx, s_gate, o_pos, o_id, o_gate);
        // a speculative run: a pick with no pool slot stops the run here,
        // before the routing is counted or published.  Every workgroup routes
        // the same logits, so every one of them stops; the weight waves see
        // stage 3 and end too.
        if constexpr (STOP) {
            const bool miss = lane < K && s_slot[o_id] < 0;
            if (__builtin_amdgcn_ballot_w64(miss) != 0) {  // wave-uniform
                if (lane == 0) {
                    if (blockIdx.x == 0) atomicCAS(A.stop, 0u, A.stop_code);
                    __hip_atomic_store(&s_stage, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
                return;
            }
        }
        if (blockIdx.x == 0 && lane < K) cz_bump_usage(L.usage, E, o_id);
        // each slot keeps its predicted expert if it was picked (each pick
        // matched once, slots in order: the n-th slot predicting e takes the
        // n-th pick of e); the other slots take the unmatched picks in pick
        // order and load after the routing.  Lane z = slot z = pick z.  Test
        // hooks: mode 1 matches no slot, mode 2 leaves slot 0 unmatched.
        {
            const uint32_t a = lane < K ? o_id : 0xfffffffeu;
            const uint32_t pe = (SPEC && lane < K) ? s_pe[lane] : 0xffffffffu;  // equals no id
            const bool elig = SPEC && lane < K && A.pred_mode != 1 && !(A.pred_mode == 2 && lane == 0);
            const uint32_t pel = elig ? pe : 0xffffffffu;
            uint32_t cnt_a = 0, dup_p = 0;
            for (uint32_t q = 0; q < K; ++q) {
                const uint32_t aq = (uint32_t)__builtin_amdgcn_readlane((int)a, (int)q);
                const uint32_t pq = (uint32_t)__builtin_amdgcn_readlane((int)pel, (int)q);
                cnt_a += aq == pel ? 1u : 0u;
                dup_p += (q < lane && pq == pel) ? 1u : 0u;
            }
            const bool matched = elig && dup_p < cnt_a;
            uint32_t fp = K;
            for (uint32_t q = 0, seen = 0; q < K; ++q) {
                const uint32_t aq = (uint32_t)__builtin_amdgcn_readlane((int)a, (int)q);
                if (matched && aq == pel) {
                    if (seen == dup_p && fp == K) fp = q;
                    ++seen;
                }
            }
            uint32_t used = 0;  // picks taken by matched slots
            for (uint32_t q = 0; q < K; ++q) {
                const uint32_t fq = (uint32_t)__builtin_amdgcn_readlane((int)fp, (int)q);
                used |= fq < K ? 1u << fq : 0u;
            }
            const uint32_t kmask = K >= 32 ? 0xffffffffu : (1u << K) - 1u;
            const uint32_t rl = (uint32_t)__builtin_amdgcn_ballot_w64(lane < K && !matched) & kmask;
            if (lane < K && !matched) {  // the r-th unmatched slot takes the r-th untaken pick
                const uint32_t r = (uint32_t)__builtin_popcount(rl & ((1u << lane) - 1u));
                uint32_t m = ~used & kmask;
                for (uint32_t i = 0; i < r; ++i) m &= m - 1u;
                fp = (uint32_t)__builtin_ctz(m);
            }
            if (lane < K) s_fp[lane] = fp;
            if (lane == 0) s_rl = rl;
            // the routing, the slots and the gates are in LDS (one wave's LDS
            // writes complete in order): the weight waves may go on
            asm volatile("" ::: "memory");
            if (lane == 0) __hip_atomic_store(&s_stage, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (lane == 0 && SPEC && blockIdx.x == 0) {
                atomicAdd(A.pstat, (unsigned long long)K);
                atomicAdd(A.pstat + 1, (unsigned long long)(K - (uint32_t)__builtin_popcount(rl)));
            }
        }
        if (blockIdx.x == 0 && lane < K) {
            if (A.idx_trace) A.idx_trace[lane] = o_id;
            if (A.gates_trace) A.gates_trace[lane] = o_gate;
        }
        // ---- XCD 0, workgroup 0: the next layer's predicted experts (the
        // top-k of the exchanged logits)
        if (pred_out && w == 0) {
            float pl[2] = {0.0f, 0.0f};
            cz_poll_tagged<2>(A.lgpx, E, ptag, pl, A.err);
            const uint32_t pe = cz_topk_wave(pl, E, K);
            if (lane < K) A.pred_out[lane] = pe;
        }
        return;
    }

    // ================= weight waves (threads 256..511) =================
    const uint32_t mw = wave - 4;
    const uint32_t rib = w * 4 + mw;  // the wave's row in each of the XCD's blocks
    uint32_t jr[RW], zr[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const uint32_t g = xcd + CZ_NXCD * r;
        zr[r] = min(g / NBI, K - 1);
        jr[r] = (g - (g / NBI) * NBI) * CZ_BLOCK + rib;
    }
    // down: rows r0 + DR p + lane / 8 (p < DP), columns 16 (lane % 8) of block i
    const uint32_t dj = lane & 7, dq = lane >> 3;
    const uint32_t r0 = w * OPW + mw * DR * DP;
    uint64_t slr[RW];
    float scg[NSQ], scv = 0.0f;
    uint32_t dg[RW][NB / 4], du[RW][NB / 4];
    uint4 dd[DP][RW];
    // the expert of slot z (lane-varying z < K): the prediction in lanes
    // 0..K-1 of pz until the routing is known, then the routed one
    uint32_t pz = 0;
    bool routed = !SPEC;
    // an expert's slot: with STOP from the LDS copy of the slot map (valid
    // after B1; a missing slot reads slot 0, in bounds, and never reaches a
    // product: the run stops)
    auto slot_of = [&](uint32_t e) __attribute__((always_inline)) -> uint64_t {
        if constexpr (STOP) return (uint64_t)max(s_slot[e], 0);
        else return cz_slot(L, e);
    };
    auto expert_of = [&](uint32_t z) __attribute__((always_inline)) -> uint32_t {
        if (routed) return min(s_idx[s_fp[z]], E - 1);
        return (uint32_t)__builtin_amdgcn_ds_bpermute((int)(z << 2), (int)pz);
    };
    // gate/up scales of the wave's rows (gathered, 64 to a load): every
    // lane derives its row, block and expert itself (no per-lane choice
    // among the rows' registers)
    auto load_scales = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t k = 0; k < NSQ; ++k) {
            const uint32_t t = min(lane + 64 * k, NSG - 1), r = t / (2 * NBH), m = (t / NBH) & 1, b = t % NBH;
            const uint32_t g = xcd + CZ_NXCD * r, z = min(g / NBI, K - 1), jj = (g - (g / NBI) * NBI) * CZ_BLOCK + rib;
            const uint64_t sl = slot_of(expert_of(z));
            scg[k] = L.es[sl * L.es_stride + (uint64_t)m * L.nbI * L.nbH + (uint64_t)(jj / CZ_BLOCK) * L.nbH + b];
        }
    };
    // down scale of block i in lane i (the wave's rows share one 128-row block)
    auto load_down_scale = [&]() __attribute__((always_inline)) {
        const uint32_t t = min(lane, (uint32_t)RW - 1);
        const uint32_t g = xcd + CZ_NXCD * t, z = min(g / NBI, K - 1), col = (g - (g / NBI) * NBI) * CZ_BLOCK;
        const uint64_t sl = slot_of(expert_of(z));
        scv = L.es[sl * L.es_stride + 2ull * L.nbI * L.nbH + (uint64_t)(r0 / CZ_BLOCK) * L.nbI + col / CZ_BLOCK];
    };
    auto load_row = [&](int r) __attribute__((always_inline)) {
        const uint8_t *wg = L.ew + slr[r] * L.ew_stride + (uint64_t)jr[r] * H;
#pragma unroll
        for (uint32_t q = 0; q < GQ; ++q) {
            const uint32_t c = 1024 * q + GB * lane;
            if constexpr (GB == 16) {
                const uint4 a = cz_ld_nt16(wg + c);
                const uint4 b = cz_ld_nt16(wg + (uint64_t)I * H + c);
                dg[r][4 * q] = a.x; dg[r][4 * q + 1] = a.y; dg[r][4 * q + 2] = a.z; dg[r][4 * q + 3] = a.w;
                du[r][4 * q] = b.x; du[r][4 * q + 1] = b.y; du[r][4 * q + 2] = b.z; du[r][4 * q + 3] = b.w;
            } else {
                const uint2 a = *reinterpret_cast<const uint2 *>(wg + c);
                const uint2 b = *reinterpret_cast<const uint2 *>(wg + (uint64_t)I * H + c);
                dg[r][0] = a.x; dg[r][1] = a.y;
                du[r][0] = b.x; du[r][1] = b.y;
            }
        }
    };
    auto load_down = [&](int i) __attribute__((always_inline)) {
        const uint8_t *wd = L.ew + slr[i] * L.ew_stride + 2ull * I * H + (jr[i] - rib) + 16 * dj;
#pragma unroll
        for (uint32_t p = 0; p < DP; ++p) {
            const uint32_t row = r0 + DR * p + min(dq, DR - 1);
            dd[p][i] = cz_ld_nt16(wd + (uint64_t)row * I);
        }
    };
    if constexpr (SPEC) {
        pz = min(A.pred_in[min(lane, K - 1)], E - 1);
        if (mw == 0 && lane < K) s_pe[lane] = pz;  // for the control waves' matching
    }
    // the control waves' first loads and their logits' exchange first: they
    // are on the layer's critical path (a saturated memory pipeline would
    // hold up the exchange's polls)
    __syncthreads();  // B1
    __syncthreads();  // B2
    if constexpr (SPEC) {  // the predicted experts' rows
#pragma unroll
        for (int r = 0; r < RW; ++r) slr[r] = slot_of((uint32_t)__builtin_amdgcn_readlane((int)pz, (int)zr[r]));
        load_scales();
        load_down_scale();
        // the first rows now, the rest once the logits are polled: a poll's
        // round trip waits behind every request already in the CU's memory
        // pipeline
        constexpr int RE = CZ_PRED_EARLY < RW ? CZ_PRED_EARLY : RW;
#pragma unroll
        for (int r = 0; r < RE; ++r) load_row(r);
        if constexpr (RE < RW) cz_lds_wait(&s_lgp, 1u, A.err);
#pragma unroll
        for (int r = RE; r < RW; ++r) load_row(r);
#pragma unroll
        for (int i = 0; i < RW; ++i) load_down(i);
    }
    cz_lds_wait(&s_stage, 2u, A.err);  // the slots' experts and the gates are known
    if constexpr (STOP)
        if (__hip_atomic_load(&s_stage, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 3u) return;  // the run stopped
    routed = true;
    // gated product of row r: h = g_z * silu(Wg x) * (Wu x), to its place in block r
    auto gated_products = [&]() __attribute__((always_inline)) {
        float gz[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) gz[r] = s_gate[s_fp[zr[r]]];
        // ---- the scales to the lanes that use them
#pragma unroll
        for (uint32_t k = 0; k < NSQ; ++k)
            if (lane + 64 * k < NSG) s_sc[mw][lane + 64 * k] = scg[k];
        __builtin_amdgcn_wave_barrier();
        float sg[RW][GQ], su[RW][GQ];
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (uint32_t q = 0; q < GQ; ++q) {
                const uint32_t b = (1024 * q + GB * lane) / CZ_BLOCK;
                sg[r][q] = s_sc[mw][r * 2 * NBH + b];
                su[r][q] = s_sc[mw][r * 2 * NBH + NBH + b];
            }
        float xv[NB];
#pragma unroll
        for (uint32_t q = 0; q < GQ; ++q) {
            const float4 *xs = reinterpret_cast<const float4 *>(s_x + 1024 * q + GB * lane);
#pragma unroll
            for (uint32_t k = 0; k < GB / 4; ++k) {
                const float4 t = xs[k];
                xv[GB * q + 4 * k] = t.x; xv[GB * q + 4 * k + 1] = t.y; xv[GB * q + 4 * k + 2] = t.z; xv[GB * q + 4 * k + 3] = t.w;
            }
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            float ag = 0.0f, au = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < GQ; ++q) {
                float pg = 0.0f, pu = 0.0f;
#pragma unroll
                for (uint32_t k = 0; k < GB / 4; ++k) {
                    pg = cz_dot4_raw(dg[r][GB / 4 * q + k], &xv[GB * q + 4 * k], pg);
                    pu = cz_dot4_raw(du[r][GB / 4 * q + k], &xv[GB * q + 4 * k], pu);
                }
                ag = __builtin_fmaf(pg, sg[r][q], ag);
                au = __builtin_fmaf(pu, su[r][q], au);
            }
            ag = cz_wave_sum_dpp(ag);
            au = cz_wave_sum_dpp(au);
            if (lane == (uint32_t)r)
                A.hx[(uint64_t)xcd * CR + CZ_BLOCK * r + rib] = cz_tagged(tag, gz[r] * (cz_silu_fast(ag) * au));
        }
    };
    {
        const uint32_t rl = s_rl;
        bool any = false;  // uniform: a row of the wave loads after the routing
#pragma unroll
        for (int r = 0; r < RW; ++r) any = any || ((rl >> zr[r]) & 1u) != 0u;
        if (!any) {
            // every row was requested before the routing, in the order the
            // products use them: the waits before row r's products cover its
            // own rows only, not the down rows requested after them (a join
            // with the path below would make them wait for nearly every
            // request in flight); the markers keep the two copies apart
            gated_products();
            asm volatile("; gated products: every row requested before the routing");
        } else {
#pragma unroll
            for (int r = 0; r < RW; ++r)
                if ((rl >> zr[r]) & 1u) slr[r] = slot_of(min(s_idx[s_fp[zr[r]]], E - 1));
            load_scales();
            load_down_scale();
#pragma unroll
            for (int r = 0; r < RW; ++r)
                if ((rl >> zr[r]) & 1u) load_row(r);
#pragma unroll
            for (int i = 0; i < RW; ++i)
                if ((rl >> zr[i]) & 1u) load_down(i);
            gated_products();
            asm volatile("; gated products: rows requested after the routing");
        }
    }

    // ---- dequantised down weights (e4m3 * block scale, fp8.zig:105), while
    // the XCD's gated products arrive
    float wq[DP][RW][16];
#pragma unroll
    for (uint32_t p = 0; p < DP; ++p)
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const float sc = cz_readlane(scv, i);
            const uint32_t wv[4] = {dd[p][i].x, dd[p][i].y, dd[p][i].z, dd[p][i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const cz_float2 lo = cz_fp8x2_lo(wv[k]), hi = cz_fp8x2_hi(wv[k]);
                wq[p][i][4 * k] = lo.x * sc;
                wq[p][i][4 * k + 1] = lo.y * sc;
                wq[p][i][4 * k + 2] = hi.x * sc;
                wq[p][i][4 * k + 3] = hi.y * sc;
            }
        }
    // materialise them here: without a use the compiler would move the
    // multiplies past the wait below, onto the critical path
#pragma unroll
    for (uint32_t p = 0; p < DP; ++p)
#pragma unroll
        for (int i = 0; i < RW; ++i)
#pragma unroll
            for (int k = 0; k < 16; ++k) asm volatile("" ::"v"(wq[p][i][k]));

    // ---- the XCD's gated products (every weight wave polls them all into
    // its own LDS copy: no workgroup barrier), then the down rows
    {
        float hq[NQH];
        cz_poll_tagged<NQH>(A.hx + xcd * CR, CR, ptag, hq, A.err);
#pragma unroll
        for (uint32_t q = 0; q < NQH; ++q) s_h[mw][lane + 64 * q] = hq[q];
    }
    __builtin_amdgcn_wave_barrier();
    // each h slice is read once and used for every pass; four independent
    // chains (k) per pass
    float ak[DP][4];
#pragma unroll
    for (uint32_t p = 0; p < DP; ++p)
#pragma unroll
        for (int k = 0; k < 4; ++k) ak[p][k] = 0.0f;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const float4 *hg = reinterpret_cast<const float4 *>(&s_h[mw][128 * i + 16 * dj]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 hv = hg[k];
#pragma unroll
            for (uint32_t p = 0; p < DP; ++p) {
                ak[p][k] = __builtin_fmaf(hv.x, wq[p][i][4 * k], ak[p][k]);
                ak[p][k] = __builtin_fmaf(hv.y, wq[p][i][4 * k + 1], ak[p][k]);
                ak[p][k] = __builtin_fmaf(hv.z, wq[p][i][4 * k + 2], ak[p][k]);
                ak[p][k] = __builtin_fmaf(hv.w, wq[p][i][4 * k + 3], ak[p][k]);
            }
        }
    }
#pragma unroll
    for (uint32_t p = 0; p < DP; ++p) {
        float acc = (ak[p][0] + ak[p][1]) + (ak[p][2] + ak[p][3]);
        // sum over the row's 8 lanes (xor 1, xor 2 within quads, then the two quads)
        acc = acc + cz_dpp<0xB1>(acc);
        acc = acc + cz_dpp<0x4E>(acc);
        acc = acc + cz_dpp<0x141>(acc);  // row_half_mirror: lane i <-> 7 - i of its 8
        if (dj == 0 && dq < DR) A.pout[(uint64_t)xcd * H + r0 + DR * p + dq] = acc;
    }
}

// Placement census for the one-launch decode: workgroup b of a CZ_FWG-wide
// launch records the XCD it runs on.  The layer kernel needs every XCD to
// receive exactly one workgroup of each rank b / 8 = 0 .. 31 (the round-robin
// dispatch of workgroups over the XCDs); the host checks this once at init.
__global__ __launch_bounds__(64) void k_xcd_census(uint32_t *xcc_of) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    if (threadIdx.x == 0) xcc_of[blockIdx.x] = xcc & 0xffu;
}

// After a speculative run of n streamed layers: x becomes the output of the
// last layer that ran.  Without a stop that is k_chain_final's sum over the
// last layer's parts; when layer j stopped (stop word j + 1) it is layer j's
// input, which its workgroup 0 kept in r[j % 2] (j >= 1), or x itself (j =
// 0).  Advances the run counter.
__global__ __launch_bounds__(256) void k_spec_final(float *__restrict__ x, const float *__restrict__ r,
                                                    const float *__restrict__ p, uint32_t H, uint32_t n,
                                                    const uint32_t *stop, uint32_t *run) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t s = *stop;
    if (i < H) {
        if (s == 0u) {
            const float *rin = n == 1 ? x : r + (uint64_t)((n - 1) % 2) * H;
            const float *pin = p + (uint64_t)((n - 1) % 2) * CZ_NXCD * H;
            float o = pin[i];
            for (uint32_t k = 1; k < CZ_NXCD; ++k) o = o + pin[(uint64_t)k * H + i];
            x[i] = rin[i] + o;
        } else if (s >= 2u) {
            x[i] = r[(uint64_t)((s - 1u) % 2u) * H + i];
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *run = *run + 1u;
}

// After the last layer: x = residual + (((p0 + p1) + ...) + p7); advances the
// run counter (the tags of the next chain run differ from this one's).
__global__ __launch_bounds__(256) void k_chain_final(float *__restrict__ x, const float *__restrict__ rin,
                                                     const float *__restrict__ pin, uint32_t H, uint32_t *run) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < H) {
        float o = pin[i];
        for (uint32_t k = 1; k < CZ_NXCD; ++k) o = o + pin[(uint64_t)k * H + i];
        x[i] = rin[i] + o;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *run = *run + 1u;
}
