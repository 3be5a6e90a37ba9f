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
// experts' rows form a flattened space of K*I (slot, row) pairs, and XCD x
// owns the CR = K*I/8 consecutive pairs [x*CR, (x+1)*CR).  It computes their
// gated products h (gate/up rows) and then their contribution to every output
// row (the matching down-matrix columns), so all XCDs read the same number of
// weight bytes.  Data moves between the workgroups of one XCD through that
// XCD's L2: values are stored as 64-bit (tag, f32) words with plain stores
// and read after an L1 invalidate (buffer_inv sc0) with plain loads, polled
// until every word carries this step's tag.  The tag is (run << 10 | layer
// position + 1), run being a counter the chain's last kernel advances, so a
// word left by an earlier layer or step (or the zeroed buffer) never matches.
// Across XCDs data moves only at kernel boundaries: each XCD writes its
// partial output rows, and the next layer's kernel (or the final one) adds the
// eight partials to the residual stream.
//
// Per workgroup (256 threads): its router rows and the residual + partials
// are requested at once; rms (f64 sum of squares, cz_rms_inv); its E/32
// router rows' logits in dotF32 order (bit-identical to the reference); the
// XCD's logits; routing (rank of every expert among all by value then id,
// 4 waves x E/4 candidates, identical to moe.zig:447-460's strict '>' scan);
// then every gate/up row and down row this workgroup needs is requested at
// once (96 KB + 48 KB at the Qwen3-30B-A3B shape), so the layer's 37.7 MB of
// expert weights are streamed in one pass, and the gates are formed while
// they arrive; the gated products of the XCD;
// the down partial of 64 output rows.  Every poll is bounded by the wall
// clock: a poll that runs out sets a word in host memory (the host reports
// it) and the kernel finishes with whatever it read, so no wave waits
// forever.
#pragma once

#include "cz_kernels.h"

#define CZ_NXCD 8
#define CZ_WPX 32                       // workgroups per XCD
#define CZ_FWG (CZ_NXCD * CZ_WPX)       // workgroups per layer launch
#define CZ_FEPW 4                       // router rows per workgroup (E <= 128)
#define CZ_FPOLL_TICKS 2000000ll        // poll limit: 20 ms of the 100 MHz wall clock

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

// Routing of the token from its E logits (E <= 128), by the whole workgroup,
// in two parts so that the weight loads can be issued between them.
// cz_route_picks: every wave holds all logits (lane l: experts l and l + 64),
// forms mx, v = exp(l - mx) and the 64-bit keys (bits(v) + 1) << 32 | ~id (0
// for NaN or past E), which order the experts exactly as moe.zig:447-460's
// scan picks them (larger value first, lower id first among equals), so an
// expert's pick position is the number of keys above its own.  Wave 0 puts
// the keys in LDS; wave q counts, for each expert, the keys above it among
// candidates 32 q .. 32 q + 31 (broadcast reads, independent compares); the
// four counts are summed per expert, and an expert whose count z is < K is
// pick z.  With fewer than K valid experts the scan's remaining picks are
// expert 0 (value v[0]).  R.idx[K] is in LDS after its final barrier.
// cz_route_gates: top = sum of f64(v) of the picks in pick order, den =
// norm_topk ? top : sum of f64(v_e) in expert order, gate = f32(f64(v) /
// den) into R.gate[K], in LDS after its barrier.  Every thread reaches every
// barrier of both.
struct RoutePick {
    uint32_t nvalid;  // experts with a non-NaN value
    float v0;         // v of expert 0
};

struct RouteLds {
    unsigned long long key[128];
    uint32_t cnt[4][128];
    float v[128];
    uint32_t idx[CZ_MAX_K];
    float val[CZ_MAX_K];
    float gate[CZ_MAX_K];
    double all;
};

__device__ inline RoutePick cz_route_picks(const float (&lg)[2], uint32_t E, uint32_t K, uint32_t norm_topk,
                                           RouteLds &R) {
    const uint32_t lane = cz_lane();
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    float v[2];
    float mx = -INFINITY;
#pragma unroll
    for (int m = 0; m < 2; ++m)
        if (lane + 64u * m < E) mx = fmaxf(mx, lg[m]);
    mx = cz_wave_max_dpp(mx);  // NaN-ignoring max (moe.zig:439-440)
    unsigned long long key[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t e = lane + 64u * m;
        v[m] = e < E ? cz_expf(lg[m] - mx) : __builtin_nanf("");
        key[m] = (e < E && v[m] == v[m])
                     ? ((unsigned long long)(__builtin_bit_cast(uint32_t, v[m]) + 1u) << 32) | (0xffffffffull - e)
                     : 0ull;
    }
    const uint32_t nvalid = (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(key[0] != 0)) +
                            (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(key[1] != 0));
    const float v0 = cz_readlane(v[0], 0);
    if (wave == 0) {
        R.key[lane] = key[0];
        R.key[lane + 64] = key[1];
        R.v[lane] = v[0];
        R.v[lane + 64] = v[1];
    }
    __syncthreads();
    uint32_t c0 = 0, c1 = 0;
    const ulonglong2 *kp = reinterpret_cast<const ulonglong2 *>(R.key + 32 * wave);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const ulonglong2 kk = kp[i];  // the same address in every lane
        c0 += (kk.x > key[0]) + (kk.y > key[0]);
        c1 += (kk.x > key[1]) + (kk.y > key[1]);
    }
    R.cnt[wave][lane] = c0;
    R.cnt[wave][lane + 64] = c1;
    if (!norm_topk && wave == 1) {  // sum of f64(v_e) in expert order (moe.zig:445)
        double all = 0.0;
        for (uint32_t e = 0; e < E; ++e) all += (double)cz_readlane(v[e >> 6], e & 63);
        if (lane == 0) R.all = all;
    }
    __syncthreads();
    if (threadIdx.x < 128 && threadIdx.x < E && R.key[threadIdx.x] != 0) {
        const uint32_t e = threadIdx.x;
        const uint32_t z = ((R.cnt[0][e] + R.cnt[1][e]) + R.cnt[2][e]) + R.cnt[3][e];
        if (z < K) {  // z < nvalid
            R.idx[z] = e;
            R.val[z] = R.v[e];
        }
    }
    if (threadIdx.x < K && threadIdx.x >= nvalid) R.idx[threadIdx.x] = 0;  // the scan's pick when nothing is left
    __syncthreads();
    return RoutePick{nvalid, v0};
}

__device__ inline void cz_route_gates(const RoutePick &P, uint32_t K, uint32_t norm_topk, RouteLds &R) {
    if (threadIdx.x < K) {
        const uint32_t z = threadIdx.x;
        double top = 0.0;
        for (uint32_t y = 0; y < K; ++y) top += (double)(y < P.nvalid ? R.val[y] : P.v0);
        const float vz = z < P.nvalid ? R.val[z] : P.v0;
        const double den = norm_topk ? top : R.all;
        R.gate[z] = (float)((double)vz / den);
    }
    __syncthreads();
}

// NB = H/64 bytes per lane of a gate/up row; RW = gate/up rows per wave
// (CR = 128 RW pairs per XCD).  Gate/up rows: lane l reads the 16-byte
// pieces 1024 q + 16 l of the row (q < NB/16; for H = 512 the 8 bytes 8 l),
// so every load instruction covers whole lines.  Down: a wave owns
// DR = min(8, NB/2) output rows per pass over NB/16 passes (at least one),
// 8 lanes per row; lane j of a row reads the 16 columns 128 i + 16 j of the
// XCD's chunk, i < RW (one 128-column block each), so an instruction covers
// a whole line of each of its rows; the row's sum is taken over its 8 lanes.
template <int NB, int RW>
__global__ __launch_bounds__(256) void k_layer_fused(FusedArgs A) {
    constexpr uint32_t H = 64 * NB, H4 = H / 4;
    constexpr uint32_t QX = (H4 + 255) / 256;                    // float4 of a row per thread
    constexpr uint32_t QR = (CZ_FEPW * H4 + 255) / 256;          // float4 of the router rows per thread
    constexpr uint32_t CR = 128 * RW, RPW = CR / CZ_WPX;
    constexpr uint32_t OPW = H / CZ_WPX;                         // output rows per workgroup
    constexpr uint32_t DR = NB / 2 < 8 ? NB / 2 : 8;             // output rows per wave and pass
    constexpr uint32_t DP = NB / 16 > 1 ? NB / 16 : 1;           // passes
    constexpr uint32_t GB = NB >= 16 ? 16 : NB;                  // bytes per gate/up load
    constexpr uint32_t GQ = NB / GB;                             // gate/up loads per row
    static_assert(RPW == 4 * RW && OPW == 4 * DR * DP && OPW <= 64 && QR * 256 == CZ_FEPW * H4, "shape");
    const LayerDev &L = A.L;
    const uint32_t E = L.E, K = L.K, I = L.I;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(tid >> 6));

    // xn, and xn and the router rows chain-major for the dotF32 chains: chain
    // j (elements j + 32 i, i < H/32) is one row of RS floats (RS = H/32 + 4
    // puts the 16-byte reads of 16 consecutive chains in distinct banks)
    constexpr uint32_t RS = H / 32 + 4;
    __shared__ __align__(16) float s_x[H];
    __shared__ __align__(16) float s_xt[32 * RS];
    __shared__ __align__(16) float s_rc[CZ_FEPW * 32 * RS];
    __shared__ __align__(16) float s_h[CR];                 // the XCD's gated products
    __shared__ float s_sc[4][2 * (H / CZ_BLOCK) * RW];      // each wave's gate/up block scales
    __shared__ double s_ss[4];
    __shared__ RouteLds s_rt;
    const uint32_t *s_idx = s_rt.idx;
    const float *s_gate = s_rt.gate;

    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    const uint32_t xcd = xcc & (CZ_NXCD - 1), w = blockIdx.x / CZ_NXCD;
    // the run counter through the scalar cache (written before this launch)
    const uint32_t tag = (*(const __attribute__((address_space(4))) uint32_t *)A.run << 10) | ((A.pos + 1u) & 1023u);

    // ---- every load of the first phase at once: residual, partials, router rows
    const uint32_t e0 = w * CZ_FEPW;
    const uint32_t ne = E > e0 ? min((uint32_t)CZ_FEPW, E - e0) : 0u;
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
    // router rows to LDS, chain-major (rows past ne are never read); they arrive after the residual
#pragma unroll
    for (uint32_t q = 0; q < QR; ++q) {
        const uint32_t f = tid + 256 * q, row = f / H4, c = 4 * (f % H4);  // elements c .. c + 3 of the row
        float *d = s_rc + (row * 32 + c % 32) * RS + c / 32;
        d[0] = rr[q].x;
        d[RS] = rr[q].y;
        d[2 * RS] = rr[q].z;
        d[3 * RS] = rr[q].w;
    }
    __syncthreads();
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
    __syncthreads();

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

    // ---- the XCD's logits, routing
    float lg[2] = {0.0f, 0.0f};
    cz_poll_tagged<2>(A.lgx + (uint64_t)xcd * E, E, tag, lg, A.err);
    const RoutePick pick = cz_route_picks(lg, E, K, L.norm_topk, s_rt);
    if (blockIdx.x == 0 && tid < K) cz_bump_usage(L.usage, E, s_idx[tid]);

    // ---- every weight this workgroup needs, requested at once: the block
    // scales of the wave's rows first (gathered, 64 to a load), then the
    // gate/up rows, then the down rows (fewer than 64 loads per lane, so none
    // waits for an earlier one to return)
    const uint32_t f0 = xcd * CR + w * RPW + wave * RW;  // this wave's gate/up rows (flattened pairs)
    constexpr uint32_t NBH = H / CZ_BLOCK;                // scale blocks of a gate/up row
    constexpr uint32_t NSG = 2 * NBH * RW, NSQ = (NSG + 63) / 64;
    uint64_t slr[RW];
    uint32_t jr[RW], zr[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const uint32_t f = f0 + r, z = min(f / I, K - 1);
        zr[r] = z;
        jr[r] = f - z * I;
        slr[r] = cz_slot(L, min(s_idx[z], E - 1));
    }
    float scg[NSQ];
#pragma unroll
    for (uint32_t k = 0; k < NSQ; ++k) {
        const uint32_t t = min(lane + 64 * k, NSG - 1), r = t / (2 * NBH), m = (t / NBH) & 1, b = t % NBH;
        uint64_t sl = slr[0];
        uint32_t jj = jr[0];
#pragma unroll
        for (int q = 1; q < RW; ++q)
            if (r == (uint32_t)q) { sl = slr[q]; jj = jr[q]; }
        scg[k] = L.es[sl * L.es_stride + (uint64_t)m * L.nbI * L.nbH + (uint64_t)(jj / CZ_BLOCK) * L.nbH + b];
    }
    // down: rows r0 + DR p + lane / 8 (p < DP), columns 128 i + 16 (lane % 8) of the chunk
    const uint32_t dj = lane & 7, dq = lane >> 3;
    const uint32_t r0 = w * OPW + wave * DR * DP;
    uint64_t sld[RW];
    uint32_t jcd[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const uint32_t fc = xcd * CR + 128 * i, zc = min(fc / I, K - 1);
        jcd[i] = fc - zc * I;
        sld[i] = cz_slot(L, min(s_idx[zc], E - 1));
    }
    float scd;
    {
        const uint32_t t = min(lane, DP * RW - 1), pp = t / RW, ii = t % RW;
        uint64_t sl = sld[0];
        uint32_t jj = jcd[0];
#pragma unroll
        for (int q = 1; q < RW; ++q)
            if (ii == (uint32_t)q) { sl = sld[q]; jj = jcd[q]; }
        const uint32_t row = r0 + DR * pp;  // the pass's rows share one 128-row block
        scd = L.es[sl * L.es_stride + 2ull * L.nbI * L.nbH + (uint64_t)(row / CZ_BLOCK) * L.nbI + jj / CZ_BLOCK];
    }
    uint32_t dg[RW][NB / 4], du[RW][NB / 4];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
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
    }
    __builtin_amdgcn_sched_barrier(0);  // the scales and every gate/up row are requested

    // ---- the gates, while the weights are on their way
    cz_route_gates(pick, K, L.norm_topk, s_rt);
    float gz[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) gz[r] = s_gate[zr[r]];
    if (blockIdx.x == 0 && tid < K) {
        if (A.idx_trace) A.idx_trace[tid] = s_idx[tid];
        if (A.gates_trace) A.gates_trace[tid] = s_gate[tid];
    }

    // ---- the scales to the lanes that use them
#pragma unroll
    for (uint32_t k = 0; k < NSQ; ++k)
        if (lane + 64 * k < NSG) s_sc[wave][lane + 64 * k] = scg[k];
    __builtin_amdgcn_wave_barrier();
    float sg[RW][GQ], su[RW][GQ];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (uint32_t q = 0; q < GQ; ++q) {
            const uint32_t b = (1024 * q + GB * lane) / CZ_BLOCK;
            sg[r][q] = s_sc[wave][r * 2 * NBH + b];
            su[r][q] = s_sc[wave][r * 2 * NBH + NBH + b];
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
    // gated product of row r: h = g_z * silu(Wg x) * (Wu x)
    auto gate_up_row = [&](int r) {
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
        if (lane == (uint32_t)r) A.hx[f0 + r] = cz_tagged(tag, gz[r] * (cz_silu_fast(ag) * au));
    };
    // the first half of the rows while the down rows are still to be requested
#pragma unroll
    for (int r = 0; r < RW / 2; ++r) gate_up_row(r);
    __builtin_amdgcn_sched_barrier(0);
    uint4 dd[DP][RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const uint8_t *wd = L.ew + sld[i] * L.ew_stride + 2ull * I * H + jcd[i] + 16 * dj;
#pragma unroll
        for (uint32_t p = 0; p < DP; ++p) {
            const uint32_t row = r0 + DR * p + min(dq, DR - 1);
            dd[p][i] = cz_ld_nt16(wd + (uint64_t)row * I);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every weight load is in flight
#pragma unroll
    for (int r = RW / 2; r < RW; ++r) gate_up_row(r);

    // ---- dequantised down weights (e4m3 * block scale, fp8.zig:105), while
    // the XCD's gated products arrive
    float wq[DP][RW][16];
#pragma unroll
    for (uint32_t p = 0; p < DP; ++p)
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const float sc = cz_readlane(scd, p * RW + i);
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

    // ---- the XCD's gated products (each wave polls a quarter), then the down rows
    constexpr uint32_t HQ = CR / 4, NQH = (HQ + 63) / 64;
    float hq[NQH] = {};
    cz_poll_tagged<NQH>(A.hx + xcd * CR + wave * HQ, HQ, tag, hq, A.err);
#pragma unroll
    for (uint32_t q = 0; q < NQH; ++q)
        if (lane + 64 * q < HQ) s_h[wave * HQ + lane + 64 * q] = hq[q];
    __syncthreads();
    // each h slice is read once and used for every pass; four independent
    // chains (k) per pass
    float ak[DP][4];
#pragma unroll
    for (uint32_t p = 0; p < DP; ++p)
#pragma unroll
        for (int k = 0; k < 4; ++k) ak[p][k] = 0.0f;
#pragma unroll
    for (int i = 0; i < RW; ++i) {
        const float4 *hg = reinterpret_cast<const float4 *>(s_h + 128 * i + 16 * dj);
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
