// cz_grouped.h - grouped (dispatch) regime of the MoE expert path on gfx950:
// many tokens per layer (prefill, batch decode).  moe.zig:597-665
// forwardGrouped restated for MFMA:
//
//   k_route_tokens  one wave per token: top-k ids / gates (the decode routing
//                   wave), shared-expert sigmoid gate
//   k_dispatch      one workgroup: per-expert counts, offsets, a stable
//                   counting sort of the S*K slots by expert id (per-expert
//                   contiguous row lists), the M-tile table of the grouped
//                   GEMMs, and each token's slots in ascending expert id
//   k_gg<GATEUP>    grouped GEMM, one M-tile (32 rows of one expert) x 128
//                   output columns per workgroup: h = silu(X Wg^T) * (X Wu^T)
//   k_gg<DOWN>      O = h Wd^T per slot row
//   k_combine       out[t] = xres[t] + (sgate*shared[t] + sum_z g_z O[z]) with
//                   the experts in ascending id order (moe.zig:633-662)
//
// MFMA: v_mfma_f32_32x32x16_f16.  E4M3 weights convert exactly to f16;
// activations (f32) are split into f16 hi + lo (x ~= hi + lo, 22 significant
// bits), two MFMAs per k-step, f32 accumulation.  The 128x128 block scale is
// applied once per 128-wide K block to that block's f32 partial tile.
// Lane l of an MFMA: A[l%32][8(l/32)+i], B[8(l/32)+i][l%32] (i < 8),
// D[(i/4)*8 + (l/32)*4 + i%4][l%32] (i < 16).  The K order inside a 128-wide
// K block is a free permutation (the dot product is a sum): half-wave h of
// k-step s covers K offsets 64h + 8s .. 64h + 8s + 7, so each lane reads 64
// contiguous weight bytes of its row per K block.
#pragma once

#include "cz_kernels.h"

typedef _Float16 cz_half8 __attribute__((ext_vector_type(8)));
typedef float cz_float16v __attribute__((ext_vector_type(16)));

#define CZ_GG_M 32        // rows (slots) per M-tile
#define CZ_GG_N 128       // output columns per workgroup (4 waves x 32)
#define CZ_GG_KB 128      // K block (= scale block)
#define CZ_GG_LDS_ROW 136 // halves per LDS row (128 + 8 padding)

struct GroupArgs {
    LayerDev L;
    int S;
    const float *xn;           // [S][H] router input (= MoE input)
    const float *logits;       // [S][E]
    uint32_t *idx;             // [S][K]
    float *gates;              // [S][K]
    float *sgate;              // [S]
    uint32_t *idx_trace;       // nullable
    float *gates_trace;        // nullable
    // dispatch
    uint32_t *counts;          // [E]
    uint32_t *offsets;         // [E+1]
    uint32_t *sorted_slot;     // [S*K]  slot id (t*K + z) at each sorted position
    uint32_t *slot_pos;        // [S*K]  sorted position of each slot
    uint32_t *tok_order;       // [S][K] the token's slots in ascending expert id
    uint32_t *tile_expert;     // [max_tiles] expert of each M-tile
    uint32_t *tile_row0;       // [max_tiles] first sorted position of each M-tile
    uint32_t *ntiles;          // [1] M-tiles of the routed experts
    uint32_t max_tiles;
    // grouped GEMM buffers
    float *h;                  // [S*K][I] sorted rows
    float *o;                  // [S*K][H] sorted rows
    float *hs;                 // [S][SI]
    float *os;                 // [S][H]
    const float *xres;         // [S][H] nullable
    float *out;                // [S][H]
};

// ---------------------------------------------------------------------------
// routing of every token (one wave per token, 4 tokens per workgroup)
// ---------------------------------------------------------------------------
template <int M>
__global__ __launch_bounds__(256) void k_route_tokens(GroupArgs G) {
    const LayerDev &L = G.L;
    __shared__ uint32_t s_idx[4][CZ_MAX_K];
    __shared__ float s_gate[4][CZ_MAX_K];
    const uint32_t lane = cz_lane(), wave = threadIdx.x >> 6;
    const uint32_t t = blockIdx.x * 4 + wave;
    if (t >= (uint32_t)G.S) return;  // wave-uniform
    uint32_t o_pos = 0, o_id = 0;
    float o_gate = 0.0f;
    cz_route_wave_m<M>(G.logits + (uint64_t)t * L.E, L.E, L.K, L.norm_topk, s_idx[wave], s_gate[wave], o_pos, o_id,
                       o_gate);
    const uint32_t my_e = lane < L.K ? o_id : 0xffffffffu;
    if (lane < L.K) {  // lane z holds one pick; o_pos is its place in pick order
        const uint64_t o = (uint64_t)t * L.K + o_pos;
        G.idx[o] = o_id;
        G.gates[o] = o_gate;
        if (G.idx_trace) G.idx_trace[o] = o_id;
        if (G.gates_trace) G.gates_trace[o] = o_gate;
    }
    // the token's slots in ascending expert id: a pick's rank is the number
    // of the token's picks with a lower id (equal ids, possible only when NaN
    // logits leave fewer than K candidates, are ordered by lane); its slot is
    // t*K + its place in pick order
    uint32_t rank = 0;
    for (uint32_t q = 0; q < L.K; ++q) {
        const uint32_t eq = (uint32_t)__builtin_amdgcn_readlane((int)my_e, q);
        rank += (eq < my_e || (eq == my_e && q < lane)) ? 1u : 0u;
    }
    if (lane < L.K) G.tok_order[(uint64_t)t * L.K + rank] = t * L.K + o_pos;
    if (L.SI != 0) {  // shared-expert gate sigmoid(x . sh_gate) (moe.zig:475-477)
        const float *xs = G.xn + (uint64_t)t * L.H;
        float d = 0.0f;
        for (uint32_t i = lane; i < L.H; i += 64) {
            const float prod = xs[i] * L.sh_gate[i];
            d = d + prod;
        }
        d = cz_wave_sum_dpp(d);
        if (lane == 0) G.sgate[t] = cz_sigmoid(d);
    }
}

// ---------------------------------------------------------------------------
// dispatch: one workgroup of 1024 threads (16 waves) over the S*K slot ids
// (S*K <= CZ_DISPATCH_MAX, E <= CZ_MAX_E).  Counts by LDS integer atomics
// (order-independent), offsets by one prefix, then a stable placement in
// rounds of 1024 slots: inside a wave, equal ids are ranked by ballot in lane
// order; across the round's waves, per-expert running bases are prefixed in
// wave order.  Within an expert, rows keep slot order.
// ---------------------------------------------------------------------------
#define CZ_DISPATCH_MAX 8192

__global__ __launch_bounds__(1024) void k_dispatch(GroupArgs G) {
    const LayerDev &L = G.L;
    const uint32_t E = L.E, SK = (uint32_t)G.S * L.K;
    __shared__ uint16_t s_slot_e[CZ_DISPATCH_MAX];
    __shared__ uint16_t s_wcnt[16][CZ_MAX_E];  // this round's count per (wave, expert), then its base
    __shared__ uint32_t s_cnt[CZ_MAX_E];
    __shared__ uint32_t s_off[CZ_MAX_E + 1];
    __shared__ uint32_t s_run[CZ_MAX_E];       // rows placed so far per expert
    const uint32_t tid = threadIdx.x, lane = cz_lane(), wave = tid >> 6;
    for (uint32_t i = tid; i < E; i += blockDim.x) {
        s_cnt[i] = 0;
        s_run[i] = 0;
    }
    for (uint32_t i = tid; i < 16 * CZ_MAX_E; i += blockDim.x) (&s_wcnt[0][0])[i] = 0;
    for (uint32_t i = tid; i < SK; i += blockDim.x) s_slot_e[i] = (uint16_t)min(G.idx[i], E - 1);
    __syncthreads();
    for (uint32_t i = tid; i < SK; i += blockDim.x) atomicAdd(&s_cnt[s_slot_e[i]], 1u);
    __syncthreads();
    if (tid < 64) {  // one wave: exclusive prefix of counts and of M-tile counts
        uint32_t acc = 0, tacc = 0;
        for (uint32_t e0 = 0; e0 < E; e0 += 64) {
            const uint32_t e = e0 + lane;
            const uint32_t c = e < E ? s_cnt[e] : 0u;
            const uint32_t tc = (c + CZ_GG_M - 1) / CZ_GG_M;
            // inclusive scans over the 64 lanes (shuffles; tiny)
            uint32_t ic = c, it = tc;
            for (uint32_t off = 1; off < 64; off <<= 1) {
                const uint32_t a = __shfl_up(ic, off, 64), b = __shfl_up(it, off, 64);
                if (lane >= off) { ic += a; it += b; }
            }
            if (e < E) {
                s_off[e] = acc + ic - c;
                const uint32_t tile0 = tacc + it - tc;
                for (uint32_t k = 0; k < tc; ++k) {
                    const uint32_t tile = tile0 + k;
                    if (tile < G.max_tiles) {
                        G.tile_expert[tile] = e;
                        G.tile_row0[tile] = acc + ic - c + k * CZ_GG_M;
                    }
                }
            }
            acc += (uint32_t)__shfl(ic, 63, 64);
            tacc += (uint32_t)__shfl(it, 63, 64);
        }
        if (lane == 0) {
            s_off[E] = acc;
            G.ntiles[0] = min(tacc, G.max_tiles);
        }
    }
    __syncthreads();
    for (uint32_t e = tid; e <= E; e += blockDim.x) {
        G.offsets[e] = s_off[e];
        if (e < E) G.counts[e] = s_cnt[e];
    }
    for (uint32_t r0 = 0; r0 < SK; r0 += blockDim.x) {
        const uint32_t i = r0 + tid;
        const bool valid = i < SK;
        const uint32_t e = valid ? s_slot_e[i] : 0u;
        // rank among the wave's equal ids, and the wave's count per id
        uint32_t rank = 0;
        bool pending = valid;
        while (__ballot(pending)) {
            const uint64_t pm = __ballot(pending);
            const uint32_t leader = (uint32_t)__builtin_ctzll(pm);
            const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)e, leader);
            const uint64_t m = __ballot(pending && e == v);
            if (pending && e == v) {
                rank = (uint32_t)__builtin_popcountll(m & ((1ull << lane) - 1ull));
                pending = false;
            }
            if (lane == leader) s_wcnt[wave][v] = (uint16_t)__builtin_popcountll(m);
        }
        __syncthreads();
        // per expert: bases of the round's waves in wave order
        for (uint32_t x = tid; x < E; x += blockDim.x) {
            uint32_t run = s_run[x];
            for (uint32_t w = 0; w < 16; ++w) {
                const uint32_t c = s_wcnt[w][x];
                s_wcnt[w][x] = (uint16_t)run;  // this wave's base (fits: run < S*K <= 8192)
                run += c;
            }
            s_run[x] = run;
        }
        __syncthreads();
        if (valid) {
            const uint32_t pos = s_off[e] + s_wcnt[wave][e] + rank;
            G.sorted_slot[pos] = i;
            G.slot_pos[i] = pos;
        }
        __syncthreads();
        for (uint32_t x = tid; x < 16 * CZ_MAX_E; x += blockDim.x) (&s_wcnt[0][0])[x] = 0;
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
// 8 E4M3 bytes (two dwords) -> 8 f16, exact: every E4M3 value is an f16,
// and gfx950's v_cvt_scalef32_pk_f16_fp8 with scale 1.0 converts two bytes
// of a dword per instruction (word_sel picks bytes 0-1 or 2-3)
__device__ inline cz_half8 cz_fp8x8_to_f16(uint32_t w0, uint32_t w1) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w0, 1.0f, false);
    const f16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w0, 1.0f, true);
    const f16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w1, 1.0f, false);
    const f16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w1, 1.0f, true);
    cz_half8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

enum GGMode { GG_GATEUP = 0, GG_DOWN = 1 };

// One problem of the grouped GEMM (routed experts or the shared expert).
struct GGProblem {
    const uint8_t *w0;      // expert 0 (or the shared expert) first matrix: gate (GATEUP) / down
    const float *s0;        // its scales
    uint64_t w_stride;      // bytes between experts (0 for the shared expert)
    uint64_t s_stride;      // floats between experts
    uint64_t w1_off;        // GATEUP: up matrix offset from gate (bytes), scales likewise
    uint64_t s1_off;
    uint32_t N, Kd;         // output columns, reduction length (both multiples of 128)
    uint32_t nbK;           // scale blocks along K (= Kd/128)
    const float *a;         // A rows: GATEUP xn [S][H] (row = token), DOWN h [rows][Kd]
    float *c;               // C rows [rows][N]
    int routed;             // 1: tiles from the dispatch table; 0: shared (rows = tokens in order)
    uint32_t rows_total;    // shared: S
};

template <int MODE>
__global__ __launch_bounds__(256) void k_gg(GroupArgs G, GGProblem P) {
    constexpr int NMAT = MODE == GG_GATEUP ? 2 : 1;
    __shared__ _Float16 a_hi[2][CZ_GG_M * CZ_GG_LDS_ROW];
    __shared__ _Float16 a_lo[2][CZ_GG_M * CZ_GG_LDS_ROW];
    __shared__ uint32_t s_rowsrc[CZ_GG_M];  // A row index of each tile row (~0u = padding)
    __shared__ uint32_t s_rowdst[CZ_GG_M];  // C row index of each tile row

    const uint32_t lane = cz_lane(), wave = threadIdx.x >> 6, tid = threadIdx.x;
    // XCD-aware order: workgroup b runs on XCD b % 8, so M-tile mt is pinned to
    // XCD mt % 8 for all of its N-tiles and its A rows are read into one L2:
    // b = ((mt / 8) * ntn + nt) * 8 + mt % 8
    const uint32_t ntn = P.N / CZ_GG_N;
    const uint32_t grp = blockIdx.x >> 3, mt = (grp / ntn) * 8 + (blockIdx.x & 7), nt = grp % ntn;
    uint32_t e = 0, row0 = 0, rows = 0;
    if (P.routed) {
        if (mt >= G.ntiles[0]) return;  // block-uniform
        e = G.tile_expert[mt];
        row0 = G.tile_row0[mt];
        rows = min((uint32_t)CZ_GG_M, G.offsets[e + 1] - row0);
    } else {
        row0 = mt * CZ_GG_M;
        if (row0 >= P.rows_total) return;
        rows = min((uint32_t)CZ_GG_M, P.rows_total - row0);
    }
    if (tid < CZ_GG_M) {
        uint32_t src = ~0u, dst = ~0u;
        if (tid < rows) {
            const uint32_t pos = row0 + tid;
            dst = pos;
            // GATEUP routed: the slot's token row of xn; DOWN routed: the sorted h row;
            // shared: token rows in order
            src = (MODE == GG_GATEUP && P.routed) ? G.sorted_slot[pos] / G.L.K : pos;
        }
        s_rowsrc[tid] = src;
        s_rowdst[tid] = dst;
    }
    __syncthreads();

    const uint64_t sl = P.routed ? cz_slot(G.L, e) : 0;
    const uint8_t *W0 = P.w0 + sl * P.w_stride;
    const float *S0 = P.s0 + sl * P.s_stride;
    // this wave's 32 output columns, this lane's weight row n and K half
    const uint32_t n_base = nt * CZ_GG_N + wave * 32;
    const uint32_t n = n_base + (lane & 31);
    const uint32_t hk = (lane >> 5) * 64;
    const uint8_t *wrow[NMAT];
    const float *srow[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        wrow[m] = W0 + (m ? P.w1_off : 0) + (uint64_t)n * P.Kd + hk;
        srow[m] = S0 + (m ? P.s1_off : 0) + (uint64_t)(n_base / CZ_BLOCK) * P.nbK;
    }
    // A staging: thread tid loads row r = tid/8, 16 floats at column 16*(tid%8)
    const uint32_t ar = tid >> 3, ac = (tid & 7) * 16;
    const uint32_t asrc = s_rowsrc[ar];
    const float *arow = asrc != ~0u ? P.a + (uint64_t)asrc * P.Kd + ac : nullptr;

    cz_float16v acc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][i] = 0.0f;

    // K blocks kb+1 and kb+2 are in flight while kb is multiplied: weights in
    // registers (two sets), the A rows of kb+1 staged to LDS at the end of
    // iteration kb (double-buffered LDS)
    uint4 wA[NMAT][4], wB[NMAT][4];
    float4 aA[4], aB[4];
    auto load_w = [&](uint32_t kb, uint4 (&w)[NMAT][4]) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) w[m][q] = ((const uint4 *)(wrow[m] + (uint64_t)kb * CZ_GG_KB))[q];
    };
    auto load_a = [&](uint32_t kb, float4 (&a)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            a[q] = arow ? ((const float4 *)(arow + (uint64_t)kb * CZ_GG_KB))[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    // f32 -> f16 hi + lo (hi = f16(v), lo = f16(v - hi)), two 16-byte LDS
    // stores per array
    auto stage_a = [&](int buf, const float4 (&a)[4]) {
        cz_half8 hv[2], lv[2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float v[4] = {a[q].x, a[q].y, a[q].z, a[q].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const _Float16 h = (_Float16)v[j];
                hv[q >> 1][4 * (q & 1) + j] = h;
                lv[q >> 1][4 * (q & 1) + j] = (_Float16)(v[j] - (float)h);
            }
        }
        cz_half8 *hi = (cz_half8 *)(a_hi[buf] + ar * CZ_GG_LDS_ROW + ac);
        cz_half8 *lo = (cz_half8 *)(a_lo[buf] + ar * CZ_GG_LDS_ROW + ac);
        hi[0] = hv[0]; hi[1] = hv[1];
        lo[0] = lv[0]; lo[1] = lv[1];
    };

    const uint32_t nkb = P.Kd / CZ_GG_KB;  // >= 1
    load_w(0, wA);
    load_a(0, aA);
    if (nkb > 1) {
        load_w(1, wB);
        load_a(1, aB);
    }
    stage_a(0, aA);
    __syncthreads();
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        // this block's weights leave wA; wA then takes kb+2
        uint4 wcur[NMAT][4];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) wcur[m][q] = wA[m][q];
        float sc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) sc[m] = srow[m][kb];
        if (kb + 2 < nkb) {
            load_w(kb + 2, wA);
            load_a(kb + 2, aA);
        }
        cz_float16v part[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int i = 0; i < 16; ++i) part[m][i] = 0.0f;
        const _Float16 *ahi = a_hi[buf] + (lane & 31) * CZ_GG_LDS_ROW + hk;
        const _Float16 *alo = a_lo[buf] + (lane & 31) * CZ_GG_LDS_ROW + hk;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const cz_half8 xh = *(const cz_half8 *)(ahi + 8 * s);
            const cz_half8 xl = *(const cz_half8 *)(alo + 8 * s);
#pragma unroll
            for (int m = 0; m < NMAT; ++m) {
                const uint4 wv = wcur[m][s >> 1];
                const cz_half8 b = (s & 1) ? cz_fp8x8_to_f16(wv.z, wv.w) : cz_fp8x8_to_f16(wv.x, wv.y);
                part[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, b, part[m], 0, 0, 0);
                part[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, b, part[m], 0, 0, 0);
            }
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[m][i] = __builtin_fmaf(sc[m], part[m][i], acc[m][i]);
        if (kb + 1 < nkb) stage_a(buf ^ 1, aB);  // kb+1's rows (loaded an iteration ago)
        // rotate: kb+1's weights/rows move to the A set's successor
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 t = wB[m][q];
                wB[m][q] = wA[m][q];
                wA[m][q] = t;
            }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 t = aB[q];
            aB[q] = aA[q];
            aA[q] = t;
        }
        __syncthreads();
    }
    // epilogue: lane holds rows (i/4)*8 + (l/32)*4 + i%4 of column n
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t r = (i / 4) * 8 + (lane >> 5) * 4 + (i % 4);
        const uint32_t dst = s_rowdst[r];
        if (dst != ~0u) {
            float v;
            if constexpr (MODE == GG_GATEUP) v = cz_silu_fast(acc[0][i]) * acc[1][i];
            else v = acc[0][i];
            P.c[(uint64_t)dst * P.N + n] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// combine: out[t][d] = xres + ((0 + sgate*os) + g_a*O_a) + g_b*O_b ... in
// ascending expert id (moe.zig:633-662; shared first, moe.zig:614-630)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_combine(GroupArgs G) {
    const LayerDev &L = G.L;
    const uint32_t t = blockIdx.y;
    const uint32_t d = blockIdx.x * 256 + threadIdx.x;
    if (d >= L.H || t >= (uint32_t)G.S) return;
    float ys = 0.0f;
    if (L.SI != 0) ys = ys + G.sgate[t] * G.os[(uint64_t)t * L.H + d];
    for (uint32_t z = 0; z < L.K; ++z) {
        const uint32_t s = G.tok_order[(uint64_t)t * L.K + z];
        const float g = G.gates[s];
        const float v = G.o[(uint64_t)G.slot_pos[s] * L.H + d];
        ys = ys + g * v;
    }
    const uint64_t o = (uint64_t)t * L.H + d;
    G.out[o] = (G.xres ? G.xres[o] : 0.0f) + ys;
}
