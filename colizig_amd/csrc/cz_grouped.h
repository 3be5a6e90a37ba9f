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
    cz_route_wave_m<M>(G.logits + (uint64_t)t * L.E, L.E, L.K, L.norm_topk, s_idx[wave], s_gate[wave]);
    if (lane < L.K) {  // lane z reads back the entry it wrote
        const uint64_t o = (uint64_t)t * L.K + lane;
        G.idx[o] = s_idx[wave][lane];
        G.gates[o] = s_gate[wave][lane];
        if (G.idx_trace) G.idx_trace[o] = s_idx[wave][lane];
        if (G.gates_trace) G.gates_trace[o] = s_gate[wave][lane];
    }
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
// dispatch: one workgroup of 1024 threads, the S*K slot ids in LDS
// (S*K <= CZ_DISPATCH_MAX).  Stable: within an expert, rows keep slot order.
// ---------------------------------------------------------------------------
#define CZ_DISPATCH_MAX 8192

__global__ __launch_bounds__(1024) void k_dispatch(GroupArgs G) {
    const LayerDev &L = G.L;
    const uint32_t E = L.E, K = L.K, SK = (uint32_t)G.S * L.K;
    __shared__ uint32_t s_slot_e[CZ_DISPATCH_MAX];
    __shared__ uint32_t s_cnt[CZ_MAX_E];
    __shared__ uint32_t s_off[CZ_MAX_E + 1];
    __shared__ uint32_t s_tile0[CZ_MAX_E + 1];
    const uint32_t tid = threadIdx.x, lane = cz_lane(), wave = tid >> 6, nwaves = blockDim.x >> 6;
    for (uint32_t i = tid; i < E; i += blockDim.x) s_cnt[i] = 0;
    for (uint32_t i = tid; i < SK; i += blockDim.x) s_slot_e[i] = min(G.idx[i], E - 1);
    __syncthreads();
    // 1. counts (integer atomics: order-independent)
    for (uint32_t i = tid; i < SK; i += blockDim.x) atomicAdd(&s_cnt[s_slot_e[i]], 1u);
    __syncthreads();
    // 2. exclusive prefix over experts, and of their M-tile counts (one thread)
    if (tid == 0) {
        uint32_t acc = 0, tacc = 0;
        for (uint32_t e = 0; e < E; ++e) {
            s_off[e] = acc;
            s_tile0[e] = tacc;
            acc += s_cnt[e];
            tacc += (s_cnt[e] + CZ_GG_M - 1) / CZ_GG_M;
        }
        s_off[E] = acc;
        s_tile0[E] = tacc;
        G.ntiles[0] = min(tacc, G.max_tiles);
    }
    __syncthreads();
    for (uint32_t e = tid; e <= E; e += blockDim.x) {
        G.offsets[e] = s_off[e];
        if (e < E) G.counts[e] = s_cnt[e];
    }
    // 3. stable placement: wave w owns experts w, w + nwaves, ...; a ballot over
    //    each 64-slot chunk ranks equal ids in slot order
    for (uint32_t e = wave; e < E; e += nwaves) {
        if (s_cnt[e] == 0) continue;  // wave-uniform
        uint32_t base = s_off[e];
        for (uint32_t c0 = 0; c0 < SK; c0 += 64) {
            const uint32_t i = c0 + lane;
            const bool hit = i < SK && s_slot_e[i] == e;
            const uint64_t m = __ballot(hit);
            if (hit) {
                const uint32_t pos = base + (uint32_t)__builtin_popcountll(m & ((1ull << lane) - 1ull));
                G.sorted_slot[pos] = i;
                G.slot_pos[i] = pos;
            }
            base += (uint32_t)__builtin_popcountll(m);
        }
        // 4. this expert's M-tiles
        const uint32_t nt = (s_cnt[e] + CZ_GG_M - 1) / CZ_GG_M;
        for (uint32_t k = lane; k < nt; k += 64) {
            const uint32_t tile = s_tile0[e] + k;
            if (tile < G.max_tiles) {
                G.tile_expert[tile] = e;
                G.tile_row0[tile] = s_off[e] + k * CZ_GG_M;
            }
        }
    }
    // 5. each token's slots in ascending expert id (insertion sort of K)
    for (uint32_t t = tid; t < (uint32_t)G.S; t += blockDim.x) {
        uint32_t ord[CZ_MAX_K];
        for (uint32_t z = 0; z < K; ++z) {
            const uint32_t s = t * K + z, e = s_slot_e[s];
            uint32_t j = z;
            while (j > 0 && s_slot_e[ord[j - 1]] > e) { ord[j] = ord[j - 1]; --j; }
            ord[j] = s;
        }
        for (uint32_t z = 0; z < K; ++z) G.tok_order[(uint64_t)t * K + z] = ord[z];
    }
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
// 8 E4M3 bytes (two dwords) -> 8 f16, exact (every E4M3 value is an f16)
__device__ inline cz_half8 cz_fp8x8_to_f16(uint32_t w0, uint32_t w1) {
    typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
    const cz_float2 a = cz_fp8x2_lo(w0), b = cz_fp8x2_hi(w0), c = cz_fp8x2_lo(w1), d = cz_fp8x2_hi(w1);
    const fp16x2 p[4] = {__builtin_amdgcn_cvt_pkrtz(a.x, a.y), __builtin_amdgcn_cvt_pkrtz(b.x, b.y),
                         __builtin_amdgcn_cvt_pkrtz(c.x, c.y), __builtin_amdgcn_cvt_pkrtz(d.x, d.y)};
    cz_half8 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t bits = __builtin_bit_cast(uint32_t, p[q]);
        r[2 * q] = __builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
        r[2 * q + 1] = __builtin_bit_cast(_Float16, (uint16_t)(bits >> 16));
    }
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
    const uint32_t ntn = P.N / CZ_GG_N;
    const uint32_t mt = blockIdx.x / ntn, nt = blockIdx.x - mt * ntn;
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

    const uint8_t *W0 = P.w0 + (uint64_t)e * P.w_stride;
    const float *S0 = P.s0 + (uint64_t)e * P.s_stride;
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

    uint4 wreg[NMAT][4];
    float4 areg[4];
    auto load_kb = [&](uint32_t kb) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) wreg[m][q] = ((const uint4 *)(wrow[m] + (uint64_t)kb * CZ_GG_KB))[q];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            areg[q] = arow ? ((const float4 *)(arow + (uint64_t)kb * CZ_GG_KB))[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    // f32 -> f16 hi + lo (hi = f16(v), lo = f16(v - hi)), two 16-byte LDS
    // stores per array
    auto stage_a = [&](int buf) {
        cz_half8 hv[2], lv[2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float v[4] = {areg[q].x, areg[q].y, areg[q].z, areg[q].w};
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

    const uint32_t nkb = P.Kd / CZ_GG_KB;
    load_kb(0);
    stage_a(0);
    __syncthreads();
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        uint4 wcur[NMAT][4];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) wcur[m][q] = wreg[m][q];
        float sc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) sc[m] = srow[m][kb];
        if (kb + 1 < nkb) load_kb(kb + 1);  // next block in flight during this one's MFMAs
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
        if (kb + 1 < nkb) stage_a(buf ^ 1);
        __syncthreads();
    }
    // epilogue: lane holds rows (i/4)*8 + (l/32)*4 + i%4 of column n
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t r = (i / 4) * 8 + (lane >> 5) * 4 + (i % 4);
        const uint32_t dst = s_rowdst[r];
        if (dst != ~0u) {
            float v;
            if constexpr (MODE == GG_GATEUP) v = cz_silu(acc[0][i]) * acc[1][i];
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
