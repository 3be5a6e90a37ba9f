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

#include <type_traits>

typedef _Float16 cz_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 cz_half4 __attribute__((ext_vector_type(4)));
typedef float cz_float16v __attribute__((ext_vector_type(16)));

#define CZ_GG_M 32        // rows (slots) per M-tile
#define CZ_GG_KB 128      // K block (= scale block)
#define CZ_GG_WLD 144     // LDS bytes per staged weight row (128 + 16: rows r..r+7 start in distinct bank groups)

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
    _Float16 *xh, *xl;         // [S][H]    x as f16 hi + lo
    _Float16 *hh, *hl;         // [S*K][I]  h of the sorted rows as f16 hi + lo
    _Float16 *hsh, *hsl;       // [S][SI]   shared-expert h as f16 hi + lo
    float *o;                  // [S*K][H] sorted rows
    float *os;                 // [S][H]
    const float *xres;         // [S][H] nullable
    float *out;                // [S][H]
    // S = 1 routing read back by the host without a copy: the picks go to
    // host_idx (host memory), then host_seq to host_flag (system scope; a
    // null flag: a later kernel publishes it)
    uint32_t *host_idx;        // nullable
    uint32_t *host_flag;
    uint32_t host_seq;
    uint32_t sgate_ready;      // 1: the RMS rows kernel already wrote sgate
    unsigned long long *usage; // [E] routed-selection counters to bump, or null: k_route_tokens
                               // bumps one counter per pick (one atomic each, for S = 1),
                               // k_dispatch adds each expert's count of the launch (one atomic
                               // per routed expert, for S > 1: a hot expert picked by most
                               // tokens would otherwise serialise hundreds of atomics on one
                               // address); null in a routing pass whose picks another kernel
                               // routes and counts again
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
    // the token's row of x as f16 hi + lo (x ~= hi + lo), the A operand of the
    // gate/up GEMMs (callers that only route pass no split buffers): its first
    // 256*XB columns are requested before the routing and split after it
    constexpr uint32_t XB = 16;
    const bool split = G.xh && G.xl;
    const float *xrow = G.xn + (uint64_t)t * L.H;
    float4 xv[XB];
    if (split) {
#pragma unroll
        for (uint32_t q = 0; q < XB; ++q) {
            const uint32_t i = 4 * lane + 256 * q;
            xv[q] = i < L.H ? *(const float4 *)(xrow + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    uint32_t o_pos = 0, o_id = 0;
    float o_gate = 0.0f;
    cz_route_wave_m<M>(G.logits + (uint64_t)t * L.E, L.E, L.K, L.norm_topk, s_idx[wave], s_gate[wave], o_pos, o_id,
                       o_gate);
    const uint32_t my_e = lane < L.K ? o_id : 0xffffffffu;
    if (lane < L.K) {  // lane z holds one pick; o_pos is its place in pick order
        const uint64_t o = (uint64_t)t * L.K + o_pos;
        cz_bump_usage(G.usage, L.E, o_id);
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
    if (G.host_idx) {  // one token (one wave): picks to host memory, then the flag
        if (lane < L.K) G.host_idx[(uint64_t)t * L.K + o_pos] = o_id;
        __threadfence_system();
        if (lane == 0 && G.host_flag)
            __hip_atomic_store(G.host_flag, G.host_seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (split) {
        _Float16 *xh = G.xh + (uint64_t)t * L.H, *xl = G.xl + (uint64_t)t * L.H;
        for (uint32_t i0 = 0; i0 < L.H; i0 += 256 * XB) {
            if (i0 != 0) {
#pragma unroll
                for (uint32_t q = 0; q < XB; ++q) {
                    const uint32_t i = i0 + 4 * lane + 256 * q;
                    xv[q] = i < L.H ? *(const float4 *)(xrow + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
            }
#pragma unroll
            for (uint32_t q = 0; q < XB; ++q) {
                const uint32_t i = i0 + 4 * lane + 256 * q;
                if (i < L.H) {
                    const float f[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
                    cz_half4 hv, lv;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        hv[c] = (_Float16)f[c];
                        lv[c] = (_Float16)(f[c] - (float)hv[c]);
                    }
                    *(cz_half4 *)(xh + i) = hv;
                    *(cz_half4 *)(xl + i) = lv;
                }
            }
        }
    }
    if (L.SI != 0 && !G.sgate_ready) {  // shared-expert gate sigmoid(x . sh_gate) (moe.zig:475-477)
        const float d = cz_sgate_dot(G.xn + (uint64_t)t * L.H, L.sh_gate, L.H, lane);
        if (lane == 0) G.sgate[t] = cz_sigmoid(d);
    }
}

// ---------------------------------------------------------------------------
// dispatch (moe.zig:597-612: the routed rows grouped by expert): one
// workgroup of 1024 threads (16 waves) over the S*K slot ids (S*K <=
// CZ_DISPATCH_MAX, E <= CZ_MAX_E).  Each slot takes its rank among its
// expert's rows from an LDS atomic on the expert's count, the offsets come
// from one prefix of the counts, and the slot goes to offset + rank.  Rows of
// one expert come in the order the atomics were served, which is not fixed;
// no result depends on it (a row's products do not depend on the other rows
// of its M-tile, and the combine reads each slot's row through slot_pos).
// ---------------------------------------------------------------------------
#define CZ_DISPATCH_MAX 8192

__global__ __launch_bounds__(1024) void k_dispatch(GroupArgs G) {
    const LayerDev &L = G.L;
    const uint32_t E = L.E, SK = (uint32_t)G.S * L.K;
    constexpr uint32_t NQ = CZ_DISPATCH_MAX / 1024;
    __shared__ uint32_t s_cnt[CZ_MAX_E];
    __shared__ uint32_t s_off[CZ_MAX_E + 1];
    const uint32_t tid = threadIdx.x, lane = cz_lane();
    // the slots' expert ids: all of a thread's loads in flight at once
    // (indices past SK re-read slot SK - 1, unconditionally, so the loads are
    // not serialised by branches)
    uint32_t ev[NQ], rk[NQ];
#pragma unroll
    for (uint32_t q = 0; q < NQ; ++q) ev[q] = G.idx[min(tid + 1024u * q, SK - 1)];
#pragma unroll
    for (uint32_t q = 0; q < NQ; ++q) ev[q] = min(ev[q], E - 1);
    for (uint32_t i = tid; i < E; i += blockDim.x) s_cnt[i] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t q = 0; q < NQ; ++q)
        if (tid + 1024u * q < SK) rk[q] = atomicAdd(&s_cnt[ev[q]], 1u);
    __syncthreads();
    if (tid < 64) {  // one wave: exclusive prefix of counts and of M-tile counts
        uint32_t acc = 0, tacc = 0;
        for (uint32_t e0 = 0; e0 < E; e0 += 64) {
            const uint32_t e = e0 + lane;
            const uint32_t c = e < E ? s_cnt[e] : 0u;
            const uint32_t tc = (c + CZ_GG_M - 1) / CZ_GG_M;
            const uint32_t ic = cz_wave_incl_scan_u32(c), it = cz_wave_incl_scan_u32(tc);
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
            acc += (uint32_t)__builtin_amdgcn_readlane((int)ic, 63);
            tacc += (uint32_t)__builtin_amdgcn_readlane((int)it, 63);
        }
        if (lane == 0) {
            s_off[E] = acc;
            G.ntiles[0] = min(tacc, G.max_tiles);
        }
    }
    __syncthreads();
    for (uint32_t e = tid; e <= E; e += blockDim.x) {
        G.offsets[e] = s_off[e];
        if (e < E) {
            G.counts[e] = s_cnt[e];
            if (G.usage && s_cnt[e]) atomicAdd(G.usage + e, (unsigned long long)s_cnt[e]);
        }
    }
#pragma unroll
    for (uint32_t q = 0; q < NQ; ++q) {
        const uint32_t i = tid + 1024u * q;
        if (i < SK) {
            const uint32_t pos = s_off[ev[q]] + rk[q];
            G.sorted_slot[pos] = i;
            G.slot_pos[i] = pos;
        }
    }
}

// ---------------------------------------------------------------------------
// grouped GEMM
// ---------------------------------------------------------------------------
// 8 E4M3 bytes (two dwords) -> 8 f16, exact: every E4M3 value is an f16,
// and gfx950's v_cvt_scalef32_pk_f16_fp8 with scale 1.0 converts two bytes
// of a dword per instruction (word_sel picks bytes 0-1 or 2-3)
__device__ __forceinline__ cz_half8 cz_fp8x8_to_f16(uint32_t w0, uint32_t w1) {
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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A raw buffer resource over the bytes from p on (offsets below 2 GiB; gfx9
// word 3: 32-bit data format), p read from the first lane so the resource
// lives in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t cz_rsrc(const void *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return __builtin_amdgcn_make_buffer_rsrc((void *)(((uint64_t)hi << 32) | lo), (short)0, 0x7fffffff, 0x00020000);
}

// A pointer that every lane of the wave holds, read from the first lane so
// that it lives in scalar registers.
__device__ __forceinline__ const uint8_t *cz_uniform_ptr(const uint8_t *p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return (const uint8_t *)(((uint64_t)hi << 32) | lo);
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
    uint32_t N, Kd;         // output columns, reduction length (N % 256 == 0 for DOWN, Kd % 128 == 0)
    uint32_t nbK;           // scale blocks along K (= Kd/128)
    const _Float16 *a_hi;   // A rows as f16 hi/lo: GATEUP x [S][H] (row = token), DOWN h [rows][Kd]
    const _Float16 *a_lo;
    _Float16 *c_hi;         // GATEUP: h rows as f16 hi/lo [rows][N]
    _Float16 *c_lo;
    float *c;               // DOWN: O rows [rows][N]
    int routed;             // 1: tiles from the dispatch table; 0: shared (rows = tokens in order)
    uint32_t rows_total;    // shared: S
    // FP8-MFMA form (k_gg8): A rows as three E4M3 terms with E8M0 exponents
    // per 32 columns (cz_q3_scale); GATEUP writes h in the same form, the
    // A rows of the down GEMM
    const uint8_t *aq;      // [3][rows][Kd] (term planes aq_plane bytes apart)
    const uint8_t *ae;      // [3][rows][Kd/32] (planes ae_plane bytes apart)
    uint64_t aq_plane, ae_plane;
    uint8_t *cq;            // GATEUP: h as [3][rows][N] terms (planes cq_plane bytes apart)
    uint8_t *ce;            // GATEUP: its exponents [3][rows][N/32] (planes ce_plane bytes apart)
    uint64_t cq_plane, ce_plane;
};

// Output columns of one workgroup: 4 waves x 2 subtiles of 32 columns.  A
// GATEUP wave's two subtiles are the gate and up columns of the same 32
// outputs; a DOWN wave's are 64 adjacent columns.
template <int MODE>
__host__ __device__ constexpr uint32_t cz_gg_cols() { return MODE == GG_GATEUP ? 128u : 256u; }

// A tile of one K block in LDS: CZ_GG_M rows of 128 f16 (256 B = 16 chunks of
// 16 B); chunk c of row r is stored at chunk c ^ (r & 15), so the 32 rows that
// one MFMA operand read touches at one chunk lie in distinct banks.
__device__ __forceinline__ uint32_t cz_gg_lds_off(uint32_t r, uint32_t c) { return r * 256u + ((c ^ (r & 15u)) << 4); }

// A staging: the K block's 32 rows x 16 chunks of 16 B per array; thread t
// moves chunks t and t + 256 (row j/16, logical chunk j%16) of each of hi and
// lo, so one wave instruction reads 4 whole 256-byte row segments.  The loads
// go into registers and are stored to LDS after the current block's reads.
// off[i] is the thread's byte offset of chunk t + 256i in the A arrays for K
// block 0 (padding rows read row 0 of the problem; their results are not
// stored).
struct CzA4 {
    uint4 h0, h1, l0, l1;
};
__device__ __forceinline__ CzA4 cz_gg_load_a(const _Float16 *__restrict__ ahi, const _Float16 *__restrict__ alo,
                                             const uint32_t (&off)[2], uint32_t kb) {
    const uint64_t o = (uint64_t)kb * (CZ_GG_KB * 2u);
    const uint8_t *bh = (const uint8_t *)ahi + o, *bl = (const uint8_t *)alo + o;
    return CzA4{*(const uint4 *)(bh + off[0]), *(const uint4 *)(bh + off[1]), *(const uint4 *)(bl + off[0]),
                *(const uint4 *)(bl + off[1])};
}
__device__ __forceinline__ void cz_gg_store_a(uint8_t *lds, uint32_t tid, const CzA4 &r) {
    const uint32_t j0 = tid, j1 = tid + 256u;
    const uint32_t o0 = cz_gg_lds_off(j0 >> 4, j0 & 15u), o1 = cz_gg_lds_off(j1 >> 4, j1 & 15u);
    *(uint4 *)(lds + o0) = r.h0;
    *(uint4 *)(lds + o1) = r.h1;
    *(uint4 *)(lds + CZ_GG_M * 256 + o0) = r.l0;
    *(uint4 *)(lds + CZ_GG_M * 256 + o1) = r.l1;
}

// One K block of a wave's 32 x (2 x 32) tile: 8 k-steps x 2 subtiles x (hi,
// lo) MFMAs accumulated straight into acc, which holds the sum so far in
// units of this block's scale.  Lane l's weights w[m][q] are bytes [64(l/32) +
// 16q, +16) of its column's row in this K block; k-step s uses bytes
// 8s..8s+7 of that half, so the A operand of row l%32 is logical chunk 8(l/32)
// + s.  Step s+1's operands are fetched while step s multiplies.
__device__ __forceinline__ void cz_gg_block(const uint8_t *lds_hi, const uint8_t *lds_lo, const uint4 (&w)[2][4],
                                   cz_float16v (&acc)[2], uint32_t lane) {
    const uint32_t rl = lane & 31u, ch = (lane >> 5) * 8u;
    cz_half8 b[2][2], xh[2], xl[2];
    auto fetch = [&](int s, int u) {
        const uint32_t o = cz_gg_lds_off(rl, ch + s);
        xh[u] = *(const cz_half8 *)(lds_hi + o);
        xl[u] = *(const cz_half8 *)(lds_lo + o);
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const uint4 wv = w[m][s >> 1];
            b[u][m] = (s & 1) ? cz_fp8x8_to_f16(wv.z, wv.w) : cz_fp8x8_to_f16(wv.x, wv.y);
        }
    };
    fetch(0, 0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int u = s & 1;
        if (s < 7) fetch(s + 1, u ^ 1);
#pragma unroll
        for (int m = 0; m < 2; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[u], b[u][m], acc[m], 0, 0, 0);
#pragma unroll
        for (int m = 0; m < 2; ++m) acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl[u], b[u][m], acc[m], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Block scale of subtile m at K block kb, folded into acc: acc holds
// sum_{j < kb} s_j P_j / cur; before block kb's products are added it is
// multiplied by cur / s_kb, and at the end by the last scale, so the result is
// sum_j s_j P_j with one extra rounding per block.  A zero scale makes the
// block contribute 0: its weight bytes are cleared (E4M3 0x00 = +0) and cur is
// kept.  sc and cur are wave-uniform.
__device__ __forceinline__ void cz_gg_rescale(float sc, float &cur, cz_float16v &acc, uint4 (&w)[4]) {
    const bool zero = sc == 0.0f;
    const float r = (zero || cur == 0.0f) ? 1.0f : cur / sc;
    cur = zero ? cur : sc;
    const uint32_t keep = zero ? 0u : ~0u;
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = make_uint4(w[q].x & keep, w[q].y & keep, w[q].z & keep, w[q].w & keep);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= r;
}

// Grouped GEMM: one M-tile (32 rows of one expert) x cz_gg_cols() output
// columns per workgroup.  Work item t of the problem's T = tiles x column
// tiles is mt = t / ntn, nt = t % ntn (an M-tile's column tiles are
// consecutive); workgroup b runs on XCD b % 8 and takes item (b % 8) * ceil(T
// / 8) + b / 8, so each XCD walks a contiguous range of items and an M-tile's
// A rows are reused from its L2.  The next K block's A rows (f16 hi/lo, split
// once by their producer) and weights are loaded into registers while this
// block is multiplied, then stored to LDS: A to the workgroup's tile, each
// wave's weights to its own stage.  Three workgroups per CU (168 VGPRs,
// 52 KiB of LDS each) hide the latency.
// MFMA-layout reads of a wave's staged weights: lane L reads the 64 bytes
// 64(L/32) .. +63 of row 32m + L%32 (rows CZ_GG_WLD bytes apart, so the 8
// rows one read phase touches start in distinct bank groups).
__device__ __forceinline__ void cz_gg_read_w(const uint8_t *lw, uint32_t lane, uint4 (&w)[2][4]) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t R = 32u * m + (lane & 31u);
#pragma unroll
        for (int q = 0; q < 4; ++q) w[m][q] = *(const uint4 *)(lw + R * CZ_GG_WLD + 64u * (lane >> 5) + 16u * q);
    }
}

// Work items: the shared expert's (PS, when PS.N != 0) take blocks 0 .. ns-1,
// so its long items start first and run beside the routed ones; the routed
// items (PR) take the blocks from ns rounded up to 8, each XCD walking a
// contiguous range of them.
template <int MODE>
__global__ __launch_bounds__(256, 3) void k_gg(GroupArgs G, GGProblem PR, GGProblem PS) {
    constexpr uint32_t NCOL = cz_gg_cols<MODE>();
    const uint32_t ns = PS.N ? (PS.rows_total + CZ_GG_M - 1) / CZ_GG_M * (PS.N / NCOL) : 0u;
    const uint32_t ns8 = (ns + 7u) & ~7u;
    const bool sh = blockIdx.x < ns8;
    if (sh && blockIdx.x >= ns) return;  // block-uniform
    const GGProblem P = sh ? PS : PR;
    // the A tile of the current K block (hi at +0, lo at +CZ_GG_M*256)
    __shared__ __align__(16) uint8_t lds0[2 * CZ_GG_M * 256];
    // per wave: its 64 weight rows x 128 bytes of the current K block
    __shared__ __align__(16) uint8_t ldsw[4][64 * CZ_GG_WLD];
    __shared__ uint32_t s_rowsrc[CZ_GG_M];  // A row of each tile row (padding: row 0 of the problem)
    __shared__ uint32_t s_rowdst[CZ_GG_M];  // C row of each tile row (~0u = padding)

    const uint32_t lane = cz_lane(), tid = threadIdx.x;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform
    const uint32_t ntn = P.N / NCOL;
    uint32_t t = blockIdx.x;
    if (!sh) {
        const uint32_t b = blockIdx.x - ns8;
        const uint32_t mtiles = P.routed ? G.ntiles[0] : (P.rows_total + CZ_GG_M - 1) / CZ_GG_M;
        const uint32_t T = mtiles * ntn, per = (T + 7) / 8;
        const uint32_t j = b >> 3;
        t = (b & 7) * per + j;
        if (j >= per || t >= T) return;  // block-uniform
    }
    const uint32_t mt = t / ntn, nt = t - mt * ntn;
    uint32_t e = 0, row0, rows;
    if (P.routed) {
        e = G.tile_expert[mt];
        row0 = G.tile_row0[mt];
        rows = min((uint32_t)CZ_GG_M, G.offsets[e + 1] - row0);
    } else {
        row0 = mt * CZ_GG_M;
        rows = min((uint32_t)CZ_GG_M, P.rows_total - row0);
    }
    if (tid < CZ_GG_M) {
        const uint32_t pos = row0 + min(tid, rows - 1);
        // GATEUP routed: the slot's token row of x; DOWN routed: the sorted h
        // row; shared: token rows in order
        s_rowsrc[tid] = (MODE == GG_GATEUP && P.routed) ? G.sorted_slot[pos] / G.L.K : pos;
        s_rowdst[tid] = tid < rows ? row0 + tid : ~0u;
    }
    __syncthreads();
    // this thread's A chunks j = tid, tid + 256: row j/16, logical chunk j%16
    uint32_t aoff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t j = tid + 256u * i;
        aoff[i] = (s_rowsrc[j >> 4] * P.Kd + (j & 15u) * 8u) * 2u;
    }

    const uint64_t sl = P.routed ? cz_slot(G.L, e) : 0;
    const uint8_t *W0 = P.w0 + sl * P.w_stride;
    const float *S0 = P.s0 + sl * P.s_stride;
    // subtile m of this wave: its 32 columns (weight rows)
    const uint8_t *wbase[2];
    const float *srow[2];
    uint32_t ncol[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t nb = MODE == GG_GATEUP ? nt * NCOL + wave * 32u : nt * NCOL + wave * 64u + 32u * m;
        ncol[m] = nb + (lane & 31u);
        const uint64_t moff = (MODE == GG_GATEUP && m) ? P.w1_off : 0;
        const uint64_t soff = (MODE == GG_GATEUP && m) ? P.s1_off : 0;
        wbase[m] = W0 + moff + (uint64_t)nb * P.Kd;                 // wave-uniform
        srow[m] = S0 + soff + (uint64_t)(nb / CZ_BLOCK) * P.nbK;
    }
    // Weights of a K block: the wave's 64 rows (row R: subtile R/32, column
    // R%32) x 128 bytes.  Load p reads rows 8p .. 8p+7 whole (lane l: row 8p +
    // l/8, 16-byte chunk l%8), so each instruction covers 8 full 128-byte
    // lines.  In the wave's LDS buffer chunk c of row R sits at chunk c ^ (R %
    // 8): the MFMA-layout reads (lane L: row 32m + L%32, chunks 4(L/32) .. +3)
    // of 8 consecutive lanes then fall in distinct banks.
    uint8_t *lw = ldsw[wave];
    const uint32_t wl_off = (lane >> 3) * P.Kd + (lane & 7u) * 16u;                   // global, per lane
    const uint32_t wl_lds = (lane >> 3) * CZ_GG_WLD + (lane & 7u) * 16u;  // LDS, + p*8 rows


    cz_float16v acc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][i] = 0.0f;
    float cur[2] = {0.0f, 0.0f};

    const uint32_t nkb = P.Kd / CZ_GG_KB;  // >= 1
    uint4 w[2][4];
    // the 8 weight loads of a K block: lane base (subtile p/4) + uniform row
    // offset 8(p%4) rows + K offset.  One register set (a) of a block's A
    // chunks and weights: block kb+1 is in flight while block kb multiplies.
    const uint8_t *gl0 = wbase[0] + wl_off, *gl1 = wbase[1] + wl_off;
    const uint64_t r8 = 8ull * P.Kd;
    uint4 a0, a1, a2, a3, a4, a5, a6, a7;
    CzA4 an_a;
#define CZ_GG_LOAD(X, kb_)                                                      \
    {                                                                           \
        const uint32_t kc_ = (kb_);                                             \
        an_##X = cz_gg_load_a(P.a_hi, P.a_lo, aoff, kc_);                       \
        const uint64_t ko_ = (uint64_t)kc_ * CZ_GG_KB;                          \
        X##0 = *(const uint4 *)(gl0 + ko_);                                     \
        X##1 = *(const uint4 *)(gl0 + r8 + ko_);                                \
        X##2 = *(const uint4 *)(gl0 + 2 * r8 + ko_);                            \
        X##3 = *(const uint4 *)(gl0 + 3 * r8 + ko_);                            \
        X##4 = *(const uint4 *)(gl1 + ko_);                                     \
        X##5 = *(const uint4 *)(gl1 + r8 + ko_);                                \
        X##6 = *(const uint4 *)(gl1 + 2 * r8 + ko_);                            \
        X##7 = *(const uint4 *)(gl1 + 3 * r8 + ko_);                            \
    }
#define CZ_GG_STORE(X, abuf_)                                                   \
    {                                                                           \
        cz_gg_store_a((abuf_), tid, an_##X);                                    \
        uint8_t *d_ = lw + wl_lds;                                              \
        *(uint4 *)(d_) = X##0;                                                  \
        *(uint4 *)(d_ + 1 * 8 * CZ_GG_WLD) = X##1;                               \
        *(uint4 *)(d_ + 2 * 8 * CZ_GG_WLD) = X##2;                               \
        *(uint4 *)(d_ + 3 * 8 * CZ_GG_WLD) = X##3;                               \
        *(uint4 *)(d_ + 4 * 8 * CZ_GG_WLD) = X##4;                               \
        *(uint4 *)(d_ + 5 * 8 * CZ_GG_WLD) = X##5;                               \
        *(uint4 *)(d_ + 6 * 8 * CZ_GG_WLD) = X##6;                               \
        *(uint4 *)(d_ + 7 * 8 * CZ_GG_WLD) = X##7;                               \
    }
    // one K block: multiply block kb (A from LDS, the wave's weights from its
    // LDS stage), then, once every wave is done with the A tile, move block
    // kb+1 (loaded during this block) into LDS and request block kb+2 (past
    // the end the last block is requested again, never stored)
    CZ_GG_LOAD(a, 0)
    CZ_GG_STORE(a, lds0)  // the wave's own weight buffer: its DS operations stay in program order
    CZ_GG_LOAD(a, min(1u, nkb - 1))
    __syncthreads();
    for (uint32_t kb = 0; kb < nkb; ++kb) {
        const float s0_ = cz_const_f32(srow[0] + kb), s1_ = cz_const_f32(srow[1] + kb);
        cz_gg_read_w(lw, lane, w);
        cz_gg_rescale(s0_, cur[0], acc[0], w[0]);
        cz_gg_rescale(s1_, cur[1], acc[1], w[1]);
        cz_gg_block(lds0, lds0 + CZ_GG_M * 256, w, acc, lane);
        if (kb + 1 < nkb) {  // block-uniform
            __syncthreads();
            CZ_GG_STORE(a, lds0)
            CZ_GG_LOAD(a, min(kb + 2, nkb - 1))
            __syncthreads();
        }
    }
#undef CZ_GG_LOAD
#undef CZ_GG_STORE
    // epilogue: lane holds rows (i/4)*8 + (l/32)*4 + i%4 of its columns
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t r = (i / 4) * 8u + (lane >> 5) * 4u + (i % 4);
        const uint32_t dst = s_rowdst[r];
        if (dst == ~0u) continue;
        if constexpr (MODE == GG_GATEUP) {
            const float v = cz_silu_fast(acc[0][i] * cur[0]) * (acc[1][i] * cur[1]);
            const _Float16 hi = (_Float16)v;
            const uint64_t o = (uint64_t)dst * P.N + ncol[0];
            P.c_hi[o] = hi;
            P.c_lo[o] = (_Float16)(v - (float)hi);
        } else {
#pragma unroll
            for (int m = 0; m < 2; ++m) P.c[(uint64_t)dst * P.N + ncol[m]] = acc[m][i] * cur[m];
        }
    }
}

// ---------------------------------------------------------------------------
// FP8-MFMA grouped GEMM (the prefill's alternative to k_gg): the E4M3 weights
// go straight into v_mfma_scale_f32_32x32x64_f8f6f4 as the B operand; the A
// rows (x for gate/up, h for down) come as three E4M3 terms, each with an
// E8M0 exponent per 32 columns (x ~= sum_t 2^(e_t - 127) q_t, about 12
// significant bits), applied by the instruction itself.  Lane layout of one
// 32 x 32 x 64 product (checked on the device): lane l gives row (or
// column) l % 32; its bytes 0-15 are K positions 16 (l/32) + 0..15 of the
// first 32-column group, bytes 16-31 positions 32 + 16 (l/32) + 0..15 of the
// second; the exponent of row m, group b comes from lane m + 32 b.
// ---------------------------------------------------------------------------

// Rows of K columns (K % 32 == 0) to three E4M3 terms (cz_q3_group4): each
// 32-column group is 8 consecutive lanes with one float4 each, so a wave's
// loads and term stores are contiguous.  For inputs no producing kernel
// splits (x without the RMS rows kernel).
__global__ __launch_bounds__(256) void k_quant3(const float *__restrict__ src, uint32_t rows, uint32_t K,
                                               uint8_t *__restrict__ q, uint64_t q_plane, uint8_t *__restrict__ e,
                                               uint64_t e_plane) {
    const uint64_t g4 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;  // float4 index
    // whole 8-lane groups leave together (rows * K / 4 is a multiple of 8)
    if (g4 >= (uint64_t)rows * K / 4) return;
    const float4 v = reinterpret_cast<const float4 *>(src)[g4];
    float r[4] = {v.x, v.y, v.z, v.w};
    const uint64_t el = 4 * g4;  // first element: row el / K, column el % K
    cz_q3_group4(r, q + el, q_plane, e + el / 32, e_plane, (g4 & 7u) == 0, true);
}

typedef int cz_i8x32 __attribute__((ext_vector_type(8)));

// A tile of one K block in LDS for k_gg8: 3 term planes x CZ_GG_M rows of 128
// bytes (8 chunks of 16 B) CZ_GG8_ALD bytes apart, then the exponents: 3
// planes x CZ_GG_M rows x 4 bytes.
#define CZ_GG8_ALD 144  // LDS bytes per A row (128 + 16: the rows one read phase touches start in distinct bank groups)
#define CZ_GG8_APLANE (CZ_GG_M * CZ_GG8_ALD)
#define CZ_GG8_EOFF (3 * CZ_GG8_APLANE)
#define CZ_GG8_STAGE (CZ_GG8_EOFF + 3 * CZ_GG_M * 4)
#define CZ_GG8_HT 36  // floats per row of a wave's h tile in its weight buffer (144 B: float4-aligned)
static_assert(32 * CZ_GG8_HT * 4 <= 64 * CZ_GG_WLD, "a wave's h tile fits in its weight buffer");
__device__ __forceinline__ uint32_t cz_gg8_off(uint32_t r, uint32_t c) { return r * CZ_GG8_ALD + (c << 4); }

// Grouped GEMM on FP8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4): one M-tile
// (32 rows of one expert) x cz_gg_cols() output columns per workgroup, the
// work items and their XCD mapping as in k_gg.  A K block (128 columns) is
// the A tile's three E4M3 term planes with their E8M0 exponents (shared by
// the four waves, in LDS) and each wave's 64 weight rows (its own LDS
// buffer).  Loads run two K blocks ahead in two register sets, written to
// LDS after the block before them is multiplied; one barrier per block.
// Two workgroups per CU.
template <int MODE>
__global__ __launch_bounds__(256, 2) void k_gg8(GroupArgs G, GGProblem PR, GGProblem PS) {
    constexpr uint32_t NCOL = cz_gg_cols<MODE>();
    const uint32_t ns = PS.N ? (PS.rows_total + CZ_GG_M - 1) / CZ_GG_M * (PS.N / NCOL) : 0u;
    const uint32_t ns8 = (ns + 7u) & ~7u;
    const bool sh = blockIdx.x < ns8;
    if (sh && blockIdx.x >= ns) return;  // block-uniform
    const GGProblem P = sh ? PS : PR;
    __shared__ __align__(16) uint8_t lds0[2][CZ_GG8_STAGE];
    __shared__ uint32_t s_rowsrc[CZ_GG_M];
    __shared__ uint32_t s_rowdst[CZ_GG_M];

    const uint32_t lane = cz_lane(), tid = threadIdx.x;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t ntn = P.N / NCOL;
    uint32_t t = blockIdx.x;
    if (!sh) {
        const uint32_t b = blockIdx.x - ns8;
        const uint32_t mtiles = P.routed ? G.ntiles[0] : (P.rows_total + CZ_GG_M - 1) / CZ_GG_M;
        const uint32_t T = mtiles * ntn, per = (T + 7) / 8;
        const uint32_t j = b >> 3;
        t = (b & 7) * per + j;
        if (j >= per || t >= T) return;  // block-uniform
    }
    const uint32_t mt = t / ntn, nt = t - mt * ntn;
    uint32_t e = 0, row0, rows;
    if (P.routed) {
        e = G.tile_expert[mt];
        row0 = G.tile_row0[mt];
        rows = min((uint32_t)CZ_GG_M, G.offsets[e + 1] - row0);
    } else {
        row0 = mt * CZ_GG_M;
        rows = min((uint32_t)CZ_GG_M, P.rows_total - row0);
    }
    if (tid < CZ_GG_M) {
        const uint32_t pos = row0 + min(tid, rows - 1);
        s_rowsrc[tid] = (MODE == GG_GATEUP && P.routed) ? G.sorted_slot[pos] / G.L.K : pos;
        s_rowdst[tid] = tid < rows ? row0 + tid : ~0u;
    }
    __syncthreads();
    // A staging: thread t moves chunk t%8 of row t/8 of each term plane;
    // threads < 96 move one 4-byte exponent word (plane t/32, row t%32)
    const uint32_t ar = tid >> 3, ac = tid & 7u;
    const uint32_t a_src = s_rowsrc[ar] * P.Kd + ac * 16u;  // < 4 GiB: rows x Kd of one term plane
    const uint32_t a_dst = cz_gg8_off(ar, ac);
    const uint32_t nbe = P.Kd / 32u;
    const uint32_t ep = min(tid >> 5, 2u), er = tid & 31u;
    const uint32_t e_src = ep * (uint32_t)P.ae_plane + s_rowsrc[min(er, (uint32_t)CZ_GG_M - 1)] * nbe;

    const uint64_t sl = P.routed ? cz_slot(G.L, e) : 0;
    const uint8_t *W0 = P.w0 + sl * P.w_stride;
    const float *S0 = P.s0 + sl * P.s_stride;
    const uint8_t *wbase[2];
    const float *srow[2];
    uint32_t ncol[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        const uint32_t nb = MODE == GG_GATEUP ? nt * NCOL + wave * 32u : nt * NCOL + wave * 64u + 32u * m;
        ncol[m] = nb + (lane & 31u);
        const uint64_t moff = (MODE == GG_GATEUP && m) ? P.w1_off : 0;
        const uint64_t soff = (MODE == GG_GATEUP && m) ? P.s1_off : 0;
        wbase[m] = W0 + moff + (uint64_t)nb * P.Kd;
        srow[m] = S0 + soff + (uint64_t)(nb / CZ_BLOCK) * P.nbK;
    }
    // Weights: each wave stages its own 64 rows (32 per subtile) of a K block
    // in its LDS buffer (rows CZ_GG_WLD bytes apart); lane l loads 16 bytes
    // (l % 8) of rows l / 8 + 8 i, so one wave instruction reads 8 whole
    // 128-byte row segments.  Every load is a buffer load: a wave-uniform
    // resource (the block of weight rows, a term plane), a 32-bit lane
    // offset that does not change along K, and the K block's offset (plus
    // 8 i rows) as the scalar offset.
    const uint32_t rl = lane & 31u, hh = lane >> 5;
    __shared__ __align__(16) uint8_t ldsw[4][64 * CZ_GG_WLD];
    uint8_t *lw = ldsw[wave];
    const __amdgpu_buffer_rsrc_t rw0 = cz_rsrc(wbase[0]), rw1 = cz_rsrc(wbase[1]);
    const uint32_t w_lane = (lane >> 3) * P.Kd + (lane & 7u) * 16u;
    const uint32_t wl_lds = (lane >> 3) * CZ_GG_WLD + (lane & 7u) * 16u;
    const int r8 = (int)(8u * P.Kd);

    cz_float16v acc[2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][i] = 0.0f;
    float cur[2] = {0.0f, 0.0f};
    const uint32_t nkb = P.Kd / CZ_GG_KB;
    // Two K blocks ahead: while block kb is multiplied (A from LDS stage
    // kb % 2, weights from the wave's LDS buffer), the A rows and weights of
    // blocks kb + 1 and kb + 2 are in flight into register sets (kb + 1) % 2
    // and kb % 2.  After block kb's products, block kb + 1 goes from its
    // registers to LDS.  One barrier per K block.
    struct WSet {
        u32x4 v[8];
    };
    struct ASet {
        u32x4 q[3];
        uint32_t ev;
    };
    const __amdgpu_buffer_rsrc_t ra0 = cz_rsrc(P.aq), ra1 = cz_rsrc(P.aq + P.aq_plane),
                                 ra2 = cz_rsrc(P.aq + 2 * P.aq_plane), re0 = cz_rsrc(P.ae);
    WSet w0, w1;
    ASet a0, a1;
    // the register sets by compile-time index (distinct variables, so they stay in registers)
    auto wset = [&](auto I) __attribute__((always_inline)) -> WSet & {
        if constexpr (decltype(I)::value == 0) return w0;
        else return w1;
    };
    auto aset = [&](auto I) __attribute__((always_inline)) -> ASet & {
        if constexpr (decltype(I)::value == 0) return a0;
        else return a1;
    };
    auto load = [&](uint32_t kb, ASet &as, WSet &ws) __attribute__((always_inline)) {
        const int ko = (int)(kb * CZ_GG_KB);
        as.q[0] = __builtin_amdgcn_raw_buffer_load_b128(ra0, a_src, ko, 0);
        as.q[1] = __builtin_amdgcn_raw_buffer_load_b128(ra1, a_src, ko, 0);
        as.q[2] = __builtin_amdgcn_raw_buffer_load_b128(ra2, a_src, ko, 0);
        as.ev = __builtin_amdgcn_raw_buffer_load_b32(re0, e_src, (int)(kb * 4u), 0);  // threads >= 96: a copy, never stored
        u32x4 *w = ws.v;
        w[0] = __builtin_amdgcn_raw_buffer_load_b128(rw0, w_lane, ko, 0);
        w[1] = __builtin_amdgcn_raw_buffer_load_b128(rw0, w_lane, ko + r8, 0);
        w[2] = __builtin_amdgcn_raw_buffer_load_b128(rw0, w_lane, ko + 2 * r8, 0);
        w[3] = __builtin_amdgcn_raw_buffer_load_b128(rw0, w_lane, ko + 3 * r8, 0);
        w[4] = __builtin_amdgcn_raw_buffer_load_b128(rw1, w_lane, ko, 0);
        w[5] = __builtin_amdgcn_raw_buffer_load_b128(rw1, w_lane, ko + r8, 0);
        w[6] = __builtin_amdgcn_raw_buffer_load_b128(rw1, w_lane, ko + 2 * r8, 0);
        w[7] = __builtin_amdgcn_raw_buffer_load_b128(rw1, w_lane, ko + 3 * r8, 0);
    };
    // A rows to an LDS stage, the wave's weights to its buffer (the wave's
    // DS operations stay in program order: its reads of the previous block
    // are done before these writes)
    auto store = [&](uint8_t *st, const ASet &as, const WSet &ws) __attribute__((always_inline)) {
        *(u32x4 *)(st + a_dst) = as.q[0];
        *(u32x4 *)(st + CZ_GG8_APLANE + a_dst) = as.q[1];
        *(u32x4 *)(st + 2 * CZ_GG8_APLANE + a_dst) = as.q[2];
        if (tid < 96) *(uint32_t *)(st + CZ_GG8_EOFF + 4u * tid) = as.ev;
        uint8_t *d = lw + wl_lds;
#pragma unroll
        for (int p = 0; p < 8; ++p) *(u32x4 *)(d + p * 8 * CZ_GG_WLD) = ws.v[p];
    };
    // block scales folded into acc as in k_gg (cz_gg_rescale): before block
    // kb's products acc is rescaled by cur / s_kb, and a zero-scale block's
    // weights are cleared.  The factors of block kb + 1 are worked out while
    // block kb's MFMAs run.
    float rr[2];
    uint32_t keep[2];
    auto scales = [&](uint32_t kb) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const float sc = cz_const_f32(srow[m] + kb);
            const bool zero = sc == 0.0f;
            rr[m] = (zero || cur[m] == 0.0f) ? 1.0f : cur[m] / sc;
            cur[m] = zero ? cur[m] : sc;
            keep[m] = zero ? 0u : ~0u;
        }
    };
    auto block = [&](uint32_t kb, const uint8_t *st) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[m][i] *= rr[m];
        const uint32_t kp[2] = {keep[0], keep[1]};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            // the wave's weights in MFMA layout: subtile m, K half kk: row 32m
            // + lane%32, bytes 64kk + 16(l/32) and 64kk + 32 + 16(l/32)
            cz_i8x32 bm[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const uint8_t *rowp = lw + (32u * m + rl) * CZ_GG_WLD + 64u * kk + 16u * hh;
                const uint4 lo = *(const uint4 *)rowp, hi = *(const uint4 *)(rowp + 32u);
                const uint32_t k_ = kp[m];
                bm[m] = cz_i8x32{(int)(lo.x & k_), (int)(lo.y & k_), (int)(lo.z & k_), (int)(lo.w & k_),
                                 (int)(hi.x & k_), (int)(hi.y & k_), (int)(hi.z & k_), (int)(hi.w & k_)};
            }
#pragma unroll
            for (int tt = 0; tt < 3; ++tt) {
                const uint8_t *pl = st + tt * CZ_GG8_APLANE;
                const uint4 lo = *(const uint4 *)(pl + cz_gg8_off(rl, 4u * kk + hh));
                const uint4 hi = *(const uint4 *)(pl + cz_gg8_off(rl, 4u * kk + 2u + hh));
                const cz_i8x32 am = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z,
                                     (int)hi.w};
                // exponent of row lane%32, group 2 kk + lane/32 of this K block
                const int sa = (int)st[CZ_GG8_EOFF + (tt * CZ_GG_M + rl) * 4u + 2u * kk + hh];
#pragma unroll
                for (int m = 0; m < 2; ++m)
                    acc[m] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(am, bm[m], acc[m], 0, 0, 0, sa, 0, 127);
            }
            // the K half's products stay here: without a use, the compiler
            // sinks pure MFMAs past the next block's loads and barrier
            asm volatile("" : "+v"(acc[0]), "+v"(acc[1]));
            if (kk == 0 && kb + 1 < nkb) scales(kb + 1);  // beside the second half's MFMAs
        }
    };
    // one K block; S = kb % 2 names the register sets and the A stage at
    // compile time.  Every step issues the loads of block kb + 2 (in the
    // last two steps: the last block again, never stored), so every path
    // through the loop issues the same loads and the waits the compiler
    // places count exactly the loads issued after the ones they wait for.
    auto step = [&](uint32_t kb, auto Sc, auto CLc) __attribute__((always_inline)) {
        constexpr int S = decltype(Sc)::value;
        using Cur = std::integral_constant<int, S>;
        using Nxt = std::integral_constant<int, 1 - S>;
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();  // stage S holds A(kb); every wave is done with stage 1 - S
        load(decltype(CLc)::value ? min(kb + 2, nkb - 1) : kb + 2, aset(Cur{}), wset(Cur{}));
        block(kb, lds0[S]);
        if (kb + 1 < nkb) store(lds0[1 - S], aset(Nxt{}), wset(Nxt{}));
        __builtin_amdgcn_sched_barrier(0);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using IN = std::integral_constant<bool, false>;  // block kb + 2 exists
    using CL = std::integral_constant<bool, true>;   // clamp to the last block
    load(0, a0, w0);
    load(min(1u, nkb - 1), a1, w1);
    store(lds0[0], a0, w0);
    scales(0);
    uint32_t kb = 0;
    for (; kb + 4 <= nkb; kb += 2) {  // every load of these two steps is in range
        step(kb, I0{}, IN{});
        step(kb + 1, I1{}, IN{});
    }
    // the last 1 .. 3 blocks; each step is reached only through the one before
    step(kb, I0{}, CL{});
    if (kb + 1 < nkb) {
        step(kb + 1, I1{}, CL{});
        if (kb + 2 < nkb) step(kb + 2, I0{}, CL{});
    }
    if constexpr (MODE == GG_GATEUP) {
        // h = silu(g) * u of the wave's 32 rows x 32 columns (one 32-column
        // group) goes through the wave's own weight stage (its DS operations
        // stay in program order, so no barrier) to k_quant3's layout, 8 lanes
        // per row with four columns each, and leaves as the three E4M3 terms
        // of the down GEMM's A rows: the bytes k_quant3 makes of the f32 rows
        float *ht = reinterpret_cast<float *>(lw);  // [32][CZ_GG8_HT], 4.5 KB of the wave's 9 KB buffer
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = (i / 4) * 8u + (lane >> 5) * 4u + (i % 4);
            ht[r * CZ_GG8_HT + (lane & 31u)] = cz_silu_fast(acc[0][i] * cur[0]) * (acc[1][i] * cur[1]);
        }
        const uint32_t nb = ncol[0] - (lane & 31u), c4 = lane & 7u;  // nb: the wave's first column
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // rows of padding (dst ~0u) hold a copy of the tile's last row:
            // finite, quantised with the rest, not stored
            const uint32_t r = 8u * p + (lane >> 3);
            const float4 v = *reinterpret_cast<const float4 *>(ht + r * CZ_GG8_HT + 4u * c4);
            float rv[4] = {v.x, v.y, v.z, v.w};
            const uint32_t dst = s_rowdst[r];
            const uint64_t o = (uint64_t)(dst == ~0u ? 0u : dst) * P.N + nb;
            cz_q3_group4(rv, P.cq + o + 4u * c4, P.cq_plane, P.ce + o / 32u, P.ce_plane, c4 == 0, dst != ~0u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t r = (i / 4) * 8u + (lane >> 5) * 4u + (i % 4);
            const uint32_t dst = s_rowdst[r];
            if (dst == ~0u) continue;
#pragma unroll
            for (int m = 0; m < 2; ++m) P.c[(uint64_t)dst * P.N + ncol[m]] = acc[m][i] * cur[m];
        }
    }
}

// ---------------------------------------------------------------------------
// combine: out[t][d] = xres + ((0 + sgate*os) + g_a*O_a) + g_b*O_b ... in
// ascending expert id (moe.zig:633-662; shared first, moe.zig:614-630)
// ---------------------------------------------------------------------------
// One workgroup per (token, 1024 columns), 4 columns per thread (H % 4 == 0).
// The token's slot positions and gates are wave-uniform scalar loads; each
// batch of 8 slots has all its loads in flight before the sums.
#define CZ_COMBINE_COLS 1024

__device__ __forceinline__ uint32_t cz_const_u32(const uint32_t *p) {
    return *(const __attribute__((address_space(4))) uint32_t *)p;
}

__global__ __launch_bounds__(256) void k_combine(GroupArgs G) {
    const LayerDev &L = G.L;
    const uint32_t t = blockIdx.y;
    const uint32_t d = blockIdx.x * CZ_COMBINE_COLS + 4u * threadIdx.x;
    if (d >= L.H || t >= (uint32_t)G.S) return;
    const uint64_t H = L.H;
    float4 ys = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (L.SI != 0) {
        const float sg = G.sgate[t];
        const float4 v = *(const float4 *)(G.os + t * H + d);
        ys.x = ys.x + sg * v.x;
        ys.y = ys.y + sg * v.y;
        ys.z = ys.z + sg * v.z;
        ys.w = ys.w + sg * v.w;
    }
    const uint32_t *order = G.tok_order + (uint64_t)t * L.K;
    for (uint32_t z0 = 0; z0 < L.K; z0 += 8) {
        // unconditional loads (slots past K re-read slot K - 1): the scalar
        // index loads of all 8 slots are issued together, then the rows
        uint32_t sl[8], pos[8];
        float g[8];
        float4 v[8];
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) sl[q] = cz_const_u32(order + min(z0 + q, L.K - 1));
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
            g[q] = cz_const_f32(G.gates + sl[q]);
            pos[q] = cz_const_u32(G.slot_pos + sl[q]);
        }
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) v[q] = *(const float4 *)(G.o + (uint64_t)pos[q] * H + d);
#pragma unroll
        for (uint32_t q = 0; q < 8; ++q) {
            if (z0 + q < L.K) {
                ys.x = ys.x + g[q] * v[q].x;
                ys.y = ys.y + g[q] * v[q].y;
                ys.z = ys.z + g[q] * v[q].z;
                ys.w = ys.w + g[q] * v[q].w;
            }
        }
    }
    const uint64_t o = t * H + d;
    float4 r = G.xres ? *(const float4 *)(G.xres + o) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    r.x = r.x + ys.x;
    r.y = r.y + ys.y;
    r.z = r.z + ys.z;
    r.w = r.w + ys.w;
    *(float4 *)(G.out + o) = r;
}

// The combine of one token's whole row (thread tid: float4 columns tid +
// 256 k, each formed as k_combine forms it), then the next layer's RMS rows
// of that row (cz_rms_row_tail with the next layer's arguments An): one
// launch fewer per layer of a chain, and the row is not read back.
template <int Q>
__global__ __launch_bounds__(256) void k_combine_rms(GroupArgs G, StepArgs An) {
    __shared__ __align__(16) float s_row[Q * 1024];
    __shared__ float s_inv;
    const LayerDev &L = G.L;
    const uint32_t t = blockIdx.x, tid = threadIdx.x, n4 = L.H / 4;
    const uint64_t H = L.H;
    const uint32_t *order = G.tok_order + (uint64_t)t * L.K;
    const float sg = L.SI != 0 ? G.sgate[t] : 0.0f;  // read before the tail writes the next layer's
    float4 r[Q];
#pragma unroll
    for (uint32_t k = 0; k < Q; ++k) {
        const uint32_t q = min(tid + 256 * k, n4 - 1);  // clamped: in bounds, not stored
        const uint32_t d = 4u * q;
        float4 ys = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (L.SI != 0) {
            const float4 v = *(const float4 *)(G.os + t * H + d);
            ys.x = ys.x + sg * v.x;
            ys.y = ys.y + sg * v.y;
            ys.z = ys.z + sg * v.z;
            ys.w = ys.w + sg * v.w;
        }
        for (uint32_t z0 = 0; z0 < L.K; z0 += 8) {
            uint32_t sl[8], pos[8];
            float g[8];
            float4 v[8];
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) sl[i] = cz_const_u32(order + min(z0 + i, L.K - 1));
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) {
                g[i] = cz_const_f32(G.gates + sl[i]);
                pos[i] = cz_const_u32(G.slot_pos + sl[i]);
            }
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) v[i] = *(const float4 *)(G.o + (uint64_t)pos[i] * H + d);
#pragma unroll
            for (uint32_t i = 0; i < 8; ++i) {
                if (z0 + i < L.K) {
                    ys.x = ys.x + g[i] * v[i].x;
                    ys.y = ys.y + g[i] * v[i].y;
                    ys.z = ys.z + g[i] * v[i].z;
                    ys.w = ys.w + g[i] * v[i].w;
                }
            }
        }
        const uint64_t o = t * H + d;
        float4 x = G.xres ? *(const float4 *)(G.xres + o) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        x.x = x.x + ys.x;
        x.y = x.y + ys.y;
        x.z = x.z + ys.z;
        x.w = x.w + ys.w;
        r[k] = x;
    }
#pragma unroll
    for (uint32_t k = 0; k < Q; ++k)
        if (tid + 256 * k < n4) *(float4 *)(G.out + t * H + 4u * (tid + 256 * k)) = r[k];
    cz_rms_row_tail<Q>(An, t, r, s_row, &s_inv);
}
