// cz_device.h - device helpers for the gfx950 MoE expert path: f32 exp,
// sigmoid/SiLU, OCP E4M3 decode, wave64 reductions.
//
// Everything here is compiled with -ffp-contract=off: a fused multiply-add
// appears only where it is written (__builtin_fmaf / __builtin_fma).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define CZ_BLOCK 128
#define CZ_WAVE 64

typedef float cz_float2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// f32 exp: the f32 rounding of a double-precision evaluation
//   k = nearest integer to x/ln2 (shifter 0x1.8p52, two separate roundings)
//   r = (x - k*ln2_hi) - k*ln2_lo via two fma
//   p = sum_{n<=13} r^n/n! by Horner with fma  (|r| <= ln2/2, truncation < 2^-57)
//   exp(x) ~= p * 2^k, exact power-of-two scaling, then one RNE to f32.
// Every step is an IEEE-754 double add/mul/fma or an exact conversion, so the
// host and the GPU produce the same bits.  Exhaustively (all 2^32 inputs) it
// equals the correctly rounded f32 exp.  Used by the router softmax
// (moe.zig:443) and the sigmoid in SiLU (activation.zig:9-20).
// ---------------------------------------------------------------------------
__host__ __device__ inline float cz_expf(float xf) {
    if (xf != xf) return xf + xf;
    double x = (double)xf;
    x = x > 100.0 ? 100.0 : x;    // exp(100) rounds to +inf in f32
    x = x < -120.0 ? -120.0 : x;  // exp(-120) rounds to +0 in f32
    const double t0 = x * 0x1.71547652b82fep+0;  // 1/ln2
    const double t1 = t0 + 0x1.8p52;
    const double kd = t1 - 0x1.8p52;
    double r = __builtin_fma(-kd, 0x1.62e42fefa39efp-1, x);  // ln2 high part
    r = __builtin_fma(-kd, 0x1.abc9e3b39803fp-56, r);         // ln2 low part
    double p = 0x1.6124613a86d09p-33;                         // 1/13!
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);           // 1/12!
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);           // 1/11!
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);           // 1/10!
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);           // 1/9!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);           // 1/8!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);           // 1/7!
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);           // 1/6!
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);            // 1/5!
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);            // 1/4!
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);            // 1/3!
    p = __builtin_fma(p, r, 0x1.0p-1);                        // 1/2!
    p = __builtin_fma(p, r, 1.0);                             // 1/1!
    p = __builtin_fma(p, r, 1.0);                             // 1/0!
    const int k = (int)kd;
    const uint64_t sbits = (uint64_t)(int64_t)(k + 1023) << 52;
    const double scale = __builtin_bit_cast(double, sbits);
    return (float)(p * scale);
}

// activation.zig:9-16: two-branch stable sigmoid, f32 arithmetic.
__host__ __device__ inline float cz_sigmoid(float x) {
    if (x >= 0.0f) {
        const float z = cz_expf(-x);
        return 1.0f / (1.0f + z);
    }
    const float z = cz_expf(x);
    return z / (1.0f + z);
}

// activation.zig:18-20
__host__ __device__ inline float cz_silu(float x) { return x * cz_sigmoid(x); }

// The same two-branch silu on the hardware exponential and reciprocal
// (v_exp_f32, v_rcp_f32: about 1 ulp each).  The expert activations use it:
// their results are held to a relative L2 of 1e-3, not to the bit, while
// routing keeps the correctly rounded cz_expf.
__device__ inline float cz_silu_fast(float x) {
    const float z = __expf(-__builtin_fabsf(x));  // (0, 1]
    const float r = __builtin_amdgcn_rcpf(1.0f + z);
    return x * (x >= 0.0f ? r : z * r);
}

// ---------------------------------------------------------------------------
// OCP E4M3 (e4m3fn) decode with gfx950's v_cvt_pk_f32_fp8: two bytes of a
// dword per instruction, exact (every E4M3 value is an f32).  The dequantised
// weight is then ONE f32 multiply by the 128x128 block scale, the definition
// fp8.zig:105 uses.
// ---------------------------------------------------------------------------
// 16 bytes of streamed weights, loaded non-temporal: they are read once per
// token, so they should not displace what the caches hold for the next steps
// (router rows, exchanged values, activations).
__device__ inline uint4 cz_ld_nt16(const uint8_t *p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ inline cz_float2 cz_fp8x2_lo(uint32_t w) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false); }
__device__ inline cz_float2 cz_fp8x2_hi(uint32_t w) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true); }

// acc += x[0..3] * (e4m3(bytes of w) * s), element order = byte order.
__device__ inline float cz_dot4_fp8(uint32_t w, float s, const float *x4, float acc) {
    const cz_float2 lo = cz_fp8x2_lo(w);
    const cz_float2 hi = cz_fp8x2_hi(w);
    acc = __builtin_fmaf(x4[0], lo.x * s, acc);
    acc = __builtin_fmaf(x4[1], lo.y * s, acc);
    acc = __builtin_fmaf(x4[2], hi.x * s, acc);
    acc = __builtin_fmaf(x4[3], hi.y * s, acc);
    return acc;
}

// ---------------------------------------------------------------------------
// wave64 reductions
// cz_wave_sum / cz_wave_max: xor butterfly through ds_bpermute (any lane
// order; kept where a specific combine order is part of the contract).
// cz_wave_sum_dpp / cz_wave_max_dpp: four DPP steps inside each 16-lane row
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror),
// after which every lane of a row holds the row's result, then the four rows
// combined as (r0 + r1) + (r2 + r3) from readlane.  The result is uniform.
// ---------------------------------------------------------------------------
__device__ inline float cz_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, CZ_WAVE);
    return v;
}

__device__ inline float cz_wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, CZ_WAVE));
    return v;
}

template <int CTRL>
__device__ inline float cz_dpp(float v) {
    const int i = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(i, i, CTRL, 0xF, 0xF, false));
}

__device__ inline float cz_readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ inline float cz_wave_sum_dpp(float v) {
    v = v + cz_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v = v + cz_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v = v + cz_dpp<0x141>(v);  // row_half_mirror
    v = v + cz_dpp<0x140>(v);  // row_mirror
    const float r0 = cz_readlane(v, 0), r1 = cz_readlane(v, 16), r2 = cz_readlane(v, 32), r3 = cz_readlane(v, 48);
    return (r0 + r1) + (r2 + r3);
}

__device__ inline float cz_wave_max_dpp(float v) {
    v = fmaxf(v, cz_dpp<0xB1>(v));
    v = fmaxf(v, cz_dpp<0x4E>(v));
    v = fmaxf(v, cz_dpp<0x141>(v));
    v = fmaxf(v, cz_dpp<0x140>(v));
    const float r0 = cz_readlane(v, 0), r1 = cz_readlane(v, 16), r2 = cz_readlane(v, 32), r3 = cz_readlane(v, 48);
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ inline uint32_t cz_lane() { return threadIdx.x & (CZ_WAVE - 1); }

// Sum of a double over the 64 lanes (xor butterfly), returned to every lane.
__device__ inline double cz_wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, CZ_WAVE);
    return v;
}

template <int CTRL>
__device__ inline double cz_dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
    const uint32_t l2 = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, 0xF, 0xF, false);
    const uint32_t h2 = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)h2 << 32) | l2);
}

// The same sum through DPP moves inside each 16-lane row, then the four row
// sums as (r0 + r1) + (r2 + r3); uniform result.
__device__ inline double cz_wave_sum_f64_dpp(double v) {
    v = v + cz_dpp_f64<0xB1>(v);   // quad_perm [1,0,3,2]
    v = v + cz_dpp_f64<0x4E>(v);   // quad_perm [2,3,0,1]
    v = v + cz_dpp_f64<0x141>(v);  // row_half_mirror
    v = v + cz_dpp_f64<0x140>(v);  // row_mirror
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
    double r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        r[k] = __builtin_bit_cast(double, ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, 16 * k) << 32) |
                                              (uint32_t)__builtin_amdgcn_readlane(lo, 16 * k));
    return (r[0] + r[1]) + (r[2] + r[3]);
}

// rmsnorm.zig:32-40 `rms` with a unit weight, from ss = the f64 sum of the
// row's squares (each f64(v)*v is exact in f64, so the sum differs from the
// reference's row-order sum only by f64 rounding far below an f32 ulp):
// mean = f32(ss / n), r = 1 / sqrt(mean + eps) in f32 (correctly rounded
// division and square root); the row is then x_i * r.
__device__ inline float cz_rms_inv(double ss, uint32_t n, float eps) {
    const float mean = (float)(ss / (double)n);
    return 1.0f / sqrtf(mean + eps);
}

// Wave max of unsigned integers, returned to every lane: four butterfly DPP
// steps inside each 16-lane row, row_bcast:15 and row_bcast:31 across rows
// (a missing DPP source reads 0, the identity of an unsigned max, so every
// step is exact), then lane 63.  Each DPP move folds into the v_max_u32.
__device__ inline uint32_t cz_wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));   // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));   // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));  // row_half_mirror
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));  // row_mirror
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x142, 0xF, 0xF, true));  // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x143, 0xF, 0xF, true));  // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// DPP move of an integer; lanes whose source lane does not exist (or whose
// row is masked off) read 0.
template <int CTRL, int ROWS = 0xF>
__device__ inline uint32_t cz_dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, false);
}

// Inclusive prefix sum over the 64 lanes of a wave (integers: the order of
// the additions does not matter): row_shr 1, 2, 4, 8 inside each 16-lane row,
// then row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3.
__device__ inline uint32_t cz_wave_incl_scan_u32(uint32_t v) {
    v += cz_dpp_u32<0x111>(v);
    v += cz_dpp_u32<0x112>(v);
    v += cz_dpp_u32<0x114>(v);
    v += cz_dpp_u32<0x118>(v);
    v += cz_dpp_u32<0x142, 0xA>(v);
    v += cz_dpp_u32<0x143, 0xC>(v);
    return v;
}

// Inclusive prefix sum inside aligned groups of g lanes (g = 1, 2, 4, 8 or
// 16, wave-uniform; a group lies inside one 16-lane row).
__device__ inline uint32_t cz_group_incl_scan_u32(uint32_t v, uint32_t g) {
    const uint32_t p = cz_lane() & (g - 1);
    if (g > 1) { const uint32_t t = cz_dpp_u32<0x111>(v); v += p >= 1 ? t : 0u; }
    if (g > 2) { const uint32_t t = cz_dpp_u32<0x112>(v); v += p >= 2 ? t : 0u; }
    if (g > 4) { const uint32_t t = cz_dpp_u32<0x114>(v); v += p >= 4 ? t : 0u; }
    if (g > 8) { const uint32_t t = cz_dpp_u32<0x118>(v); v += p >= 8 ? t : 0u; }
    return v;
}
