// cz_plan.h - the HBM plan (budget.plan, src/runtime/budget.zig:184-264,
// restated for one GPU's HBM): which layers' routers, shared experts and
// scratch stay resident, and whether every routed expert fits beside them or
// how many expert slots the streaming tier's pool gets.  Plain host C++ (no
// device code): the library wraps it in colizig_hip_plan_hbm, and the CPU
// sanitizer build of the host code compiles it as it is.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdio>

#include "colizig_hip.h"

namespace cz {

// budget.zig:62 cap_ladder: candidate per-layer expert caps, largest first.
constexpr uint32_t kCapLadder[] = {128, 96, 64, 48, 32, 24, 16, 12, 8, 6, 4};

// The forward's regimes as far as its scratch goes: the grouped regime from
// this many tokens on, with M-tiles of this many rows.
constexpr uint32_t kPlanGroupedMinTokens = 16;
constexpr uint32_t kPlanTileRows = 32;

inline uint64_t plan_nblk(uint64_t x) { return (x + 127) / 128; }

// The forward's scratch for S tokens, byte for byte what the library's
// decode scratch and, in the grouped regime, its grouped scratch allocate in
// the given prefill mode (FP8: three E4M3 terms and their exponents of the
// GEMM operands; f16: hi + lo splits).
inline uint64_t work_bytes(const colizig_dims &d, uint64_t S, bool prefill_fp8) {
    const uint64_t sk = S * d.topk, H = d.hidden, SI = d.shared_inter;
    const uint64_t mt = sk / kPlanTileRows + std::min<uint64_t>(d.experts, sk) + 1;
    const uint64_t si = std::max<uint64_t>(1, S * SI);
    uint64_t b = 4 * (3 * S * H + S * d.experts + 2 * sk + S + sk * d.inter + si);  // xin, out, xn, logits, ..
    if (SI) b += 4 * (2 * S * SI + S * H + S);  // the shared expert's gate, up, down rows and gate
    if (S < kPlanGroupedMinTokens) return b;
    b += 4 * (2 * (uint64_t)d.experts + 1 + 3 * sk + 2 * mt + 1 + sk * H + std::max<uint64_t>(1, S * H));
    if (prefill_fp8)
        b += 3 * (S * H + sk * d.inter) + 3 * (S * H + sk * d.inter) / 32 + std::max<uint64_t>(1, 3 * S * SI) +
             std::max<uint64_t>(1, 3 * S * SI / 32);
    else
        b += 2 * (2 * S * H + 2 * sk * d.inter + 2 * si);
    return b;
}

// budget.plan for `layers` layers of dims d within hbm_budget bytes and a
// forward of up to max_tokens tokens; the arguments are checked by the caller.
inline colizig_hbm_plan plan_hbm(const colizig_dims &d, uint32_t layers, uint64_t hbm_budget, uint32_t max_tokens,
                                 bool prefill_fp8) {
    colizig_hbm_plan p{};
    p.hbm_budget = hbm_budget;
    const uint64_t H = d.hidden, nbH = plan_nblk(d.hidden);
    p.per_expert_bytes = (3ull * d.inter * H + 12ull * plan_nblk(d.inter) * nbH + 15) / 16 * 16;
    p.per_layer_fixed = 4ull * d.experts * H + 8ull * d.experts + 4ull * d.experts;
    if (d.shared_inter) p.per_layer_fixed += 3ull * d.shared_inter * H + 12ull * plan_nblk(d.shared_inter) * nbH + 4 * H;
    p.scratch = work_bytes(d, std::max<uint32_t>(1, max_tokens), prefill_fp8);
    p.fixed_resident = (uint64_t)layers * p.per_layer_fixed + p.scratch;
    const uint64_t all_experts = (uint64_t)layers * d.experts;
    if (p.fixed_resident > hbm_budget) {
        snprintf(p.reason, sizeof p.reason, "the resident routers, shared experts and scratch exceed the HBM budget");
    } else if (p.fixed_resident + all_experts * p.per_expert_bytes <= hbm_budget) {
        p.all_resident = 1;
        p.expert_bytes = all_experts * p.per_expert_bytes;
        p.expert_cap = d.experts;
        for (uint32_t c : kCapLadder)
            if (c <= p.expert_cap) {
                p.ladder_cap = c;
                break;
            }
        p.fits = 1;
    } else {
        const uint64_t slots = std::min<uint64_t>((hbm_budget - p.fixed_resident) / p.per_expert_bytes, all_experts);
        if (slots < d.topk) {
            snprintf(p.reason, sizeof p.reason, "the expert pool would hold %llu experts, fewer than top-k %u",
                     (unsigned long long)slots, d.topk);
        } else {
            p.pool_slots = (uint32_t)std::min<uint64_t>(slots, 1u << 24);
            p.expert_bytes = (uint64_t)p.pool_slots * p.per_expert_bytes;
            p.expert_cap = p.pool_slots / layers;
            for (uint32_t c : kCapLadder)
                if (c <= p.expert_cap) {
                    p.ladder_cap = c;
                    break;
                }
            p.fits = 1;
        }
    }
    p.total = p.fixed_resident + p.expert_bytes;
    return p;
}

}  // namespace cz
