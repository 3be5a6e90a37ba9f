"""The HBM plan (budget.plan, src/runtime/budget.zig:184-264, restated for
one GPU's HBM) on the CPU: the reference's own three plan tests
(budget.zig:276-301) restated for the HBM budget, and the closed forms of
the configs' sizes."""
from __future__ import annotations

from colizig_amd import moe

GB = 1 << 30


def nblk(x):
    return (x + 127) // 128


def test_more_tokens_never_lower_the_resident_target():
    """budget.zig:276-283: more context (here: more tokens per forward) never
    lowers the resident set."""
    d = moe.dims(512, 16, 4, 256)
    a = moe.plan_hbm(d, 4, 1 * GB, max_tokens=16)
    b = moe.plan_hbm(d, 4, 1 * GB, max_tokens=512)
    assert b["scratch"] > a["scratch"] and b["fixed_resident"] >= a["fixed_resident"]


def test_cap_shrinks_with_the_budget():
    """budget.zig:285-292: a smaller budget never gives a larger expert cap;
    both fit."""
    d = moe.dims(2048, 128, 8, 768)
    big = moe.plan_hbm(d, 48, 24 * GB)
    small = moe.plan_hbm(d, 48, 6 * GB)
    assert big["fits"] and small["fits"]
    assert big["expert_cap"] >= small["expert_cap"] and big["pool_slots"] > small["pool_slots"]
    assert not big["all_resident"] and not small["all_resident"]


def test_tiny_budget_fails_gracefully():
    """budget.zig:294-301: a budget below the resident set does not fit, says
    why, and gives no cap."""
    d = moe.dims(2048, 128, 8, 768)
    p = moe.plan_hbm(d, 48, 1 << 20, max_tokens=512)
    assert not p["fits"] and p["reason"] and p["expert_cap"] == 0 and p["pool_slots"] == 0
    # the resident set fits but not even top-k expert slots after it
    d4 = moe.dims(4096, 512, 10, 512, 4096)
    fixed = moe.plan_hbm(d4, 36, 1 << 40)["fixed_resident"]
    q = moe.plan_hbm(d4, 36, fixed + 9 * moe.plan_hbm(d4, 36, 1 << 40)["per_expert_bytes"])
    assert not q["fits"] and "top-k" in q["reason"]


def test_config_sizes_closed_form():
    """Qwen3-30B-A3B (48 layers) and Qwen4-Exp (36 layers) resident in 288 GB;
    the 16 GB pool of the streaming tier holds 3,390 experts of 4,719,744 B."""
    d2 = moe.dims(2048, 128, 8, 768)
    per = 3 * 768 * 2048 + 12 * nblk(768) * nblk(2048)
    assert per == 4_719_744
    p = moe.plan_hbm(d2, 48, 288 * 10**9)
    assert p["per_expert_bytes"] == per and p["all_resident"] and p["fits"]
    assert p["expert_bytes"] == 48 * 128 * per
    assert p["per_layer_fixed"] == 128 * 2048 * 4 + 128 * 12
    assert p["expert_cap"] == 128 and p["ladder_cap"] == 128
    s = moe.plan_hbm(d2, 48, p["fixed_resident"] + 16 * 10**9)
    assert not s["all_resident"] and s["pool_slots"] == 16 * 10**9 // per == 3390
    assert s["expert_cap"] == 3390 // 48 and s["ladder_cap"] == 64
    d4 = moe.dims(4096, 512, 10, 512, 4096)
    q = moe.plan_hbm(d4, 36, 288 * 10**9)
    per4 = 3 * 512 * 4096 + 12 * nblk(512) * nblk(4096)
    assert q["all_resident"] and q["expert_bytes"] == 36 * 512 * per4
    assert q["per_layer_fixed"] == 512 * 4096 * 4 + 512 * 12 + 3 * 4096 * 4096 + 12 * 32 * 32 + 4 * 4096
    assert 115e9 < q["total"] < 120e9
