// The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer
// (the counterpart of the reference's Debug-build safety checks): the
// streaming tier's scheduler and last-token predictor (cz_sched.h), the HBM
// plan (cz_plan.h) and the engine-side loader (cz_gpu_loader.cpp, linked in
// and driven against host-only stub backends).  The cases restate the
// reference's own tests of these parts (io.zig:145-197, predict.zig:94-124,
// budget.zig:276-301, gpu.zig:72-190) and add invariants over many plan
// shapes.  Exits 0 when every check holds; a sanitizer finding aborts.
//
//   host_check <stub ok .so> <stub init-fails .so> <stub missing-symbol .so>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "cz_lru.h"
#include "cz_plan.h"
#include "cz_sched.h"

extern "C" {
int czgpu_init(const char *lib_path, char *err, size_t errlen);
void czgpu_deinit(void);
int czgpu_available(void);
int czgpu_has_moe(void);
const char *czgpu_device_name(void);
void czgpu_set_vram_budget(uint64_t bytes);
int czgpu_stats_line(char *buf, size_t n);
int czgpu_matmul_fp8(float *y, const float *x, const unsigned char *w, const float *scales, size_t S, size_t I,
                     size_t O, uint64_t key);
int czgpu_moe_forward(uint32_t layer, const float *x, size_t S, float *out, uint32_t *idx, float *gates);
}

static int failures = 0;
#define CHECK(c)                                                                  \
    do {                                                                          \
        if (!(c)) {                                                               \
            std::fprintf(stderr, "check failed: %s (%s:%d)\n", #c, __FILE__, __LINE__); \
            ++failures;                                                           \
        }                                                                         \
    } while (0)

static void sched_cases() {
    using cz::ExpertKey;
    // io.zig:147-161: strongest priority first, FIFO within one
    cz::Scheduler s(16);
    CHECK(s.submit(ExpertKey{0, 1}, cz::kLow));
    CHECK(s.submit(ExpertKey{9, 100}, cz::kMedium));
    CHECK(s.submit(ExpertKey{7, 3}, cz::kHigh));
    CHECK(s.submit(ExpertKey{9, 101}, cz::kHigh));
    const uint32_t want[4][2] = {{7, 3}, {9, 101}, {9, 100}, {0, 1}};
    for (const auto &w : want) {
        ExpertKey k;
        CHECK(s.next(&k) && k.layer == w[0] && k.id == w[1]);
    }
    ExpertKey k;
    CHECK(!s.next(&k));
    CHECK(s.stats().serviced[0] == 2 && s.stats().serviced[1] == 1 && s.stats().serviced[2] == 1);
    // io.zig:163-179: a re-submit dedups and upgrades; a full queue refuses
    cz::Scheduler f(2);
    CHECK(f.submit(ExpertKey{1, 1}, cz::kLow) && f.submit(ExpertKey{1, 1}, cz::kHigh));
    CHECK(f.stats().deduped == 1 && f.stats().upgraded == 1 && f.len() == 1);
    CHECK(f.submit(ExpertKey{1, 2}, cz::kLow) && !f.submit(ExpertKey{1, 3}, cz::kLow));
    CHECK(f.stats().rejected_full == 1 && f.stats().queue_peak == 2);
    CHECK(f.cancel(ExpertKey{1, 2}) && !f.cancel(ExpertKey{1, 2}) && f.stats().cancelled == 1);
    CHECK(f.next(&k) && k.id == 1 && f.len() == 0);
    // a long mixed sequence against a plain model of the queue
    std::mt19937 rng(7);
    cz::Scheduler q(24);
    std::vector<std::pair<ExpertKey, int>> model;
    for (int i = 0; i < 20000; ++i) {
        const ExpertKey key{(uint32_t)(rng() % 4), (uint32_t)(rng() % 16)};
        const int op = (int)(rng() % 4);
        if (op < 2) {
            const auto p = (cz::Prio)(rng() % 3);
            bool found = false;
            for (auto &m : model)
                if (m.first == key) {
                    found = true;
                    if (p < m.second) m.second = p;
                }
            const bool full = model.size() >= 24;
            const bool ok = q.submit(key, p);
            if (!found && !full) model.push_back({key, p});
            CHECK(ok == (found || !full));
        } else if (op == 2) {
            ExpertKey got;
            const bool ok = q.next(&got);
            CHECK(ok == !model.empty());
            if (ok) {
                size_t best = 0;
                for (size_t j = 1; j < model.size(); ++j)
                    if (model[j].second < model[best].second) best = j;
                CHECK(model[best].first == got);
                model.erase(model.begin() + (std::ptrdiff_t)best);
            }
        } else {
            bool found = false;
            for (size_t j = 0; j < model.size(); ++j)
                if (model[j].first == key) {
                    model.erase(model.begin() + (std::ptrdiff_t)j);
                    found = true;
                    break;
                }
            CHECK(q.cancel(key) == found);
        }
        CHECK(q.len() == model.size());
    }
}

static void predictor_cases() {
    // predict.zig:94-110
    cz::LastTokenPredictor p(2);
    CHECK(p.predict(0).empty());
    const uint32_t a[2] = {5, 9}, b[2] = {5, 3};
    p.record(0, a, 2);
    CHECK(p.predict(0).size() == 2 && p.predict(0)[0] == 5 && p.predict(0)[1] == 9);
    p.record(0, a, 2);
    p.record(0, b, 2);
    CHECK(p.stats().predicted == 6 && p.stats().correct == 3);
    // predict.zig:112-124 (predictScored)
    cz::LastTokenPredictor q(3);
    const uint32_t c[5] = {1, 2, 3, 4, 5};
    q.record(1, c, 5);
    cz::PrefetchPrediction rows[4];
    const size_t n = q.predict_scored(1, rows, 4);
    CHECK(n == 3 && rows[0].layer == 1 && rows[1].expert == 2 && rows[2].expected_use_distance == 1);
    CHECK(rows[0].confidence == 0.1f);
    CHECK(q.predict_scored(0, rows, 4) == 0 && q.predict_scored(1, rows, 1) == 1);
}

// The pool's victim choice (cz_lru.h) against a scan of every slot, as the
// pool chose before: the first free slot, else the held slot with the lowest
// last-use clock among those the layer in flight does not pin; nslots when
// all are pinned.  Random fills, hits, drops and pins over small pools.
static void lru_cases() {
    std::mt19937_64 rng(7);
    for (uint32_t n : {1u, 2u, 5u, 63u, 64u, 65u, 130u}) {
        cz::SlotLru lru;
        lru.reset(n);
        std::vector<uint64_t> used(n, 0), pin(n, 0);
        std::vector<uint8_t> held(n, 0);
        uint64_t clock = 0, epoch = 0;
        auto scan = [&]() {
            uint32_t best = n;
            uint64_t bu = ~0ull;
            for (uint32_t i = 0; i < n; ++i) {
                if (!held[i]) return i;
                if (epoch != 0 && pin[i] == epoch) continue;
                if (used[i] < bu) {
                    bu = used[i];
                    best = i;
                }
            }
            return best;
        };
        auto pinned = [&](uint32_t i) { return epoch != 0 && pin[i] == epoch; };
        for (int step = 0; step < 20000; ++step) {
            const uint32_t op = (uint32_t)(rng() % 10);
            const uint32_t i = (uint32_t)(rng() % n);
            if (op < 4) {  // a fill into the victim, which the layer in flight then pins
                const uint32_t v = lru.victim(pinned);
                CHECK(v == scan());
                if (v < n) {
                    held[v] = 1;
                    used[v] = ++clock;
                    lru.touch(v);
                    pin[v] = epoch;
                }
            } else if (op < 7) {  // a hit
                if (held[i]) {
                    used[i] = ++clock;
                    lru.touch(i);
                    pin[i] = epoch;
                }
            } else if (op < 8) {  // the entry is dropped
                held[i] = 0;
                lru.release(i);
            } else {  // the next layer: a new pin epoch
                ++epoch;
            }
            CHECK(lru.held(i) == (held[i] != 0));
        }
        // every slot held and pinned: no victim
        ++epoch;
        for (uint32_t i = 0; i < n; ++i) {
            if (!held[i]) {
                held[i] = 1;
                used[i] = ++clock;
                lru.touch(i);
            }
            pin[i] = epoch;
        }
        CHECK(lru.victim(pinned) == n && scan() == n);
        lru.reset(n);
        CHECK(lru.victim(pinned) == 0);
    }
}

static void plan_cases() {
    const uint64_t GB = 1ull << 30;
    const colizig_dims small{512, 16, 4, 256, 0, 1}, q3{2048, 128, 8, 768, 0, 1}, q4{4096, 512, 10, 512, 4096, 1};
    // budget.zig:276-283: more tokens never lower the resident target
    const colizig_hbm_plan a = cz::plan_hbm(small, 4, GB, 16, true), b = cz::plan_hbm(small, 4, GB, 512, true);
    CHECK(b.scratch > a.scratch && b.fixed_resident >= a.fixed_resident);
    // budget.zig:285-292: a smaller budget never gives a larger cap
    const colizig_hbm_plan big = cz::plan_hbm(q3, 48, 24 * GB, 1, true), lit = cz::plan_hbm(q3, 48, 6 * GB, 1, true);
    CHECK(big.fits && lit.fits && big.expert_cap >= lit.expert_cap && big.pool_slots > lit.pool_slots);
    // budget.zig:294-301: a budget below the resident set fails and says why
    const colizig_hbm_plan tiny = cz::plan_hbm(q3, 48, 1ull << 20, 512, true);
    CHECK(!tiny.fits && std::strlen(tiny.reason) > 0 && tiny.expert_cap == 0);
    // closed forms: one Qwen3-30B-A3B expert and the whole c2 stack resident
    CHECK(q3.inter == 768 && cz::plan_hbm(q3, 48, 288 * GB, 1, true).all_resident == 1);
    CHECK(cz::plan_hbm(q3, 48, 288 * GB, 1, true).per_expert_bytes ==
          (3ull * 768 * 2048 + 12ull * 6 * 16 + 15) / 16 * 16);
    CHECK(cz::plan_hbm(q4, 36, 288 * GB, 32, true).all_resident == 1);
    // invariants over many shapes, budgets and token counts
    std::mt19937_64 rng(11);
    for (int i = 0; i < 50000; ++i) {
        colizig_dims d{};
        d.hidden = 128u << (rng() % 6);
        d.experts = 1u + (uint32_t)(rng() % 1024);
        d.topk = 1u + (uint32_t)(rng() % std::min<uint32_t>(d.experts, 32));
        d.inter = 128u * (1u + (uint32_t)(rng() % 32));
        d.shared_inter = (rng() % 2) ? 128u * (uint32_t)(rng() % 32) : 0u;
        d.norm_topk = 1;
        const uint32_t layers = 1u + (uint32_t)(rng() % 96), toks = (uint32_t)(rng() % 4096);
        const uint64_t budget = rng() % (400 * GB);
        const colizig_hbm_plan p = cz::plan_hbm(d, layers, budget, toks, (rng() % 2) != 0);
        CHECK(p.total == p.fixed_resident + p.expert_bytes);
        CHECK(!p.fits || p.total <= budget);
        CHECK(!p.all_resident || (p.fits && p.expert_cap == d.experts && p.pool_slots == 0));
        CHECK(!p.fits || p.all_resident || (p.pool_slots >= d.topk && p.expert_bytes == (uint64_t)p.pool_slots * p.per_expert_bytes));
        CHECK(p.ladder_cap <= p.expert_cap);
        CHECK(p.fits || std::strlen(p.reason) > 0);
        CHECK(p.scratch >= cz::work_bytes(d, 1, true) || toks == 0);
    }
}

static void loader_cases(const char *ok_so, const char *fail_so, const char *missing_so) {
    char err[256];
    // gpu.zig:79-82: no library
    CHECK(czgpu_init("/nonexistent/libcolizig_hip.so", err, sizeof err) == 0);
    CHECK(std::strstr(err, "not found - using CPU") != nullptr && czgpu_available() == 0);
    // gpu.zig:84-89: a missing symbol is named
    CHECK(czgpu_init(missing_so, err, sizeof err) == 0);
    CHECK(std::strstr(err, "colizig_cuda_matmul_fp8 missing") != nullptr && czgpu_available() == 0);
    // gpu.zig:91-96: init rc != 0
    CHECK(czgpu_init(fail_so, err, sizeof err) == 0);
    CHECK(std::strstr(err, "no usable GPU device (colizig_cuda_init rc=-1)") != nullptr);
    float y[6] = {0}, x[4] = {0};
    unsigned char w[16] = {0};
    CHECK(czgpu_matmul_fp8(y, x, w, x, 1, 4, 4, 0) == 0);  // unavailable: the CPU path
    // the success path, then a few calls and the status line
    CHECK(czgpu_init(ok_so, err, sizeof err) == 1 && czgpu_available() == 1 && czgpu_has_moe() == 0);
    CHECK(std::strcmp(czgpu_device_name(), "host stub backend") == 0);
    czgpu_set_vram_budget(1ull << 30);
    CHECK(czgpu_matmul_fp8(y, x, w, x, 2, 4, 3, 42) == 1 && y[5] == 3.0f);
    CHECK(czgpu_moe_forward(0, x, 1, y, nullptr, nullptr) == 0);  // optional symbol absent
    char line[8];  // truncated on purpose: snprintf must stay in bounds
    CHECK(czgpu_stats_line(line, sizeof line) > 0 && std::strlen(line) == sizeof line - 1);
    char full[256];
    CHECK(czgpu_stats_line(full, sizeof full) > 0 && std::strstr(full, "2 matmuls") != nullptr);  // hits 1 + misses 1
    czgpu_deinit();
    CHECK(czgpu_available() == 0 && czgpu_stats_line(full, sizeof full) == 0);
}

int main(int argc, char **argv) {
    if (argc != 4) {
        std::fprintf(stderr, "usage: host_check <stub ok> <stub init fails> <stub missing symbol>\n");
        return 2;
    }
    sched_cases();
    predictor_cases();
    plan_cases();
    lru_cases();
    loader_cases(argv[1], argv[2], argv[3]);
    std::printf("host_check: %s (%d failed checks)\n", failures ? "FAILED" : "ok", failures);
    return failures ? 1 : 0;
}
