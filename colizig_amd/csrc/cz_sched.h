// cz_sched.h - host-side policy of the expert-streaming tier: the bounded
// priority queue of expert fills (Scheduler, src/runtime/io.zig:58-140) and
// the routing predictors that feed it (LastTokenPredictor,
// src/runtime/predict.zig:29-90, and its accuracy Stats, :19-27).  Plain C++,
// no device code: the library's streaming tier drives them and the C-ABI
// exposes them for tests.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <unordered_map>
#include <vector>

namespace cz {

// io.zig:19-21: HIGH = needed by the layer in flight, MEDIUM = predicted next
// working set, LOW = speculative.
enum Prio : int { kHigh = 0, kMedium = 1, kLow = 2 };

struct ExpertKey {
    uint32_t layer = 0, id = 0;
    bool operator==(const ExpertKey &o) const { return layer == o.layer && id == o.id; }
};

// io.zig:38-52
struct SchedStats {
    uint64_t submitted = 0, deduped = 0, upgraded = 0, rejected_full = 0;
    uint64_t serviced[3] = {0, 0, 0};
    uint64_t cancelled = 0, queue_peak = 0;
};

// io.zig:60-140: a bounded queue; next() returns the strongest priority
// first, FIFO within a priority; a re-submit dedups and may upgrade the
// entry's priority; submit refuses when full (the caller then serves the key
// some other way or drops a speculative one).
class Scheduler {
   public:
    explicit Scheduler(size_t capacity) : cap_(capacity) {}

    size_t len() const { return q_.size(); }
    const SchedStats &stats() const { return st_; }

    bool has(const ExpertKey &k) const {
        for (const Entry &e : q_)
            if (e.key == k) return true;
        return false;
    }

    bool submit(const ExpertKey &k, Prio p) {
        for (Entry &e : q_) {
            if (e.key == k) {
                st_.deduped++;
                if (p < e.prio) {
                    e.prio = p;
                    st_.upgraded++;
                }
                return true;
            }
        }
        if (q_.size() >= cap_) {
            st_.rejected_full++;
            return false;
        }
        q_.push_back(Entry{k, p, ++seq_});
        st_.submitted++;
        st_.queue_peak = std::max<uint64_t>(st_.queue_peak, q_.size());
        return true;
    }

    bool next(ExpertKey *out) {
        if (q_.empty()) return false;
        size_t best = 0;
        for (size_t i = 1; i < q_.size(); ++i) {
            const Entry &e = q_[i], &b = q_[best];
            if (e.prio < b.prio || (e.prio == b.prio && e.seq < b.seq)) best = i;
        }
        const Entry e = q_[best];
        q_.erase(q_.begin() + (std::ptrdiff_t)best);
        st_.serviced[e.prio]++;
        *out = e.key;
        return true;
    }

    bool cancel(const ExpertKey &k) {
        for (size_t i = 0; i < q_.size(); ++i) {
            if (q_[i].key == k) {
                q_.erase(q_.begin() + (std::ptrdiff_t)i);
                st_.cancelled++;
                return true;
            }
        }
        return false;
    }

    void clear() { q_.clear(); }

    // Restarts the counters (the peak at the current queue length).
    void reset_stats() {
        st_ = SchedStats{};
        st_.queue_peak = q_.size();
    }

   private:
    struct Entry {
        ExpertKey key;
        Prio prio;
        uint64_t seq;
    };
    size_t cap_;
    std::vector<Entry> q_;
    uint64_t seq_ = 0;
    SchedStats st_;
};

// predict.zig:12-17: one predicted expert with its confidence and the
// number of layers until it is expected to be used.
struct PrefetchPrediction {
    uint32_t layer = 0, expert = 0;
    float confidence = 0.0f;
    uint32_t expected_use_distance = 0;
};

// predict.zig:19-27: of every routed id, whether the prediction held it.
struct PredStats {
    uint64_t predicted = 0, correct = 0;
    double accuracy() const { return predicted == 0 ? 0.0 : (double)correct / (double)predicted; }
    void score(const std::vector<uint32_t> &pred, const uint32_t *ids, size_t n) {
        for (size_t i = 0; i < n; ++i) {
            predicted++;
            if (std::find(pred.begin(), pred.end(), ids[i]) != pred.end()) correct++;
        }
    }
};

// predict.zig:29-90: the ids a layer routed for the previous token are the
// prediction for the next token's routing of that layer (empty until the
// first record); record scores the previous prediction, then keeps the first
// topk ids.
class LastTokenPredictor {
   public:
    explicit LastTokenPredictor(size_t topk) : topk_(topk) {}

    const std::vector<uint32_t> &predict(uint32_t layer) const {
        static const std::vector<uint32_t> none;
        const auto it = last_.find(layer);
        return it == last_.end() ? none : it->second;
    }

    // predict.zig:61-72: the prediction as rows of at most max, each with
    // the predictor's accuracy so far as its confidence (at least 0.1) and
    // an expected use distance of one layer; returns the rows written.
    size_t predict_scored(uint32_t layer, PrefetchPrediction *out, size_t max) const {
        const std::vector<uint32_t> &ids = predict(layer);
        const float conf = (float)std::max(0.1, st_.accuracy());
        const size_t n = std::min(ids.size(), max);
        for (size_t i = 0; i < n; ++i) out[i] = PrefetchPrediction{layer, ids[i], conf, 1u};
        return n;
    }

    void record(uint32_t layer, const uint32_t *ids, size_t n) {
        st_.score(predict(layer), ids, n);
        last_[layer].assign(ids, ids + std::min(n, topk_));
    }

    void reset() {
        last_.clear();
        st_ = PredStats{};
    }

    const PredStats &stats() const { return st_; }
    void reset_stats() { st_ = PredStats{}; }
    void set_topk(size_t topk) { topk_ = topk; }

   private:
    size_t topk_;
    std::unordered_map<uint32_t, std::vector<uint32_t>> last_;
    PredStats st_;
};

}  // namespace cz
