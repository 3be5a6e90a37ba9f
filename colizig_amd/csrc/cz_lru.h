// cz_lru.h - the expert pool's victim choice without a scan of every slot:
// the first free slot (lowest index), else the least recently used slot that
// the layer in flight does not pin (victimSlot, moe.zig:183-197, over one
// pool for every streamed layer).  A doubly linked list keeps the held slots
// in order of last use (filled or hit; the head is the least recent) and a
// bitmap the free ones, so the choice is the slot a scan comparing every
// held slot's last-use clock would pick.  Plain host C++ (no device code):
// the library's pool uses it, and the CPU sanitizer build checks it against
// that scan.
#pragma once

#include <cstdint>
#include <vector>

namespace cz {

class SlotLru {
  public:
    static constexpr uint32_t kNone = 0xffffffffu;

    // n slots, every one free
    void reset(uint32_t n) {
        n_ = n;
        head_ = tail_ = kNone;
        prev_.assign(n, kNone);
        next_.assign(n, kNone);
        held_.assign(n, 0);
        free_.assign((n + 63) / 64, ~0ull);
        if (n % 64) free_.back() = (1ull << (n % 64)) - 1;
    }

    // slot i holds an entry that was just used (filled or hit): the most recent
    void touch(uint32_t i) {
        if (held_[i]) {
            unlink(i);
        } else {
            held_[i] = 1;
            free_[i / 64] &= ~(1ull << (i % 64));
        }
        prev_[i] = tail_;
        next_[i] = kNone;
        if (tail_ != kNone) next_[tail_] = i;
        else head_ = i;
        tail_ = i;
    }

    // slot i holds nothing any more
    void release(uint32_t i) {
        if (!held_[i]) return;
        unlink(i);
        held_[i] = 0;
        free_[i / 64] |= 1ull << (i % 64);
    }

    // the first free slot, else the least recently used held slot for which
    // pinned(i) is false; n when every slot is held and pinned
    template <class Pinned>
    uint32_t victim(Pinned pinned) const {
        for (size_t w = 0; w < free_.size(); ++w)
            if (free_[w]) return (uint32_t)(64 * w + __builtin_ctzll(free_[w]));
        for (uint32_t i = head_; i != kNone; i = next_[i])
            if (!pinned(i)) return i;
        return n_;
    }

    bool held(uint32_t i) const { return held_[i] != 0; }

  private:
    void unlink(uint32_t i) {
        if (prev_[i] != kNone) next_[prev_[i]] = next_[i];
        else head_ = next_[i];
        if (next_[i] != kNone) prev_[next_[i]] = prev_[i];
        else tail_ = prev_[i];
        prev_[i] = next_[i] = kNone;
    }

    uint32_t n_ = 0, head_ = kNone, tail_ = kNone;
    std::vector<uint32_t> prev_, next_;
    std::vector<uint8_t> held_;
    std::vector<uint64_t> free_;  // bit i % 64 of word i / 64: slot i is free
};

}  // namespace cz
