// residency.h -- the resident-weight table of libdmc_hip and its policy.
//
// The reference keeps every bf16 weight it has seen resident on the GPU,
// keyed by content, up to 2048 entries, and starts over when the cap is hit
// (GpuCtx, compiler/src/gpu.rs:259-280).  Here the same table also answers an
// out-of-memory (drop what can be dropped, retry once) and an optional byte
// cap, and it distinguishes two kinds of entries:
//   * cached: made resident on first sight by a drop-in call; any eviction
//     may free it (the next call with the same bytes uploads them again);
//   * pinned: made resident by dmc_hip_register_weight, which hands its
//     device address to the caller; an eviction never frees it, only
//     release_all (dmc_hip_release_weights) does, so that address stays valid
//     until the caller releases it.  A pinned entry remembers the host
//     addresses it was registered from (`registered`), for callers that may
//     keep only registered operands resident (the f32 route).
// No HIP here: device allocation and freeing come in as callbacks, so the
// policy is tested on the CPU (tests/residency_test.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <unordered_map>
#include <vector>

namespace dmc {

struct WeightKey {
    uint64_t a, b;
    int64_t bytes;
    bool operator==(const WeightKey &o) const { return a == o.a && b == o.b && bytes == o.bytes; }
};

struct WeightKeyHash {
    size_t operator()(const WeightKey &k) const { return (size_t)(k.a ^ (k.b << 1)); }
};

class Residency {
  public:
    // alloc(&p, bytes) returns 0, kOom (out of memory) or another nonzero
    // code, which is passed through; free_fn(p) releases an allocation.
    // drain() runs before anything is freed (the device may still read it).
    static constexpr int kOom = 1;
    using AllocFn = std::function<int(void **, size_t)>;
    using FreeFn = std::function<int(void *)>;
    using DrainFn = std::function<int()>;

    Residency(size_t max_entries, AllocFn alloc, FreeFn free_fn, DrainFn drain)
        : max_entries_(max_entries), alloc_(std::move(alloc)), free_(std::move(free_fn)), drain_(std::move(drain)) {}

    // The device copy of `key`, or nullptr.  A pinned lookup pins the entry
    // and records `host` as an address it was registered from.
    void *find(const WeightKey &key, bool pin = false, const void *host = nullptr) {
        auto it = map_.find(key);
        if (it == map_.end()) return nullptr;
        if (pin) {
            if (!it->second.pinned) {
                it->second.pinned = true;
                pinned_bytes_ += it->second.bytes;
                ++pinned_count_;
            }
            note_host(it->second, host);
        }
        return it->second.p;
    }

    // Was `key` pinned by a registration from host address `host`?  (A
    // registration is the caller's promise that those bytes stay unchanged
    // while resident; content alone, sampled, is no such promise.)
    bool registered(const WeightKey &key, const void *host) const {
        auto it = map_.find(key);
        if (it == map_.end() || !it->second.pinned || !host) return false;
        for (const void *h : it->second.hosts)
            if (h == host) return true;
        return false;
    }

    // Device memory for a new entry of `bytes` (plus `slack` bytes that are
    // not counted against the byte cap).  When the cached entries fill the
    // table, the new entry would pass `cap_bytes` (0: no cap), or the
    // allocation runs out of memory, every cached entry is freed once and the
    // request retried; pinned entries stay.  Returns 0, kOom (also when the
    // pinned entries alone leave no room under the cap) or the allocator's
    // code.
    int reserve(int64_t bytes, int64_t slack, int64_t cap_bytes, void **out) {
        *out = nullptr;
        bool evicted = false;
        if (map_.size() - pinned_count_ >= max_entries_ || over_cap(bytes, cap_bytes)) {
            int rc = evict_cached();
            if (rc) return rc;
            evicted = true;
            if (over_cap(bytes, cap_bytes)) return kOom;
        }
        int rc = alloc_(out, (size_t)(bytes + slack));
        if (rc == kOom && !evicted) {
            rc = evict_cached();
            if (rc) return rc;
            rc = alloc_(out, (size_t)(bytes + slack));
        }
        if (rc) *out = nullptr;
        return rc;
    }

    // Scratch memory needed while an entry is being built (the transposed
    // upload), with the same out-of-memory policy; released with free_fn.
    int reserve_scratch(size_t bytes, void **out) {
        *out = nullptr;
        int rc = alloc_(out, bytes);
        if (rc == kOom) {
            rc = evict_cached();
            if (rc) return rc;
            rc = alloc_(out, bytes);
        }
        if (rc) *out = nullptr;
        return rc;
    }

    void insert(const WeightKey &key, void *p, int64_t bytes, bool pinned, const void *host = nullptr) {
        Entry &e = map_[key] = Entry{p, bytes, pinned, {}};
        if (pinned) note_host(e, host);
        bytes_ += bytes;
        if (pinned) {
            pinned_bytes_ += bytes;
            ++pinned_count_;
        }
    }

    // Free every entry, pinned ones included.
    int release_all() {
        if (map_.empty()) return 0;
        int rc = drain_();
        if (rc) return rc;
        for (auto it = map_.begin(); it != map_.end();) {  // an entry leaves the table once freed
            rc = free_(it->second.p);
            if (rc) return rc;
            bytes_ -= it->second.bytes;
            if (it->second.pinned) {
                pinned_bytes_ -= it->second.bytes;
                --pinned_count_;
            }
            it = map_.erase(it);
        }
        return 0;
    }

    size_t count() const { return map_.size(); }
    int64_t bytes() const { return bytes_; }
    int64_t pinned_bytes() const { return pinned_bytes_; }
    size_t pinned_count() const { return pinned_count_; }

  private:
    struct Entry {
        void *p;
        int64_t bytes;
        bool pinned;
        std::vector<const void *> hosts;  // addresses a registration pinned it from
    };

    static void note_host(Entry &e, const void *host) {
        if (!host) return;
        for (const void *h : e.hosts)
            if (h == host) return;
        e.hosts.push_back(host);
    }

    bool over_cap(int64_t bytes, int64_t cap) const { return cap > 0 && bytes_ + bytes > cap; }

    int evict_cached() {
        if (map_.size() == pinned_count_) return 0;
        int rc = drain_();
        if (rc) return rc;
        for (auto it = map_.begin(); it != map_.end();) {
            if (it->second.pinned) {
                ++it;
                continue;
            }
            rc = free_(it->second.p);
            if (rc) return rc;
            bytes_ -= it->second.bytes;
            it = map_.erase(it);
        }
        return 0;
    }

    size_t max_entries_;
    AllocFn alloc_;
    FreeFn free_;
    DrainFn drain_;
    std::unordered_map<WeightKey, Entry, WeightKeyHash> map_;
    int64_t bytes_ = 0, pinned_bytes_ = 0;
    size_t pinned_count_ = 0;
};

}  // namespace dmc
