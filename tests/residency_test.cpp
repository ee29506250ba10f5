// The resident-weight table's policy (demonic_amd/csrc/residency.h) on the
// CPU, with a fake device allocator: a pool of `cap` bytes that reports out
// of memory when full, and a log of every free.  Built and run by
// tests/test_residency.py; prints "ok" and exits 0 when every check holds.
#include "../demonic_amd/csrc/residency.h"

#include <cstdio>
#include <cstdlib>
#include <set>

namespace {

int failures = 0;
#define CHECK(cond)                                                  \
    do {                                                             \
        if (!(cond)) {                                               \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            ++failures;                                              \
        }                                                            \
    } while (0)

struct FakeDevice {
    size_t cap, used = 0;
    std::set<void *> live;
    std::set<void *> freed;
    int drains = 0;
    std::unordered_map<void *, size_t> size;
    int alloc(void **p, size_t bytes) {
        if (used + bytes > cap) return dmc::Residency::kOom;
        *p = std::malloc(bytes ? bytes : 1);
        live.insert(*p);
        size[*p] = bytes;
        used += bytes;
        return 0;
    }
    int release(void *p) {
        if (!live.count(p)) return -9;  // double or foreign free
        live.erase(p);
        freed.insert(p);
        used -= size[p];
        std::free(p);
        return 0;
    }
};

dmc::WeightKey key(uint64_t i, int64_t bytes) { return dmc::WeightKey{i, i * 7 + 1, bytes}; }

dmc::Residency table(FakeDevice &dev, size_t max_entries) {
    return dmc::Residency(
        max_entries, [&dev](void **p, size_t b) { return dev.alloc(p, b); },
        [&dev](void *p) { return dev.release(p); }, [&dev]() { ++dev.drains; return 0; });
}

// Add entry i of `bytes` through the table's policy; returns the address or nullptr.
void *add(dmc::Residency &t, uint64_t i, int64_t bytes, bool pin, int64_t cap = 0, int *rc_out = nullptr) {
    void *p = nullptr;
    const int rc = t.reserve(bytes, 16, cap, &p);
    if (rc_out) *rc_out = rc;
    if (rc) return nullptr;
    t.insert(key(i, bytes), p, bytes, pin);
    return p;
}

}  // namespace

int main() {
    {  // the entry cap evicts cached entries only; a pinned address survives
        FakeDevice dev{1 << 30};
        auto t = table(dev, 4);
        void *pinned = add(t, 100, 1000, true);
        for (uint64_t i = 0; i < 4; ++i) CHECK(add(t, i, 1000, false));
        CHECK(t.count() == 5 && t.pinned_count() == 1);
        void *fifth = add(t, 4, 1000, false);  // cached entries fill the table: all of them go
        CHECK(fifth != nullptr);
        CHECK(t.count() == 2 && t.bytes() == 2000);
        CHECK(dev.live.count(pinned) == 1 && dev.freed.count(pinned) == 0);
        CHECK(t.find(key(100, 1000)) == pinned);
        CHECK(t.find(key(0, 1000)) == nullptr);
        CHECK(dev.drains == 1);  // the device is drained before anything is freed
    }
    {  // out of memory: cached entries released once, pinned kept, then retried
        FakeDevice dev{10000};
        auto t = table(dev, 2048);
        void *pinned = add(t, 1, 3000, true);
        CHECK(add(t, 2, 3000, false) && add(t, 3, 3000, false));
        void *big = add(t, 4, 5000, false);  // 9032 used + 5016 > 10000: evict 2 and 3, retry
        CHECK(big != nullptr);
        CHECK(t.find(key(2, 3000)) == nullptr && t.find(key(3, 3000)) == nullptr);
        CHECK(t.find(key(1, 3000)) == pinned && dev.live.count(pinned) == 1);
        int rc = 0;
        CHECK(add(t, 5, 9000, false, 0, &rc) == nullptr);  // cannot fit even after eviction
        CHECK(rc == dmc::Residency::kOom);
        CHECK(t.find(key(1, 3000)) == pinned && dev.live.count(pinned) == 1);
    }
    {  // the byte cap (DMC_HIP_RESIDENT_CAP): pinned bytes count against it
        FakeDevice dev{1 << 30};
        auto t = table(dev, 2048);
        int rc = 0;
        CHECK(add(t, 1, 600, true, 1000));
        CHECK(add(t, 2, 300, false, 1000));
        CHECK(add(t, 3, 300, false, 1000));  // 1200 > 1000: the cached 300 goes
        CHECK(t.count() == 2 && t.bytes() == 900);
        CHECK(add(t, 4, 500, false, 1000, &rc) == nullptr && rc == dmc::Residency::kOom);
        CHECK(t.count() == 1 && t.bytes() == 600 && t.pinned_bytes() == 600);  // the cached one was dropped trying
    }
    {  // a later pinned lookup pins a cached entry; release_all frees everything once
        FakeDevice dev{1 << 30};
        auto t = table(dev, 2);
        void *a = add(t, 1, 100, false);
        CHECK(t.find(key(1, 100), true) == a && t.pinned_count() == 1);
        CHECK(add(t, 2, 100, false) && add(t, 3, 100, false));
        CHECK(add(t, 4, 100, false));  // two cached fill the table: they go, the pinned one stays
        CHECK(t.find(key(1, 100)) == a && dev.live.count(a) == 1);
        CHECK(t.release_all() == 0);
        CHECK(t.count() == 0 && t.bytes() == 0 && t.pinned_bytes() == 0 && t.pinned_count() == 0);
        CHECK(dev.live.empty());
    }
    {  // a scratch allocation under memory pressure evicts cached entries, not pinned
        FakeDevice dev{4000};
        auto t = table(dev, 2048);
        void *pinned = add(t, 1, 1000, true);
        CHECK(add(t, 2, 1000, false));
        void *s = nullptr;
        CHECK(t.reserve_scratch(2500, &s) == 0 && s != nullptr);
        CHECK(t.find(key(2, 1000)) == nullptr && t.find(key(1, 1000)) == pinned);
        dev.release(s);
    }
    {  // registered(): pinned entries only, and only from the addresses that pinned them
        FakeDevice dev{1 << 30};
        auto t = table(dev, 2048);
        int h1 = 0, h2 = 0, h3 = 0;
        void *p = nullptr;
        CHECK(t.reserve(100, 16, 0, &p) == 0);
        t.insert(key(1, 100), p, 100, true, &h1);
        CHECK(t.registered(key(1, 100), &h1));
        CHECK(!t.registered(key(1, 100), &h2) && !t.registered(key(1, 100), nullptr));
        CHECK(t.find(key(1, 100), true, &h2) == p);  // the same bytes registered from a second address
        CHECK(t.registered(key(1, 100), &h1) && t.registered(key(1, 100), &h2));
        CHECK(add(t, 2, 100, false));  // cached: found by content, never "registered"
        CHECK(t.find(key(2, 100)) != nullptr && !t.registered(key(2, 100), &h3));
        CHECK(t.find(key(2, 100), false, &h3) != nullptr && !t.registered(key(2, 100), &h3));
        CHECK(!t.registered(key(9, 100), &h1));
    }
    if (failures) return 1;
    std::printf("ok\n");
    return 0;
}
