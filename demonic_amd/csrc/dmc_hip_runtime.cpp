// dmc_hip_runtime.cpp -- host runtime and C ABI of libdmc_hip (include/dmc_hip.h).
//
// Plays the role of the reference's GpuCtx + gpu_run (compiler/src/gpu.rs:186-660)
// on a discrete MI355X instead of unified Apple memory:
//   * one HIP stream (default priority) carries every copy and launch, so all
//     device-side ordering is stream order;
//   * weights become resident in HBM on first sight, keyed by content (the
//     decode loop hands the same bytes over at fresh arena addresses every step,
//     gpu.rs:195-199), or ahead of time through dmc_hip_register_weight;
//   * activations and outputs cross PCIe through pinned staging buffers; while
//     deferred calls are pending each call takes its own slice of the staging
//     buffers, and the next synchronous call or flush copies the pending
//     outputs to their destinations (the deferred protocol of gpu.rs:439-474,
//     with the overlap guard of gpu.rs:491-499).  A deferred call's kernels
//     write y to device memory at its slice's offset; one copy kernel moves
//     every pending y to pinned staging when they are materialized;
//   * no CPU arithmetic anywhere: a device failure is reported (int entries)
//     or fatal (the void drop-in entries), never silently recomputed.
#include "../../include/dmc_hip.h"
#include "gemv_launch.h"
#include "npz_ingress.h"
#include "residency.h"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string t_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

[[noreturn]] void fatal(const char *where) {
    fprintf(stderr, "dmc_hip: fatal: %s: %s\n", where, t_err.c_str());
    fflush(stderr);
    abort();
}

bool env_flag(const char *name) {
    const char *v = getenv(name);
    return v && *v && strcmp(v, "0") != 0;
}

// ---- content key for resident weights --------------------------------------
//
// Byte length plus 256 evenly spread 8-byte samples (the reference's density,
// gpu.rs:334-358), the last word and the trailing bytes, each mixed with its
// index into two independent 64-bit lanes, the first through the splitmix64
// finalizer.  The sample positions advance without a division, and the
// finalizer chain is split four ways (recombined at the end), so the cost is
// the scattered host reads, not a serial chain of multiplies.
using Key = dmc::WeightKey;

inline uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ULL;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebULL;
    z ^= z >> 31;
    return z;
}

constexpr uint64_t kKeySamples = 256;

Key content_key(const void *ptr, int64_t bytes) {
    const unsigned char *p = static_cast<const unsigned char *>(ptr);
    uint64_t a[4];
    for (int j = 0; j < 4; ++j) a[j] = mix64((uint64_t)bytes ^ (0x6a09e667f3bcc908ULL + (uint64_t)j));
    uint64_t b = mix64((uint64_t)bytes + 0xbb67ae8584caa73bULL);
    const uint64_t words = (uint64_t)bytes / 8;
    uint64_t n = 0;
    auto fold = [&](uint64_t idx, uint64_t v) {
        a[n & 3] = mix64(a[n & 3] ^ v ^ (idx * 0x9e3779b97f4a7c15ULL));
        b = (b ^ v) * 0x100000001b3ULL + idx + 1;
        ++n;
    };
    if (words > 0) {
        // sample i at word floor(i * words / S)
        const uint64_t S = words < kKeySamples ? words : kKeySamples, q = words / S, r = words % S;
        uint64_t idx = 0, acc = 0;
        for (uint64_t i = 0; i < S; ++i) {
            uint64_t v;
            memcpy(&v, p + idx * 8, 8);
            fold(idx, v);
            idx += q;
            acc += r;
            if (acc >= S) {
                acc -= S;
                ++idx;
            }
        }
        uint64_t v;
        memcpy(&v, p + (words - 1) * 8, 8);
        fold(words - 1, v);
    }
    uint64_t tail = 0;
    for (int64_t i = (int64_t)words * 8; i < bytes; ++i) tail = (tail << 8) | p[i];
    fold(words, tail);
    return Key{mix64(a[0] ^ mix64(a[1] ^ mix64(a[2] ^ mix64(a[3])))), mix64(b), bytes};
}

// ---- context ----------------------------------------------------------------

struct Buf {
    void *p = nullptr;
    size_t cap = 0;
    char *dev = nullptr;  // pinned staging: the device address of p
};

struct Pending {
    const void *src;  // pinned staging
    void *dst;        // caller's out
    size_t bytes;
    bool dev;         // y is in Ctx::dyd at src's staging offset until materialized
};

// DMC_HIP_TIME=1 accounting, after the reference's DMC_GPU_TIME (gpu.rs:45-96):
// host phases per call, the device's view of each synchronous call from HIP
// events (x upload, kernels), and per-shape buckets with the GB/s the kernels
// reached on the weight bytes.
struct ShapeStats {
    int64_t k, n, batch;
    uint64_t calls, wait_ns, gpu_ns;
};

struct Stats {
    uint64_t calls = 0, stage_ns = 0, key_ns = 0, upload_ns = 0, enqueue_ns = 0, wait_ns = 0,
             readback_ns = 0, uploads = 0, gpu_x_ns = 0, gpu_k_ns = 0, timed = 0;
    std::vector<ShapeStats> shapes;
};

struct Ctx {
    bool tried = false, ok = false;
    int device = 0;
    int cus = 0;
    std::string arch;
    hipStream_t stream = nullptr;
    dmc::Residency *weights = nullptr;  // resident weights by content key (created at init)
    Buf dx, dy, ws;         // device scratch (reuse is stream-ordered)
    Buf dwf, dwt;           // f32 route: a weight staged for one call, and its transpose
    int live_graphs = 0;    // executable graphs not yet destroyed
    std::vector<void *> retired_ws;  // outgrown workspaces a live graph may still use
    Buf hx, hy;             // pinned staging
    size_t hx_off = 0, hy_off = 0;
    Buf dyd;                // deferred calls' y, in device memory at their hy staging offsets
    std::vector<Pending> pending;
    void *dummy = nullptr;  // non-null device address for zero-byte weights
    void *sink = nullptr;   // probe output words
    std::vector<void *> ingress;        // pinned chunks for .npz ingress, kIngressChunk bytes each
    std::vector<hipEvent_t> ingress_ev; // one per chunk: its last copy to the device
    bool timing = false;
    uint64_t time_every = 0;  // DMC_HIP_TIME=N > 1: a stats line every N calls
    bool x_kernel = false;  // DMC_HIP_X_KERNEL: upload x with a kernel instead of a copy-engine transfer
    size_t y_direct_max = 0;  // largest y a kernel writes straight to pinned staging (DMC_HIP_Y_DIRECT_MAX)
    size_t x_direct_max = 0;  // largest x a kernel reads straight from pinned staging (DMC_HIP_X_DIRECT_MAX)
    hipEvent_t tev[3] = {};  // DMC_HIP_TIME: before x, before the kernels, after them
    // the no-allocation entry's fixed scratch, resolved per device at set-up
    // (this library drives one device, `device`); null if that failed
    std::unordered_map<int, void *> noalloc_scratch;
    std::string noalloc_err;
    Stats st;
};

std::mutex g_mu;
Ctx &ctx() {
    static Ctx *c = new Ctx;  // never destroyed: no HIP calls during exit
    return *c;
}

const int kMaxResident = 2048;  // gpu.rs:266
const size_t kDirectYBytes = 256 << 10;  // largest y a kernel writes straight to pinned staging
const size_t kDirectXBytes = 64 << 10;   // largest x a kernel reads straight from pinned staging

int hip_fail(hipError_t e, const char *what) {
    return fail(e == hipErrorOutOfMemory ? DMC_HIP_ENOMEM : DMC_HIP_EDEVICE, "%s: %s (%d)", what,
                hipGetErrorString(e), (int)e);
}

#define HIP_TRY(expr, what)                                   \
    do {                                                      \
        hipError_t e_ = (expr);                               \
        if (e_ != hipSuccess) return hip_fail(e_, what);      \
    } while (0)

// Caller holds g_mu.  Returns DMC_HIP_OK when the device is usable.
int ensure_init() {
    Ctx &c = ctx();
    if (c.tried) {
        if (!c.ok) return DMC_HIP_ENODEV;
        HIP_TRY(hipSetDevice(c.device), "hipSetDevice");
        return DMC_HIP_OK;
    }
    c.tried = true;
    if (env_flag("DMC_HIP_DISABLE")) return fail(DMC_HIP_ENODEV, "disabled by DMC_HIP_DISABLE");
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
        return fail(DMC_HIP_ENODEV, "no HIP device");
    const char *dv = getenv("DMC_HIP_DEVICE");
    c.device = (dv && *dv) ? atoi(dv) : 0;
    if (c.device < 0 || c.device >= count) return fail(DMC_HIP_ENODEV, "DMC_HIP_DEVICE out of range");
    if (hipSetDevice(c.device) != hipSuccess) return fail(DMC_HIP_ENODEV, "hipSetDevice failed");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, c.device) != hipSuccess)
        return fail(DMC_HIP_ENODEV, "hipGetDeviceProperties failed");
    c.arch = prop.gcnArchName;
    const size_t colon = c.arch.find(':');
    if (colon != std::string::npos) c.arch.resize(colon);
    if (c.arch != "gfx950")
        return fail(DMC_HIP_ENODEV, "device %d is %s; this library is built for gfx950 only",
                    c.device, c.arch.c_str());
    c.cus = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking) != hipSuccess)
        return fail(DMC_HIP_ENODEV, "hipStreamCreate failed");
    if (hipMalloc(&c.dummy, 256) != hipSuccess) return fail(DMC_HIP_ENODEV, "hipMalloc failed");
    c.weights = new dmc::Residency(
        kMaxResident,
        [](void **p, size_t bytes) -> int {
            const hipError_t e = hipMalloc(p, bytes);
            if (e == hipErrorOutOfMemory) {
                (void)hipGetLastError();
                return dmc::Residency::kOom;
            }
            return e == hipSuccess ? DMC_HIP_OK : hip_fail(e, "hipMalloc(weight)");
        },
        [](void *p) -> int {
            const hipError_t e = hipFree(p);
            return e == hipSuccess ? DMC_HIP_OK : hip_fail(e, "hipFree(weight)");
        },
        []() -> int {
            const hipError_t e = hipStreamSynchronize(ctx().stream);
            return e == hipSuccess ? DMC_HIP_OK : hip_fail(e, "hipStreamSynchronize");
        });
    {
        void *p = nullptr;
        const hipError_t e = dmc::noalloc_scratch_resolve(&p);
        if (e == hipSuccess && p) {
            c.noalloc_scratch[c.device] = p;
        } else {
            (void)hipGetLastError();
            c.noalloc_err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
        }
    }
    c.timing = env_flag("DMC_HIP_TIME");
    if (c.timing) c.time_every = (uint64_t)std::max(0LL, atoll(getenv("DMC_HIP_TIME")));
    for (hipEvent_t &ev : c.tev)
        if (c.timing && hipEventCreate(&ev) != hipSuccess) c.timing = false;
    c.x_kernel = env_flag("DMC_HIP_X_KERNEL");
    {
        const char *v = getenv("DMC_HIP_Y_DIRECT_MAX");
        c.y_direct_max = v && *v ? (size_t)std::max(0LL, atoll(v)) : kDirectYBytes;
        v = getenv("DMC_HIP_X_DIRECT_MAX");
        c.x_direct_max = v && *v ? (size_t)std::max(0LL, atoll(v)) : kDirectXBytes;
    }
    c.ok = true;
    return DMC_HIP_OK;
}

// Grow a device scratch buffer; in-flight work may still read the old one, so
// drain the stream before freeing it.
int ensure_dev(Buf &b, size_t need) {
    if (need <= b.cap) return DMC_HIP_OK;
    Ctx &c = ctx();
    size_t cap = b.cap ? b.cap : (size_t)1 << 20;
    while (cap < need) cap *= 2;
    if (b.p) {
        HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
        // A captured graph holds the workspace's address: while any graph
        // lives, an outgrown workspace stays allocated (freed with the last
        // graph), so a later replay never touches freed memory.
        if (&b == &c.ws && c.live_graphs > 0) {
            c.retired_ws.push_back(b.p);
        } else {
            HIP_TRY(hipFree(b.p), "hipFree");
        }
        b.p = nullptr;
        b.cap = 0;
    }
    HIP_TRY(hipMalloc(&b.p, cap), "hipMalloc(scratch)");
    b.cap = cap;
    return DMC_HIP_OK;
}

int flush_locked();

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Reserve `need` bytes of pinned staging at a 256-byte aligned bump offset.
// The caller has already materialized pending work if the reservation does
// not fit behind it (see run_host), so a full buffer here has nothing pending
// in it and may restart at 0 or be replaced.
// A slice of pinned staging for `need` bytes: its host address in *out and,
// when dev_out is given, the same bytes' device address (kernels write the
// y staging directly, so it is allocated coherent: the stores cross PCIe
// uncached and are visible to the host once the stream has synchronized).
int stage(Buf &b, size_t &off, size_t need, unsigned flags, char **out, char **dev_out = nullptr) {
    size_t at = align256(off);
    if (at + need > b.cap) {
        Ctx &c = ctx();
        at = 0;
        if (need > b.cap) {
            HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
            if (b.p) HIP_TRY(hipHostFree(b.p), "hipHostFree");
            b.p = nullptr;
            b.dev = nullptr;
            b.cap = 0;
            size_t cap = (size_t)1 << 20;
            while (cap < need) cap *= 2;
            HIP_TRY(hipHostMalloc(&b.p, cap, flags), "hipHostMalloc(staging)");
            b.cap = cap;
            void *d = nullptr;
            HIP_TRY(hipHostGetDevicePointer(&d, b.p, 0), "hipHostGetDevicePointer(staging)");
            b.dev = static_cast<char *>(d);
        }
    }
    *out = static_cast<char *>(b.p) + at;
    if (dev_out) *dev_out = b.dev + at;
    off = at + need;
    return DMC_HIP_OK;
}

int release_weights_locked() { return ctx().weights->release_all(); }

// The residency policy's answer as a library code.
int residency_rc(int rc, int64_t bytes) {
    if (rc == dmc::Residency::kOom)
        return fail(DMC_HIP_ENOMEM, "no device memory for a %lld-byte weight (after releasing the cached ones)",
                    (long long)bytes);
    return rc;
}

// Device copy of the host weight [host, host+bytes), uploading on a miss.
// With t_rows > 0 the host bytes hold t_batch matrices W [t_rows, t_cols],
// one after another, and the device copy holds each one's W^T [t_cols,
// t_rows] in the same order: the drop-in x @ W keeps its weight in the
// row-dot layout, whose kernel needs one launch where the column-stream
// layout needs two.  `elem` is the element size (2: bf16, 4: f32) the
// transpose moves.  The layout, the column and matrix counts and the element
// size are part of the key, so the same bytes used through another entry or
// shape get their own copy.  `pin`:
// the caller keeps the device address (dmc_hip_register_weight), so no
// eviction may free this entry (residency.h).  DMC_HIP_RESIDENT_CAP (bytes)
// caps what may stay resident.
int resident(const void *host, int64_t bytes, void **dev, int64_t t_rows = 0, int64_t t_cols = 0,
             bool pin = false, int elem = 2, int64_t t_batch = 1) {
    Ctx &c = ctx();
    if (bytes <= 0) {
        *dev = c.dummy;
        return DMC_HIP_OK;
    }
    auto t0 = std::chrono::steady_clock::now();
    Key key = content_key(host, bytes);
    if (t_rows > 0)
        key.b = mix64(key.b ^ 0x7472616e73706f73ULL ^ ((uint64_t)t_cols * 0x9E3779B97F4A7C15ULL) ^
                      (elem == 4 ? 0x6633320000000000ULL : 0) ^ ((uint64_t)(t_batch - 1) << 40));
    auto t1 = std::chrono::steady_clock::now();
    c.st.key_ns += (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count();
    if (void *hit = c.weights->find(key, pin, pin ? host : nullptr)) {
        *dev = hit;
        return DMC_HIP_OK;
    }
    const char *cap_s = getenv("DMC_HIP_RESIDENT_CAP");
    const int64_t cap = cap_s && *cap_s ? strtoll(cap_s, nullptr, 10) : 0;
    void *d = nullptr, *raw = nullptr;
    int rc = residency_rc(c.weights->reserve(bytes, dmc::kWeightSlack, cap, &d), bytes);
    if (rc) return rc;
    if (t_rows > 0 && (rc = residency_rc(c.weights->reserve_scratch((size_t)bytes, &raw), bytes))) {
        (void)hipFree(d);
        return rc;
    }
    hipError_t e = hipMemcpyAsync(raw ? raw : d, host, (size_t)bytes, hipMemcpyHostToDevice, c.stream);
    const size_t t_bytes = (size_t)(t_rows * t_cols) * (size_t)elem;  // one matrix
    for (int64_t z = 0; e == hipSuccess && raw && z < t_batch; ++z) {
        const char *src = static_cast<const char *>(raw) + z * t_bytes;
        char *dst = static_cast<char *>(d) + z * t_bytes;
        e = elem == 4 ? dmc::launch_transpose_f32(reinterpret_cast<const float *>(src), reinterpret_cast<float *>(dst),
                                                  t_rows, t_cols, c.stream)
                      : dmc::launch_transpose_bf16(reinterpret_cast<const uint16_t *>(src),
                                                   reinterpret_cast<uint16_t *>(dst), t_rows, t_cols, c.stream);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c.stream);
    if (raw) (void)hipFree(raw);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "weight upload");
    }
    c.weights->insert(key, d, bytes, pin, pin ? host : nullptr);
    c.st.uploads++;
    c.st.upload_ns += (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                          std::chrono::steady_clock::now() - t1)
                          .count();
    if (env_flag("DMC_HIP_DEBUG"))
        fprintf(stderr, "[hip] upload #%zu %lld MB%s%s\n", c.weights->count(), (long long)(bytes >> 20),
                raw ? " (transposed)" : "", pin ? " (pinned)" : "");
    *dev = d;
    return DMC_HIP_OK;
}

// Pending outputs still in device memory (deferred calls) go to their pinned
// staging slices in one copy kernel on the stream: the slices are bump
// allocated, so [first, last end) covers them all, at the same offsets in
// Ctx::dyd.  Kernels that write y straight to pinned memory (synchronous
// calls) run ~4 us longer on C2 than ones that write it to HBM: their last
// stores cross PCIe while the workgroups hold their slots; a copy-engine
// transfer per call cost more still (61 against 27 us per deferred call).
int copy_pending_out() {
    Ctx &c = ctx();
    size_t lo = SIZE_MAX, hi = 0;
    for (const Pending &q : c.pending) {
        if (!q.dev) continue;
        const size_t at = (size_t)(static_cast<const char *>(q.src) - static_cast<const char *>(c.hy.p));
        lo = std::min(lo, at);
        hi = std::max(hi, at + q.bytes);
    }
    if (hi <= lo) return DMC_HIP_OK;
    HIP_TRY(dmc::launch_copy_words(c.hy.dev + lo, static_cast<const char *>(c.dyd.p) + lo, (int64_t)(hi - lo),
                                   c.stream),
            "deferred y copy");
    return DMC_HIP_OK;
}

int flush_locked() {
    Ctx &c = ctx();
    if (!c.tried || !c.ok) return DMC_HIP_OK;
    if (!c.pending.empty()) {
        int rc = copy_pending_out();
        if (rc) return rc;
        HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
        for (const Pending &p : c.pending) memcpy(p.dst, p.src, p.bytes);
        c.pending.clear();
    }
    c.hx_off = 0;
    c.hy_off = 0;
    return DMC_HIP_OK;
}

bool overlaps_pending(const void *p, size_t bytes) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(p);
    for (const Pending &q : ctx().pending) {
        const uintptr_t d0 = reinterpret_cast<uintptr_t>(q.dst);
        if (a0 < d0 + q.bytes && d0 < a0 + bytes) return true;
    }
    return false;
}

int64_t ns_since(std::chrono::steady_clock::time_point t) {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t)
        .count();
}

void stats_line(int64_t k, int64_t n) {
    Ctx &c = ctx();
    Stats &s = c.st;
    if (!c.timing) return;
    // The lm-head GEMV (the only n >= 100k call) closes a decode step, the
    // delimiter of the reference's DMC_GPU_TIME line (gpu.rs:681-683); with
    // DMC_HIP_TIME=N (N > 1) a line every N calls instead.
    if (c.time_every > 1 ? s.calls % c.time_every != 0 : (n < 100000 && s.calls % 1024 != 0)) return;
    fprintf(stderr,
            "[hip] step: calls=%llu stage=%lluus key=%lluus upload=%lluus(%llu) enqueue=%lluus "
            "wait=%lluus (gpu x=%lluus kernels=%lluus over %llu timed) readback=%lluus (last k=%lld n=%lld)\n",
            (unsigned long long)s.calls, (unsigned long long)(s.stage_ns / 1000),
            (unsigned long long)(s.key_ns / 1000), (unsigned long long)(s.upload_ns / 1000),
            (unsigned long long)s.uploads, (unsigned long long)(s.enqueue_ns / 1000),
            (unsigned long long)(s.wait_ns / 1000), (unsigned long long)(s.gpu_x_ns / 1000),
            (unsigned long long)(s.gpu_k_ns / 1000), (unsigned long long)s.timed,
            (unsigned long long)(s.readback_ns / 1000), (long long)k, (long long)n);
    for (const ShapeStats &b : s.shapes) {
        const double bytes = (double)b.calls * 2.0 * (double)b.k * (double)b.n * (double)b.batch;
        fprintf(stderr, "[hip]   k=%lld n=%lld b=%lld: %llu calls wait=%lluus gpu=%lluus  %.1f GB/s\n",
                (long long)b.k, (long long)b.n, (long long)b.batch, (unsigned long long)b.calls,
                (unsigned long long)(b.wait_ns / 1000), (unsigned long long)(b.gpu_ns / 1000),
                b.gpu_ns ? bytes / (double)b.gpu_ns : 0.0);
    }
    s = Stats{};
}

// One synchronous call's device times (events recorded around its work; x_copied:
// the x upload had events of its own).
void stats_call(int64_t k, int64_t n, int64_t batch, uint64_t wait_ns, bool x_copied) {
    Ctx &c = ctx();
    float x_ms = 0.0f, k_ms = 0.0f;
    if ((x_copied && hipEventElapsedTime(&x_ms, c.tev[0], c.tev[1]) != hipSuccess) ||
        hipEventElapsedTime(&k_ms, c.tev[1], c.tev[2]) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    Stats &s = c.st;
    const uint64_t gx = (uint64_t)(x_ms * 1e6f), gk = (uint64_t)(k_ms * 1e6f);
    s.gpu_x_ns += gx;
    s.gpu_k_ns += gk;
    s.timed++;
    for (ShapeStats &b : s.shapes) {
        if (b.k == k && b.n == n && b.batch == batch) {
            b.calls++;
            b.wait_ns += wait_ns;
            b.gpu_ns += gk;
            return;
        }
    }
    s.shapes.push_back(ShapeStats{k, n, batch, 1, wait_ns, gk});
}

bool valid_dims(int64_t m, int64_t k, int64_t n) {
    return m >= 0 && k >= 0 && n >= 0 && m <= INT32_MAX && k <= INT32_MAX && n <= INT32_MAX;
}

// Shared host-pointer path of every drop-in entry.
int run_host(bool rd, const float *l, const uint16_t *r, float *out, int64_t m, int64_t k,
             int64_t n, int64_t batch, int64_t ls, int64_t rs, bool defer) {
    if (m < 0 || k < 0 || n < 0 || batch < 0 || ls < 0 || rs < 0)
        return fail(DMC_HIP_EINVAL, "negative size or stride (m=%lld k=%lld n=%lld batch=%lld)",
                    (long long)m, (long long)k, (long long)n, (long long)batch);
    if (m == 0 || n == 0 || batch == 0) return DMC_HIP_OK;
    if (!valid_dims(m, k, n)) return fail(DMC_HIP_EINVAL, "dimension beyond int32");
    if (!out || (k > 0 && (!l || !r))) return fail(DMC_HIP_EINVAL, "null pointer");
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    const size_t x_bytes = (size_t)((batch - 1) * ls + m * k) * 4;
    const size_t w_bytes = (size_t)((batch - 1) * rs + k * n) * 2;
    const size_t y_bytes = (size_t)(batch * m * n) * 4;
    if (!c.pending.empty() &&
        (overlaps_pending(l, x_bytes) || overlaps_pending(r, w_bytes) || overlaps_pending(out, y_bytes))) {
        rc = flush_locked();
        if (rc) return rc;
    }
    // Deferred calls each keep their own staging slices until materialized.
    // If this call's slices do not fit behind them, materialize them first.
    if (!c.pending.empty() &&
        (align256(c.hx_off) + x_bytes > c.hx.cap || align256(c.hy_off) + y_bytes > c.hy.cap)) {
        rc = flush_locked();
        if (rc) return rc;
    }
    auto t0 = std::chrono::steady_clock::now();
    char *hx = nullptr, *hx_dev = nullptr, *hy = nullptr, *hy_dev = nullptr;
    if ((rc = stage(c.hx, c.hx_off, x_bytes, hipHostMallocDefault, &hx, &hx_dev))) return rc;
    if ((rc = stage(c.hy, c.hy_off, y_bytes, hipHostMallocCoherent, &hy, &hy_dev))) return rc;
    // A small y is written by the kernel straight into its pinned staging
    // slice (saves a device-to-host copy launch, ~4 us of a ~45 us call); a
    // large one goes to device memory and crosses PCIe as one copy, which
    // beats scattered stores.
    const bool y_direct = y_bytes <= c.y_direct_max;
    // A small x can likewise be read by the kernels straight from its staging
    // slice (coarse-grained pinned memory: the host's writes are visible to a
    // kernel launched after them, and the GPU's caches serve the re-reads).
    const bool x_direct = x_bytes <= c.x_direct_max;
    if (x_bytes) memcpy(hx, l, x_bytes);
    if (!x_direct && (rc = ensure_dev(c.dx, x_bytes ? x_bytes : 4))) return rc;
    // A deferred call's y goes to device memory at its staging offset (one
    // copy for all of them when they are materialized, copy_pending_out).
    // The buffer keeps the staging's size; the staging only grows while
    // nothing is pending (see above), so no pending y is ever moved.
    if (defer && (rc = ensure_dev(c.dyd, c.hy.cap))) return rc;
    if (!y_direct && !defer && (rc = ensure_dev(c.dy, y_bytes))) return rc;
    float *const ydst = static_cast<float *>(
        defer      ? static_cast<void *>(static_cast<char *>(c.dyd.p) + (hy - static_cast<char *>(c.hy.p)))
        : y_direct ? static_cast<void *>(hy_dev)
                   : c.dy.p);
    const float *const xsrc = static_cast<const float *>(x_direct ? static_cast<void *>(hx_dev) : c.dx.p);
    const bool timed = c.timing && !defer;
    if (timed && !x_direct) HIP_TRY(hipEventRecord(c.tev[0], c.stream), "hipEventRecord");
    if (x_bytes && !x_direct) {
        if (c.x_kernel) {
            HIP_TRY(dmc::launch_copy_words(c.dx.p, hx_dev, (int64_t)x_bytes, c.stream), "x upload");
        } else {
            HIP_TRY(hipMemcpyAsync(c.dx.p, hx, x_bytes, hipMemcpyHostToDevice, c.stream), "x upload");
        }
    }
    c.st.stage_ns += ns_since(t0);

    // x @ W with one slice runs on the row-dot kernel over a transposed
    // resident copy (DMC_HIP_CS_LAYOUT=1 keeps the column-stream kernels).
    // So does a batch of slices that share one activation row (ls = 0, m =
    // 1) over weights one after another (rs = k n), per-head projections of
    // one token: the slices' transposes, stacked, are one weight [batch n,
    // k] whose row-dot GEMV writes y [batch, n] in one launch.  Other batched
    // calls keep the column-stream kernels, whose one launch covers every
    // slice.
    const bool stacked = batch > 1 && ls == 0 && m == 1 && rs == k * n && k > 0 && batch * n <= INT32_MAX;
    const bool cs_as_rd = !rd && (batch == 1 || stacked) && !env_flag("DMC_HIP_CS_LAYOUT");
    const int64_t nrd = cs_as_rd ? batch * n : n;  // row-dot output rows
    void *dw = nullptr;
    if ((rc = cs_as_rd ? resident(r, (int64_t)w_bytes, &dw, k, n, false, 2, batch) : resident(r, (int64_t)w_bytes, &dw)))
        return rc;

    auto t1 = std::chrono::steady_clock::now();
    if (timed) HIP_TRY(hipEventRecord(c.tev[1], c.stream), "hipEventRecord");
    hipError_t e;
    if (rd || cs_as_rd) {
        dmc::RdProblem p{static_cast<const uint16_t *>(dw), k, xsrc, k, ydst, nrd, m, k, nrd};
        const dmc::RdPlan pl = dmc::plan_rd(p, c.cus);
        if ((rc = ensure_dev(c.ws, pl.workspace_bytes))) return rc;
        e = dmc::launch_rd(p, pl, pl.workspace_bytes ? c.ws.p : nullptr, c.stream);
    } else {
        dmc::CsProblem p{static_cast<const uint16_t *>(dw), xsrc, ydst, m, k, n, batch, ls, rs};
        const dmc::CsPlan pl = dmc::plan_cs(p, c.cus);
        if ((rc = ensure_dev(c.ws, pl.workspace_bytes))) return rc;
        e = dmc::launch_cs(p, pl, c.ws.p, c.stream);
    }
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    if (!y_direct && !defer)
        HIP_TRY(hipMemcpyAsync(hy, c.dy.p, y_bytes, hipMemcpyDeviceToHost, c.stream), "y readback");
    if (timed) HIP_TRY(hipEventRecord(c.tev[2], c.stream), "hipEventRecord");
    c.st.enqueue_ns += ns_since(t1);
    c.st.calls++;
    if (defer) {
        c.pending.push_back(Pending{hy, out, y_bytes, true});
        return DMC_HIP_OK;
    }
    if (!c.pending.empty() && (rc = copy_pending_out())) return rc;
    auto t2 = std::chrono::steady_clock::now();
    HIP_TRY(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
    const uint64_t wait_ns = (uint64_t)ns_since(t2);
    c.st.wait_ns += wait_ns;
    if (timed) stats_call(k, n, batch, wait_ns, !x_direct);
    auto t3 = std::chrono::steady_clock::now();
    for (const Pending &p : c.pending) memcpy(p.dst, p.src, p.bytes);
    c.pending.clear();
    memcpy(out, hy, y_bytes);
    c.hx_off = 0;
    c.hy_off = 0;
    c.st.readback_ns += ns_since(t3);
    stats_line(k, n);
    return DMC_HIP_OK;
}

int run_host_locked(bool rd, int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n, int64_t batch,
                    int64_t ls, int64_t rs, bool defer) {
    std::lock_guard<std::mutex> lk(g_mu);
    return run_host(rd, reinterpret_cast<const float *>(l), reinterpret_cast<const uint16_t *>(r),
                    reinterpret_cast<float *>(out), m, k, n, batch, ls, rs, defer);
}

void run_host_or_die(const char *entry, bool rd, int64_t l, int64_t r, int64_t out, int64_t m,
                     int64_t k, int64_t n, int64_t batch, int64_t ls, int64_t rs, bool defer) {
    if (run_host_locked(rd, l, r, out, m, k, n, batch, ls, rs, defer)) fatal(entry);
}

// ---- the f32 path of `@` (jit.rs:20806-20831) -----------------------------------
//
// out[m,n] = l[m,k] @ r[k,n], all f32: the reference's scalar_matmul /
// simd_matmul / dmc_matmul_par chain (jit.rs:20715-20802, jit.rs:29415-29466)
// on the row-dot f32 kernels, for the two GEMV shapes:
//   W @ x (n <= kF32MaxAct activation columns): l [m,k] is the weight, its
//     rows the output rows; r's n columns are the activation rows, gathered
//     into the pinned staging;
//   x @ W (m <= kF32MaxAct activation rows): r [k,n] is the weight, kept
//     resident as its transpose [n,k] (one transpose at first use).
// Other shapes are GEMMs this route does not take (dmc_hip_f32_selected says
// so up front).  As for bf16, x and y pass through pinned staging.  The
// weight side is another matter: the reference's f32 `@` keeps nothing
// between calls, and either operand may be an activation the program
// updates in place, so a sampled content key is no proof that the bytes are
// unchanged.  The weight side therefore stays resident only when the caller
// registered those bytes at that address (dmc_hip_register_weight: its
// promise that they stay unchanged); otherwise it is uploaded on every call
// (and, for x @ W, transposed on the device into a second scratch buffer).
constexpr int64_t kF32MaxAct = 16;

bool f32_weight_left(int64_t m, int64_t n) { return n <= kF32MaxAct && (n <= m || m > kF32MaxAct); }

int run_host_f32(const float *l, const float *r, float *out, int64_t m, int64_t k, int64_t n) {
    if (m < 0 || k < 0 || n < 0)
        return fail(DMC_HIP_EINVAL, "negative size (m=%lld k=%lld n=%lld)", (long long)m, (long long)k, (long long)n);
    if (m == 0 || n == 0) return DMC_HIP_OK;  // jit.rs:29419
    if (!valid_dims(m, k, n)) return fail(DMC_HIP_EINVAL, "dimension beyond int32");
    if (!out || (k > 0 && (!l || !r))) return fail(DMC_HIP_EINVAL, "null pointer");
    const bool w_left = f32_weight_left(m, n);
    if (!w_left && m > kF32MaxAct)
        return fail(DMC_HIP_EINVAL,
                    "f32 route: GEMV shapes only (m <= %lld or n <= %lld activation rows), got m=%lld n=%lld",
                    (long long)kF32MaxAct, (long long)kF32MaxAct, (long long)m, (long long)n);
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    // Deferred bf16 calls are materialized first, so their outputs and this
    // call's staging never meet.
    if (!c.pending.empty() && (rc = flush_locked())) return rc;
    auto t0 = std::chrono::steady_clock::now();
    const int64_t acts = w_left ? n : m, rows = w_left ? m : n;
    const size_t x_bytes = (size_t)(acts * k) * 4, w_bytes = (size_t)(rows * k) * 4;
    const size_t y_bytes = (size_t)(m * n) * 4;
    char *hx = nullptr, *hx_dev = nullptr, *hy = nullptr, *hy_dev = nullptr;
    if ((rc = stage(c.hx, c.hx_off, x_bytes ? x_bytes : 4, hipHostMallocDefault, &hx, &hx_dev))) return rc;
    if ((rc = stage(c.hy, c.hy_off, y_bytes, hipHostMallocCoherent, &hy, &hy_dev))) return rc;
    float *const hxf = reinterpret_cast<float *>(hx);
    if (w_left && n > 1) {
        for (int64_t kk = 0; kk < k; ++kk)
            for (int64_t j = 0; j < n; ++j) hxf[j * k + kk] = r[kk * n + j];
    } else if (x_bytes) {
        memcpy(hx, w_left ? r : l, x_bytes);
    }
    const bool y_direct = y_bytes <= c.y_direct_max;
    const bool x_direct = x_bytes <= c.x_direct_max;
    if (!x_direct && (rc = ensure_dev(c.dx, x_bytes))) return rc;
    if (!y_direct && (rc = ensure_dev(c.dy, y_bytes))) return rc;
    float *const ydst = static_cast<float *>(y_direct ? static_cast<void *>(hy_dev) : c.dy.p);
    const float *const xsrc = static_cast<const float *>(x_direct ? static_cast<void *>(hx_dev) : c.dx.p);
    if (!x_direct) HIP_TRY(hipMemcpyAsync(c.dx.p, hx, x_bytes, hipMemcpyHostToDevice, c.stream), "x upload");
    c.st.stage_ns += ns_since(t0);
    void *dw = nullptr;
    const void *const wsrc = w_left ? static_cast<const void *>(l) : static_cast<const void *>(r);
    if (w_bytes && c.weights->registered(content_key(wsrc, (int64_t)w_bytes), wsrc)) {
        if ((rc = w_left ? resident(l, (int64_t)w_bytes, &dw) : resident(r, (int64_t)w_bytes, &dw, k, n, false, 4)))
            return rc;
    } else if (w_bytes) {
        if ((rc = ensure_dev(c.dwf, w_bytes + dmc::kWeightSlack))) return rc;
        HIP_TRY(hipMemcpyAsync(c.dwf.p, wsrc, w_bytes, hipMemcpyHostToDevice, c.stream), "f32 weight upload");
        dw = c.dwf.p;
        if (!w_left) {  // r [k,n] -> [n,k], the row-dot layout
            if ((rc = ensure_dev(c.dwt, w_bytes + dmc::kWeightSlack))) return rc;
            HIP_TRY(dmc::launch_transpose_f32(static_cast<const float *>(c.dwf.p), static_cast<float *>(c.dwt.p), k,
                                              n, c.stream),
                    "f32 weight transpose");
            dw = c.dwt.p;
        }
    } else {
        dw = c.dummy;
    }
    auto t1 = std::chrono::steady_clock::now();
    // Output (activation a, weight row i) is out[i][a] for W @ x, out[a][i] for x @ W.
    const dmc::F32Problem p{static_cast<const float *>(dw), k, xsrc, k, ydst,
                            w_left ? 1 : n, w_left ? n : 1, acts, k, rows};
    const dmc::F32Plan pl = dmc::plan_f32(p, c.cus);
    hipError_t e = dmc::launch_f32(p, pl, c.stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    if (!y_direct) HIP_TRY(hipMemcpyAsync(hy, c.dy.p, y_bytes, hipMemcpyDeviceToHost, c.stream), "y readback");
    c.st.enqueue_ns += ns_since(t1);
    c.st.calls++;
    auto t2 = std::chrono::steady_clock::now();
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    c.st.wait_ns += (uint64_t)ns_since(t2);
    auto t3 = std::chrono::steady_clock::now();
    memcpy(out, hy, y_bytes);
    c.hx_off = 0;
    c.hy_off = 0;
    c.st.readback_ns += ns_since(t3);
    return DMC_HIP_OK;
}

int run_host_f32_locked(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    return run_host_f32(reinterpret_cast<const float *>(l), reinterpret_cast<const float *>(r),
                        reinterpret_cast<float *>(out), m, k, n);
}


// ---- weight ingress from .npz (jit.rs:29836-29944) ----------------------------
//
// The entry's uncompressed bytes stream through pinned chunks; the part that
// is array data goes to the device with asynchronous copies on the library
// stream while the next chunks are read.  A stored entry of at least
// kIngressParallelMin bytes is read by several threads (positioned reads,
// one CRC-32 per chunk, combined in order); a deflated one by one thread
// through zlib.  The whole entry is read, so its CRC-32 is checked as the
// reference's reader checks it.

constexpr size_t kIngressChunk = (size_t)8 << 20;
constexpr uint64_t kIngressParallelMin = (uint64_t)64 << 20;

struct FdCloser {
    int fd;
    ~FdCloser() {
        if (fd >= 0) close(fd);
    }
};

// Pinned chunks [0, count) of the ingress pool, allocated on first use.
int ingress_pool(size_t count) {
    Ctx &c = ctx();
    while (c.ingress.size() < count) {
        void *p = nullptr;
        HIP_TRY(hipHostMalloc(&p, kIngressChunk, hipHostMallocDefault), "hipHostMalloc(ingress)");
        hipEvent_t ev = nullptr;
        hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) {
            (void)hipHostFree(p);
            return hip_fail(e, "hipEventCreate(ingress)");
        }
        c.ingress.push_back(p);
        c.ingress_ev.push_back(ev);
    }
    return DMC_HIP_OK;
}

// Bytes [pos, pos + n) of the entry sit in pinned chunk `buf`; the part inside
// the array's bytes [doff, doff + take) is copied to dst + (offset - doff),
// then the chunk's event is recorded so its next user can wait for the copy.
hipError_t deliver(const uint8_t *buf, uint64_t pos, size_t n, uint64_t doff, uint64_t take, uint8_t *dst,
                   hipEvent_t ev, hipStream_t s) {
    const uint64_t lo = std::max(pos, doff), hi = std::min<uint64_t>(pos + n, doff + take);
    if (lo < hi) {
        hipError_t e = hipMemcpyAsync(dst + (lo - doff), buf + (lo - pos), (size_t)(hi - lo), hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
    }
    return hipEventRecord(ev, s);
}

int64_t vault_load_npz_locked(const char *path, const char *key, int64_t numel, int64_t elem_bytes,
                              int64_t convert) {
    if (!path || !key) return fail(DMC_HIP_EINVAL, "vault.load_npz: null path or key"), 0;
    if (numel < 0 || elem_bytes < 1 || elem_bytes > 8 || convert < 0 || convert > 2 ||
        (convert != 0 && elem_bytes != 2) || numel > (INT64_MAX - 256) / 8)
        return fail(DMC_HIP_EINVAL, "vault.load_npz: bad numel/elem_bytes/convert (%lld, %lld, %lld)",
                    (long long)numel, (long long)elem_bytes, (long long)convert), 0;
    if (ensure_init()) return 0;
    Ctx &c = ctx();
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(DMC_HIP_EIO, "vault.load_npz: cannot open `%s`: %s", path, strerror(errno)), 0;
    FdCloser closer{fd};
    dmc::NpzEntry ent;
    std::string err;
    if (dmc::npz_find_entry(fd, key, ent, err))
        return fail(DMC_HIP_EIO, "vault.load_npz: %s in `%s`", err.c_str(), path), 0;

    const bool parallel = ent.method == 0 && ent.usize >= kIngressParallelMin;
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t workers = parallel ? std::min<size_t>(16, hw) : 0;
    if (ingress_pool(2 + 2 * workers)) return 0;
    for (hipEvent_t ev : c.ingress_ev) {  // every chunk starts out free
        hipError_t e = hipEventRecord(ev, c.stream);
        if (e != hipSuccess) return hip_fail(e, "hipEventRecord"), 0;
    }

    // The first chunk: the .npy header.
    dmc::NpzStream zs(fd, ent);
    uint8_t *head = static_cast<uint8_t *>(c.ingress[0]);
    const int64_t hn = zs.read(head, kIngressChunk, err);
    if (hn < 0) return fail(DMC_HIP_EIO, "vault.load_npz: read error for `%s` in `%s`: %s", key, path, err.c_str()), 0;
    int major = 0;
    const int64_t doff_s = dmc::npy_data_offset(head, (size_t)hn, &major);
    if (doff_s == -1) return fail(DMC_HIP_EIO, "vault.load_npz: entry `%s` is not a valid .npy file", key), 0;
    if (doff_s < 0) return fail(DMC_HIP_EIO, "vault.load_npz: entry `%s` ends inside its .npy header", key), 0;
    const uint64_t doff = (uint64_t)doff_s;
    const uint64_t src_bytes = (uint64_t)numel * (uint64_t)elem_bytes;
    const uint64_t out_bytes = convert ? (uint64_t)numel * 4 : src_bytes;
    const uint64_t avail = ent.usize > doff ? ent.usize - doff : 0;
    const uint64_t take = std::min(avail, src_bytes);
    if (take < src_bytes)  // the reference reports the short entry and loads what it holds
        fprintf(stderr, "vault.load_npz: entry `%s` data is %llu bytes but expected %llu\n", key,
                (unsigned long long)avail, (unsigned long long)src_bytes);

    void *region = nullptr, *raw = nullptr;
    hipError_t he = hipMalloc(&region, (size_t)out_bytes + dmc::kWeightSlack);
    if (he != hipSuccess) return hip_fail(he, "hipMalloc(region)"), 0;
    // On failure after this point: drain the stream, free, return 0 (the
    // message is already set).
    auto give_up = [&]() -> int64_t {
        (void)hipStreamSynchronize(c.stream);
        if (raw) (void)hipFree(raw);
        (void)hipFree(region);
        return 0;
    };
    if (convert && take) {
        he = hipMalloc(&raw, (size_t)take);
        if (he != hipSuccess) return hip_fail(he, "hipMalloc(ingress staging)"), give_up();
    }
    uint8_t *dst = static_cast<uint8_t *>(convert ? raw : region);

    he = deliver(head, 0, (size_t)hn, doff, take, dst, c.ingress_ev[0], c.stream);
    if (he != hipSuccess) return hip_fail(he, "ingress copy"), give_up();
    uint32_t crc = zs.crc();
    uint64_t produced = (uint64_t)hn;
    if (!parallel) {
        // One reader: chunks alternate between two pinned buffers.
        for (int b = 1;; b ^= 1) {
            he = hipEventSynchronize(c.ingress_ev[b]);
            if (he != hipSuccess) return hip_fail(he, "hipEventSynchronize"), give_up();
            uint8_t *buf = static_cast<uint8_t *>(c.ingress[b]);
            const int64_t got = zs.read(buf, kIngressChunk, err);
            if (got < 0)
                return fail(DMC_HIP_EIO, "vault.load_npz: read error for `%s` in `%s`: %s", key, path, err.c_str()),
                       give_up();
            if (got == 0) break;
            he = deliver(buf, produced, (size_t)got, doff, take, dst, c.ingress_ev[b], c.stream);
            if (he != hipSuccess) return hip_fail(he, "ingress copy"), give_up();
            produced += (uint64_t)got;
        }
        crc = zs.crc();
    } else {
        // Chunk i >= 1 of the stored entry goes to worker (i - 1) % workers,
        // which alternates between its two pinned buffers.
        const uint64_t nchunks = (ent.usize + kIngressChunk - 1) / kIngressChunk;
        std::vector<uint32_t> crcs(nchunks, 0);
        std::atomic<bool> bad{false};
        std::string werr;
        std::mutex werr_mu;
        auto work = [&](size_t w) {
            for (uint64_t i = 1 + w, round = 0; i < nchunks && !bad.load(); i += workers, ++round) {
                const size_t slot = 2 + 2 * w + (round & 1);
                uint8_t *buf = static_cast<uint8_t *>(c.ingress[slot]);
                const uint64_t pos = i * kIngressChunk;
                const size_t n = (size_t)std::min<uint64_t>(kIngressChunk, ent.usize - pos);
                hipError_t e = hipEventSynchronize(c.ingress_ev[slot]);
                std::string why;
                if (e != hipSuccess) why = std::string("hipEventSynchronize: ") + hipGetErrorString(e);
                else if (!dmc::pread_exact(fd, buf, n, ent.data_pos + pos)) why = "read failed";
                if (why.empty()) {
                    crcs[i] = dmc::npz_crc32(0, buf, n);
                    e = deliver(buf, pos, n, doff, take, dst, c.ingress_ev[slot], c.stream);
                    if (e != hipSuccess) why = std::string("ingress copy: ") + hipGetErrorString(e);
                }
                if (!why.empty()) {
                    std::lock_guard<std::mutex> g(werr_mu);
                    if (!bad.exchange(true)) werr = why;
                    return;
                }
            }
        };
        std::vector<std::thread> pool;
        for (size_t w = 0; w < workers; ++w) pool.emplace_back(work, w);
        for (auto &t : pool) t.join();
        if (bad.load())
            return fail(DMC_HIP_EIO, "vault.load_npz: read error for `%s` in `%s`: %s", key, path, werr.c_str()),
                   give_up();
        for (uint64_t i = 1; i < nchunks; ++i) {
            const uint64_t n = std::min<uint64_t>(kIngressChunk, ent.usize - i * kIngressChunk);
            crc = dmc::npz_crc32_combine(crc, crcs[i], n);
            produced += n;
        }
    }
    if (produced != ent.usize)
        return fail(DMC_HIP_EIO, "vault.load_npz: read error for `%s` in `%s`: %llu bytes, the archive says %llu",
                    key, path, (unsigned long long)produced, (unsigned long long)ent.usize),
               give_up();
    if (crc != ent.crc)
        return fail(DMC_HIP_EIO, "vault.load_npz: read error for `%s` in `%s`: invalid checksum", key, path),
               give_up();

    // Widen on the device (npz_fill, jit.rs:29931-29941: take/2 elements), and
    // zero what the entry did not hold plus the padding.
    uint64_t filled = take;
    if (convert) {
        const int64_t elems = (int64_t)(take / 2);
        he = convert == 1 ? dmc::launch_bf16_upconvert(static_cast<const uint16_t *>(raw), static_cast<float *>(region),
                                                        elems, c.stream)
                          : dmc::launch_f16_upconvert(static_cast<const uint16_t *>(raw), static_cast<float *>(region),
                                                       elems, c.stream);
        if (he != hipSuccess) return hip_fail(he, "ingress widen launch"), give_up();
        filled = (uint64_t)elems * 4;
    }
    he = hipMemsetAsync(static_cast<uint8_t *>(region) + filled, 0,
                        (size_t)(out_bytes - filled) + dmc::kWeightSlack, c.stream);
    if (he != hipSuccess) return hip_fail(he, "ingress zero fill"), give_up();
    he = hipStreamSynchronize(c.stream);
    if (he != hipSuccess) return hip_fail(he, "hipStreamSynchronize"), give_up();
    if (raw) (void)hipFree(raw);
    return reinterpret_cast<int64_t>(region);
}
}  // namespace

// ---- drop-in surface ----------------------------------------------------------

extern "C" {

void dmc_matmul_bf16_gpu(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    run_host_or_die("dmc_matmul_bf16_gpu", false, l, r, out, m, k, n, 1, 0, 0, false);
}

void dmc_matmul_bf16_gpu_batched(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n,
                                 int64_t batch, int64_t ls, int64_t rs) {
    run_host_or_die("dmc_matmul_bf16_gpu_batched", false, l, r, out, m, k, n, batch, ls, rs, false);
}

void dmc_matmul_bf16_gpu_batched_deferred(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k,
                                          int64_t n, int64_t batch, int64_t ls, int64_t rs) {
    run_host_or_die("dmc_matmul_bf16_gpu_batched_deferred", false, l, r, out, m, k, n, batch, ls, rs,
                    true);
}

void dmc_matmul_bf16_gpu_flush(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (flush_locked()) fatal("dmc_matmul_bf16_gpu_flush");
}

void dmc_matmul_bf16_gpu_t(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    run_host_or_die("dmc_matmul_bf16_gpu_t", true, l, r, out, m, k, n, 1, 0, 0, false);
}

void dmc_matmul_f32_gpu(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    if (run_host_f32_locked(l, r, out, m, k, n)) fatal("dmc_matmul_f32_gpu");
}

// ---- error-returning forms of the drop-in entries ------------------------------
//
// Same arguments and results; a failure returns DMC_HIP_E* (message in
// dmc_hip_last_error) with `out` untouched -- the kernel writes pinned
// staging, copied to `out` only after the stream has completed -- so the
// caller can compute the call on its own CPU kernel, as the reference does
// when its device path is unavailable (gpu.rs:327-332, gpu.rs:483-486).

int32_t dmc_matmul_bf16_gpu_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    return run_host_locked(false, l, r, out, m, k, n, 1, 0, 0, false);
}

int32_t dmc_matmul_bf16_gpu_t_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    return run_host_locked(true, l, r, out, m, k, n, 1, 0, 0, false);
}

int32_t dmc_matmul_bf16_gpu_batched_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n,
                                        int64_t batch, int64_t ls, int64_t rs) {
    return run_host_locked(false, l, r, out, m, k, n, batch, ls, rs, false);
}

int32_t dmc_matmul_bf16_gpu_batched_deferred_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k,
                                                 int64_t n, int64_t batch, int64_t ls, int64_t rs) {
    return run_host_locked(false, l, r, out, m, k, n, batch, ls, rs, true);
}

int32_t dmc_matmul_bf16_gpu_flush_try(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return flush_locked();
}

int32_t dmc_matmul_f32_gpu_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n) {
    return run_host_f32_locked(l, r, out, m, k, n);
}

// ---- additions ----------------------------------------------------------------

int32_t dmc_hip_available(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return ensure_init() == DMC_HIP_OK ? 1 : 0;
}

int32_t dmc_hip_gemv_selected(int32_t hip_on, int32_t deterministic_depth, int64_t m, int64_t k,
                              int64_t n) {
    if (!hip_on || deterministic_depth != 0) return 0;
    if (m <= 0 || k <= 0 || n <= 0) return 0;
    const __int128 macs = (__int128)m * k * n;
    return macs >= (__int128)DMC_HIP_MIN_MACS ? 1 : 0;
}

int32_t dmc_hip_f32_selected(int32_t hip_on, int32_t deterministic_depth, int64_t m, int64_t k, int64_t n) {
    if (!hip_on || deterministic_depth != 0) return 0;
    if (m <= 0 || k <= 0 || n <= 0 || (m > kF32MaxAct && n > kF32MaxAct)) return 0;
    const __int128 macs = (__int128)m * k * n;
    return macs >= (__int128)DMC_HIP_MIN_MACS ? 1 : 0;
}

const char *dmc_hip_last_error(void) { return t_err.c_str(); }

int64_t dmc_hip_region_alloc(int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes <= 0) return fail(DMC_HIP_EINVAL, "region size must be positive"), 0;
    if (ensure_init()) return 0;
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, (size_t)bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(region)"), 0;
    return reinterpret_cast<int64_t>(d);
}

int32_t dmc_hip_region_free(int64_t dptr) {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_init();
    if (rc) return rc;
    if (!dptr) return DMC_HIP_OK;
    HIP_TRY(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
    HIP_TRY(hipFree(reinterpret_cast<void *>(dptr)), "hipFree(region)");
    return DMC_HIP_OK;
}

int32_t dmc_hip_upload(int64_t dst_dev, int64_t src_host, int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes < 0 || (bytes > 0 && (!dst_dev || !src_host))) return fail(DMC_HIP_EINVAL, "bad upload");
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return DMC_HIP_OK;
    Ctx &c = ctx();
    HIP_TRY(hipMemcpyAsync(reinterpret_cast<void *>(dst_dev), reinterpret_cast<const void *>(src_host),
                           (size_t)bytes, hipMemcpyHostToDevice, c.stream),
            "upload");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return DMC_HIP_OK;
}

int32_t dmc_hip_download(int64_t dst_host, int64_t src_dev, int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes < 0 || (bytes > 0 && (!dst_host || !src_dev))) return fail(DMC_HIP_EINVAL, "bad download");
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return DMC_HIP_OK;
    Ctx &c = ctx();
    HIP_TRY(hipMemcpyAsync(reinterpret_cast<void *>(dst_host), reinterpret_cast<const void *>(src_dev),
                           (size_t)bytes, hipMemcpyDeviceToHost, c.stream),
            "download");
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    return DMC_HIP_OK;
}

int32_t dmc_hip_copy_device(int64_t dst_dev, int64_t src_dev, int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes < 0 || (bytes > 0 && (!dst_dev || !src_dev))) return fail(DMC_HIP_EINVAL, "bad copy");
    int rc = ensure_init();
    if (rc) return rc;
    if (!bytes) return DMC_HIP_OK;
    HIP_TRY(hipMemcpyAsync(reinterpret_cast<void *>(dst_dev), reinterpret_cast<const void *>(src_dev),
                           (size_t)bytes, hipMemcpyDeviceToDevice, ctx().stream),
            "device copy");
    return DMC_HIP_OK;
}

int64_t dmc_hip_register_weight(int64_t host_ptr, int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes <= 0 || !host_ptr) return fail(DMC_HIP_EINVAL, "bad weight range"), 0;
    if (ensure_init()) return 0;
    void *d = nullptr;
    if (resident(reinterpret_cast<const void *>(host_ptr), bytes, &d, 0, 0, true)) return 0;
    return reinterpret_cast<int64_t>(d);
}

int32_t dmc_hip_release_weights(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    Ctx &c = ctx();
    if (!c.tried || !c.ok) return DMC_HIP_OK;
    int rc = flush_locked();
    if (rc) return rc;
    return release_weights_locked();
}

int64_t dmc_hip_resident_count(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return ctx().weights ? (int64_t)ctx().weights->count() : 0;
}

int64_t dmc_hip_resident_bytes(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return ctx().weights ? ctx().weights->bytes() : 0;
}

int32_t dmc_hip_gemv_cs(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k, int64_t n,
                        int64_t batch, int64_t ls, int64_t rs) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!valid_dims(m, k, n) || batch < 0 || ls < 0 || rs < 0)
        return fail(DMC_HIP_EINVAL, "bad GEMV shape");
    if (m == 0 || n == 0 || batch == 0) return DMC_HIP_OK;
    if (!y_dev || (k > 0 && (!x_dev || !w_dev))) return fail(DMC_HIP_EINVAL, "null pointer");
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    dmc::CsProblem p{reinterpret_cast<const uint16_t *>(w_dev), reinterpret_cast<const float *>(x_dev),
                     reinterpret_cast<float *>(y_dev), m, k, n, batch, ls, rs};
    const dmc::CsPlan pl = dmc::plan_cs(p, c.cus);
    if ((rc = ensure_dev(c.ws, pl.workspace_bytes))) return rc;
    hipError_t e = dmc::launch_cs(p, pl, c.ws.p, c.stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_gemv_cs_noalloc(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k, int64_t n,
                                int64_t batch, int64_t ls, int64_t rs) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!valid_dims(m, k, n) || batch < 0 || ls < 0 || rs < 0)
        return fail(DMC_HIP_EINVAL, "bad GEMV shape");
    if (m == 0 || n == 0 || batch == 0) return DMC_HIP_OK;
    if (!y_dev || (k > 0 && (!x_dev || !w_dev))) return fail(DMC_HIP_EINVAL, "null pointer");
    // No set-up here: it allocates (stream, a dummy region).  The caller sets
    // the library up beforehand, with dmc_hip_available().
    Ctx &c = ctx();
    if (!c.tried || !c.ok)
        return fail(DMC_HIP_ENODEV, "dmc_hip_gemv_cs_noalloc: library not set up (call dmc_hip_available() first)");
    HIP_TRY(hipSetDevice(c.device), "hipSetDevice");
    auto it = c.noalloc_scratch.find(c.device);
    if (it == c.noalloc_scratch.end())
        return fail(DMC_HIP_EDEVICE, "dmc_hip_gemv_cs_noalloc: no fixed scratch on device %d: %s", c.device,
                    c.noalloc_err.c_str());
    dmc::CsProblem p{reinterpret_cast<const uint16_t *>(w_dev), reinterpret_cast<const float *>(x_dev),
                     reinterpret_cast<float *>(y_dev), m, k, n, batch, ls, rs};
    const dmc::CsPlan pl = dmc::plan_cs(p, c.cus);
    if (pl.workspace_bytes > dmc::noalloc_scratch_bytes())
        return fail(DMC_HIP_EINVAL,
                    "dmc_hip_gemv_cs_noalloc: this shape needs %zu bytes of split-k scratch, the fixed maximum is "
                    "%zu (use dmc_hip_gemv_cs)",
                    pl.workspace_bytes, dmc::noalloc_scratch_bytes());
    hipError_t e = dmc::launch_cs(p, pl, it->second, c.stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_gemv_rd(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!valid_dims(m, k, n)) return fail(DMC_HIP_EINVAL, "bad GEMV shape");
    if (m == 0 || n == 0) return DMC_HIP_OK;
    if (!y_dev || (k > 0 && (!x_dev || !w_dev))) return fail(DMC_HIP_EINVAL, "null pointer");
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    dmc::RdProblem p{reinterpret_cast<const uint16_t *>(w_dev), k, reinterpret_cast<const float *>(x_dev),
                     k, reinterpret_cast<float *>(y_dev), n, m, k, n};
    const dmc::RdPlan pl = dmc::plan_rd(p, c.cus);
    if ((rc = ensure_dev(c.ws, pl.workspace_bytes))) return rc;
    hipError_t e = dmc::launch_rd(p, pl, pl.workspace_bytes ? c.ws.p : nullptr, c.stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_gemv_f32_rd(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!valid_dims(m, k, n)) return fail(DMC_HIP_EINVAL, "bad GEMV shape");
    if (m == 0 || n == 0) return DMC_HIP_OK;
    if (!y_dev || (k > 0 && (!x_dev || !w_dev))) return fail(DMC_HIP_EINVAL, "null pointer");
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    const dmc::F32Problem p{reinterpret_cast<const float *>(w_dev), k, reinterpret_cast<const float *>(x_dev), k,
                            reinterpret_cast<float *>(y_dev), n, 1, m, k, n};
    hipError_t e = dmc::launch_f32(p, dmc::plan_f32(p, c.cus), c.stream);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_probe_read(int64_t src_dev, int64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (bytes < 0 || (bytes > 0 && !src_dev)) return fail(DMC_HIP_EINVAL, "bad probe range");
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    if (!c.sink) HIP_TRY(hipMalloc(&c.sink, dmc::probe_sink_bytes()), "hipMalloc(probe sink)");
    hipError_t e = dmc::launch_probe_read(reinterpret_cast<const void *>(src_dev), bytes, c.sink, c.stream);
    if (e != hipSuccess) return hip_fail(e, "probe launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_gemv_rd_grouped(int64_t count, const int64_t *x_devs, const int64_t *w_devs,
                                const int64_t *y_devs, const int64_t *ns, int64_t m, int64_t k) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (count < 0 || (count > 0 && (!x_devs || !w_devs || !y_devs || !ns)) || !valid_dims(m, k, 0))
        return fail(DMC_HIP_EINVAL, "bad grouped GEMV arguments");
    for (int64_t i = 0; i < count; ++i) {
        if (ns[i] < 0 || ns[i] > INT32_MAX) return fail(DMC_HIP_EINVAL, "bad grouped GEMV row count");
        if (m > 0 && ns[i] > 0 && (!y_devs[i] || (k > 0 && (!x_devs[i] || !w_devs[i]))))
            return fail(DMC_HIP_EINVAL, "null pointer in grouped GEMV");
    }
    if (count == 0 || m == 0) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    for (int64_t b = 0; b < count; b += dmc::kMaxGroup) {
        dmc::RdGroup g{};
        g.count = (int)std::min<int64_t>(dmc::kMaxGroup, count - b);
        g.m = m;
        g.k = k;
        for (int i = 0; i < g.count; ++i) {
            g.w[i] = reinterpret_cast<const uint16_t *>(w_devs[b + i]);
            g.x[i] = reinterpret_cast<const float *>(x_devs[b + i]);
            g.y[i] = reinterpret_cast<float *>(y_devs[b + i]);
            g.n[i] = ns[b + i];
        }
        // A group of one is a single GEMV: the single-problem plan (the
        // shared-x and MFMA layouts included).
        const dmc::RdPlan gp = g.count > 1 ? dmc::plan_rd_group(g, c.cus) : dmc::RdPlan{};
        if (gp.kvec > 0) {
            hipError_t e = dmc::launch_rd_group(g, gp, c.stream);
            if (e != hipSuccess) return hip_fail(e, "grouped kernel launch");
            continue;
        }
        for (int i = 0; i < g.count; ++i) {  // outside the streaming kernel's range: one launch each
            if (g.n[i] == 0) continue;
            dmc::RdProblem p{g.w[i], k, g.x[i], k, g.y[i], g.n[i], m, k, g.n[i]};
            const dmc::RdPlan pl = dmc::plan_rd(p, c.cus);
            if ((rc = ensure_dev(c.ws, pl.workspace_bytes))) return rc;
            hipError_t e = dmc::launch_rd(p, pl, pl.workspace_bytes ? c.ws.p : nullptr, c.stream);
            if (e != hipSuccess) return hip_fail(e, "kernel launch");
        }
    }
    return DMC_HIP_OK;
}

int32_t dmc_hip_fill_counter_bf16(int64_t dst_dev, int64_t count, int64_t offset, uint64_t key,
                                  int64_t table_dev) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (count < 0 || offset < 0 || (count > 0 && (!dst_dev || !table_dev)))
        return fail(DMC_HIP_EINVAL, "bad fill arguments");
    if (count == 0) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = dmc::launch_fill_counter_bf16(reinterpret_cast<uint16_t *>(dst_dev), count, offset, key,
                                                 reinterpret_cast<const uint16_t *>(table_dev), ctx().stream);
    if (e != hipSuccess) return hip_fail(e, "fill launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_bf16_upconvert(int64_t src_dev, int64_t dst_dev, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (n < 0 || (n > 0 && (!src_dev || !dst_dev))) return fail(DMC_HIP_EINVAL, "bad upconvert arguments");
    if (n == 0) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = dmc::launch_bf16_upconvert(reinterpret_cast<const uint16_t *>(src_dev),
                                              reinterpret_cast<float *>(dst_dev), n, ctx().stream);
    if (e != hipSuccess) return hip_fail(e, "upconvert launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_f32_to_bf16(int64_t src_dev, int64_t dst_dev, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (n < 0 || (n > 0 && (!src_dev || !dst_dev))) return fail(DMC_HIP_EINVAL, "bad f32-to-bf16 arguments");
    if (n == 0) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = dmc::launch_f32_to_bf16(reinterpret_cast<const float *>(src_dev),
                                           reinterpret_cast<uint16_t *>(dst_dev), n, ctx().stream);
    if (e != hipSuccess) return hip_fail(e, "f32-to-bf16 launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_bf16_transpose_2d(int64_t src_dev, int64_t dst_dev, int64_t m, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (m < 0 || n < 0 || (m > 0 && n > 0 && (!src_dev || !dst_dev)))
        return fail(DMC_HIP_EINVAL, "bad transpose arguments");
    if (m == 0 || n == 0) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = dmc::launch_transpose_bf16(reinterpret_cast<const uint16_t *>(src_dev),
                                              reinterpret_cast<uint16_t *>(dst_dev), m, n, ctx().stream);
    if (e != hipSuccess) return hip_fail(e, "transpose launch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_capture_begin(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_init();
    if (rc) return rc;
    HIP_TRY(hipStreamBeginCapture(ctx().stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return DMC_HIP_OK;
}

int64_t dmc_hip_capture_end(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (ensure_init()) return 0;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx().stream, &graph);
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture (an entry that allocates or waits was "
                                            "called while capturing)"), 0;
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate"), 0;
    ctx().live_graphs++;
    return reinterpret_cast<int64_t>(exec);
}

int32_t dmc_hip_graph_launch(int64_t exec) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!exec) return fail(DMC_HIP_EINVAL, "null graph");
    int rc = ensure_init();
    if (rc) return rc;
    HIP_TRY(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(exec), ctx().stream), "hipGraphLaunch");
    return DMC_HIP_OK;
}

int32_t dmc_hip_graph_destroy(int64_t exec) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!exec) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    Ctx &c = ctx();
    HIP_TRY(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    HIP_TRY(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(exec)), "hipGraphExecDestroy");
    if (c.live_graphs > 0 && --c.live_graphs == 0) {
        for (void *p : c.retired_ws) HIP_TRY(hipFree(p), "hipFree(retired workspace)");
        c.retired_ws.clear();
    }
    return DMC_HIP_OK;
}

int32_t dmc_hip_synchronize(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_init();
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(ctx().stream), "hipStreamSynchronize");
    return DMC_HIP_OK;
}

int32_t dmc_hip_plan_f32(int64_t x_addr, int64_t w_addr, int64_t m, int64_t k, int64_t n, int64_t *out8) {
    if (!out8 || !valid_dims(m, k, n)) return fail(DMC_HIP_EINVAL, "bad plan query");
    int cus;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        cus = ctx().ok ? ctx().cus : 256;
    }
    const dmc::F32Problem p{reinterpret_cast<const float *>(w_addr), k, reinterpret_cast<const float *>(x_addr),
                            k, nullptr, n, 1, m, k, n};
    const dmc::F32Plan pl = dmc::plan_f32(p, cus);
    const int64_t v[8] = {pl.kvec, pl.rows, pl.mt, pl.grid_x, pl.grid_y, pl.waves, pl.rpw, 0};
    memcpy(out8, v, sizeof v);
    return DMC_HIP_OK;
}

int32_t dmc_hip_plan(int32_t layout_rd, int64_t x_addr, int64_t w_addr, int64_t m, int64_t k, int64_t n,
                     int64_t batch, int64_t rs, int64_t *out8) {
    if (!out8 || !valid_dims(m, k, n) || batch < 0 || rs < 0) return fail(DMC_HIP_EINVAL, "bad plan query");
    int cus;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        cus = ctx().ok ? ctx().cus : 256;
    }
    if (layout_rd) {
        dmc::RdProblem p{reinterpret_cast<const uint16_t *>(w_addr), k, reinterpret_cast<const float *>(x_addr),
                         k, nullptr, n, m, k, n};
        const dmc::RdPlan pl = dmc::plan_rd(p, cus);
        const int64_t v[8] = {pl.vec, pl.rows, pl.mt, pl.grid_x, pl.mfma ? -pl.mkind : pl.kvec,
                              (int64_t)pl.workspace_bytes, pl.waves, pl.rpw};
        memcpy(out8, v, sizeof v);
    } else {
        dmc::CsProblem p{reinterpret_cast<const uint16_t *>(w_addr), reinterpret_cast<const float *>(x_addr),
                         nullptr, m, k, n, batch, 0, rs};
        const dmc::CsPlan pl = dmc::plan_cs(p, cus);
        const int64_t v[8] = {pl.vec, pl.stream ? -(int64_t)pl.rw : pl.rw, pl.mt, pl.grid_x, pl.slices,
                              (int64_t)pl.workspace_bytes, pl.waves, pl.stream ? pl.kslice : pl.cb};
        memcpy(out8, v, sizeof v);
    }
    return DMC_HIP_OK;
}

int64_t dmc_hip_event_create(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (ensure_init()) return 0;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) return hip_fail(e, "hipEventCreate"), 0;
    return reinterpret_cast<int64_t>(ev);
}

int32_t dmc_hip_event_record(int64_t ev) {
    std::lock_guard<std::mutex> lk(g_mu);
    int rc = ensure_init();
    if (rc) return rc;
    if (!ev) return fail(DMC_HIP_EINVAL, "null event");
    HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), ctx().stream), "hipEventRecord");
    return DMC_HIP_OK;
}

int32_t dmc_hip_event_synchronize(int64_t ev) {
    if (!ev) return fail(DMC_HIP_EINVAL, "null event");
    HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev)), "hipEventSynchronize");
    return DMC_HIP_OK;
}

float dmc_hip_event_elapsed_ms(int64_t start, int64_t stop) {
    if (!start || !stop) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)) !=
        hipSuccess)
        return -1.0f;
    return ms;
}

int32_t dmc_hip_event_destroy(int64_t ev) {
    if (!ev) return DMC_HIP_OK;
    HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)), "hipEventDestroy");
    return DMC_HIP_OK;
}

int32_t dmc_hip_device_cus(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return ensure_init() == DMC_HIP_OK ? ctx().cus : 0;
}

const char *dmc_hip_device_arch(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    return ensure_init() == DMC_HIP_OK ? ctx().arch.c_str() : "";
}

int64_t dmc_hip_vault_load_npz(const char *path, const char *key, int64_t numel, int64_t elem_bytes,
                               int64_t convert) {
    std::lock_guard<std::mutex> lk(g_mu);
    return vault_load_npz_locked(path, key, numel, elem_bytes, convert);
}

int32_t dmc_hip_npz_locate(const char *path, const char *key, int64_t *info) {
    if (!path || !key || !info) return fail(DMC_HIP_EINVAL, "npz_locate: null argument");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(DMC_HIP_EIO, "vault.load_npz: cannot open `%s`: %s", path, strerror(errno));
    FdCloser closer{fd};
    dmc::NpzEntry ent;
    std::string err;
    if (dmc::npz_find_entry(fd, key, ent, err)) return fail(DMC_HIP_EIO, "vault.load_npz: %s in `%s`", err.c_str(), path);
    std::vector<uint8_t> head(4096);
    dmc::NpzStream zs(fd, ent);
    const int64_t hn = zs.read(head.data(), head.size(), err);
    if (hn < 0) return fail(DMC_HIP_EIO, "vault.load_npz: read error for `%s` in `%s`: %s", key, path, err.c_str());
    int major = -1;
    const int64_t doff = dmc::npy_data_offset(head.data(), (size_t)hn, &major);
    const int64_t v[8] = {ent.bare ? 1 : 0, ent.method, (int64_t)ent.csize, (int64_t)ent.usize, (int64_t)ent.data_pos,
                          doff == -1 ? -1 : major, doff, (int64_t)ent.crc};
    memcpy(info, v, sizeof v);
    return DMC_HIP_OK;
}

int32_t dmc_hip_f16_upconvert(int64_t src_dev, int64_t dst_dev, int64_t n) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (n < 0 || (n > 0 && (!src_dev || !dst_dev))) return fail(DMC_HIP_EINVAL, "bad f16 upconvert arguments");
    if (n == 0) return DMC_HIP_OK;
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = dmc::launch_f16_upconvert(reinterpret_cast<const uint16_t *>(src_dev),
                                             reinterpret_cast<float *>(dst_dev), n, ctx().stream);
    if (e != hipSuccess) return hip_fail(e, "f16 upconvert launch");
    return DMC_HIP_OK;
}

}  // extern "C"
