// gemv_kernels.hip -- hand-written gfx950 (CDNA4) bf16-weight x f32-vector GEMV.
//
// The hot path of demoniC's `@` with a bf16 weight: the reference computes it
// on the CPU in dmc_matmul_bf16 (compiler/src/jit.rs:29481-29566) and on Apple
// GPUs in gemv_bf16_vec4cb / gemv_bf16_tiled2d (compiler/src/gpu.rs:115-183).
// These kernels are an MI355X design, not a translation of either:
//
//  * HBM-bound streaming.  Every weight byte is read exactly once per launch
//    with wave-wide coalesced 128-bit nontemporal loads (64/32/16-bit
//    variants in the general kernels cover K or N that are not multiples of
//    8, e.g. K = 4097).
//  * Row-dot (W [N,K]): the streaming kernel splits k over a workgroup's
//    waves with x held in registers; the general kernel covers any alignment.
//    Skinny M (>= 4 activation rows) runs on bf16 MFMA against x split into
//    three bf16 terms, with weights and x staged through LDS.
//  * Column-stream (W [K,N]): lanes own 8 columns, x[k] is wave-uniform
//    (scalar loads), waves split a workgroup's k slice, and k slices over
//    workgroups are summed by a second launch in slice order.
//  * Numerics.  w = bits << 16 (exact, NaN/inf/subnormal preserving), one
//    fmaf per product in the FMA kernels (the MFMA kernels multiply exactly
//    and round once per 32-element block), accumulators start at +0.0f
//    (idle lanes at -0.0f, the additive identity), no flush-to-zero
//    (compiled with -fno-gpu-flush-denormals-to-zero, no fast-math, no fp
//    contraction), packed-fp32 disabled.  Fixed reduction order: bit-identical
//    results run to run.
#include "gemv_launch.h"

#include <algorithm>

namespace dmc {
namespace {

constexpr int kWaves = 4;  // waves per workgroup (256 threads)
constexpr int kThreads = 64 * kWaves;

// ---- bf16 vectors ---------------------------------------------------------

// VEC bf16 values loaded by one lane; element e sits in bits [16e, 16e+16).
template <int VEC> struct WVec;
template <> struct WVec<8> {
    uint32_t d[4];
    __device__ __forceinline__ void load(const uint16_t *p) {
        const uint4 v = *reinterpret_cast<const uint4 *>(p);
        d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    }
};
template <> struct WVec<4> {
    uint32_t d[2];
    __device__ __forceinline__ void load(const uint16_t *p) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        d[0] = v.x; d[1] = v.y;
    }
};
template <> struct WVec<2> {
    uint32_t d[1];
    __device__ __forceinline__ void load(const uint16_t *p) {
        d[0] = *reinterpret_cast<const uint32_t *>(p);
    }
};
template <> struct WVec<1> {
    uint32_t d[1];
    __device__ __forceinline__ void load(const uint16_t *p) { d[0] = *p; }
};

// Exact bf16 -> f32 widen of element e (compiler/src/jit.rs:29225-29227).
template <int VEC>
__device__ __forceinline__ float widen(const WVec<VEC> &v, int e) {
    const uint32_t w = v.d[e >> 1];
    return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}

// VEC consecutive f32 activations (the caller guarantees 4*VEC-byte alignment).
template <int VEC>
__device__ __forceinline__ void load_x(const float *p, float (&v)[VEC]) {
    if constexpr (VEC == 8) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        const float4 b = *reinterpret_cast<const float4 *>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else if constexpr (VEC == 4) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else if constexpr (VEC == 2) {
        const float2 a = *reinterpret_cast<const float2 *>(p);
        v[0] = a.x; v[1] = a.y;
    } else {
        v[0] = p[0];
    }
}

// Sum over the 64 lanes of a wave with DPP moves inside each row of 16 lanes
// (xor 1, xor 2, half-row mirror, row mirror), then the four row sums read
// out in a fixed order.  Every lane gets the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_mov<0xb1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Four values of every lane summed over the wave as one reduce-scatter
// instead of four reductions: lane pairs exchange half of what they hold
// (xor 1: two values left, xor 2: one), so lane class c = lane mod 4 sums
// value 2 (c & 1) + (c >> 1) over its quad; rotations by 4 and 8 within
// each row of 16 lanes and the two lane swaps across rows (xor 16, xor 32)
// finish it.  Lane c (c < 4) returns the total of that value; the order of
// the additions is fixed.  15 instructions against 4 x 11.
__device__ __forceinline__ float wave_sum4_dpp(float a0, float a1, float a2, float a3) {
    const bool b0 = (threadIdx.x & 1) != 0, b1 = (threadIdx.x & 2) != 0;
    const float c0 = (b0 ? a2 : a0) + dpp_mov<0xb1>(b0 ? a0 : a2);  // quad_perm [1,0,3,2]
    const float c1 = (b0 ? a3 : a1) + dpp_mov<0xb1>(b0 ? a1 : a3);
    float d = (b1 ? c1 : c0) + dpp_mov<0x4e>(b1 ? c0 : c1);         // quad_perm [2,3,0,1]
    d += dpp_mov<0x124>(d);                                         // row_ror:4
    d += dpp_mov<0x128>(d);                                         // row_ror:8
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(d), __float_as_uint(d), false, false);
    d = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// Two values of every lane summed over the wave the same way: one exchange
// (xor 1) leaves lane class c = lane mod 2 with value c; lane c (c < 2)
// returns its total.
__device__ __forceinline__ float wave_sum2_dpp(float a0, float a1) {
    const bool b0 = (threadIdx.x & 1) != 0;
    float d = (b0 ? a1 : a0) + dpp_mov<0xb1>(b0 ? a0 : a1);  // quad_perm [1,0,3,2]
    d += dpp_mov<0x4e>(d);                                   // quad_perm [2,3,0,1]
    d += dpp_mov<0x124>(d);                                  // row_ror:4
    d += dpp_mov<0x128>(d);                                  // row_ror:8
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(d), __float_as_uint(d), false, false);
    d = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(d), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// The V per-lane values a[0..V) summed over the wave, four (or the last two)
// per reduce-scatter: store(v, total) runs in the one lane that holds value
// v's total.
template <int V, class Store>
__device__ __forceinline__ void wave_sums(const float (&a)[V], Store store) {
    const int lane = threadIdx.x & 63;
    if constexpr (V == 1) {
        const float s = wave_sum_dpp(a[0]);
        if (lane == 0) store(0, s);
    } else {
#pragma unroll
        for (int g = 0; g < V; g += 4) {
            if (V - g == 2) {
                const float s = wave_sum2_dpp(a[g], a[g + 1]);
                if (lane < 2) store(g + lane, s);
            } else {
                const float s = wave_sum4_dpp(a[g], g + 1 < V ? a[g + 1] : 0.0f, g + 2 < V ? a[g + 2] : 0.0f,
                                              g + 3 < V ? a[g + 3] : 0.0f);
                const int v = g + 2 * (lane & 1) + ((lane >> 1) & 1);
                if (lane < 4 && v < V) store(v, s);
            }
        }
    }
}

// 128-bit weight loads through a buffer resource, marked nontemporal: weights
// are streamed once per launch, so they should not displace x or y in the
// caches.  (Measured on MI355X: ~8% more bandwidth than plain global loads.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr int kLoadNT = 2;  // cache-policy bits of a buffer load: nt

__device__ __forceinline__ u32x4 load_w16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kLoadNT);
}

// The same with a wave-uniform part of the offset in the instruction's scalar
// offset.  Measured on gfx950: the range check covers the sum of both offsets
// (per dword), like a single offset.  Keeping a loop's row offset scalar and
// the lane's offset loop-invariant leaves no per-load vector address
// arithmetic, whose temporaries the register allocator otherwise places in
// registers just freed by a load -- and the compiler then waits for that
// load's whole batch before the next one may issue.
__device__ __forceinline__ u32x4 load_w16(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t uniform_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, uniform_off, kLoadNT);
}

__device__ __forceinline__ float widen_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float widen_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---- zero outputs of the FMA kernels ------------------------------------------
//
// The FMA kernels split k, so an output is a sum of partial chains.  When that
// sum comes out exactly 0 it can differ from the reference chain (fmaf over
// ascending k from +0, jit.rs:29655-29670): a run of underflowing products of
// both signs leaves the chain at the zero of the last one's sign, where a sum
// of reordered partials is -0 only if every partial is; and reordered partials
// can cancel exactly where the chain keeps a subnormal residue.  Neither can
// happen when every product is an exact zero (some factor +-0): the chain then
// never leaves +0, and neither does the split sum (lanes with elements start
// at +0, idle ones add -0).  So a zero output is settled by the reference's
// rule: +0 when no product has two nonzero factors -- an all-zero activation
// row, an all-zero weight row, or factors that never meet -- and otherwise
// the chain itself (underflow or exact cancellation, which takes crafted
// data).  The common path costs one compare and one ballot per output.

// The reference chain for one output: K products x[k] * w[k * wstep], any
// alignment (2- and 4-byte loads; the rare path only).
__device__ float chain_strided(const uint16_t *__restrict__ w, int64_t wstep, const float *__restrict__ x, int K) {
    float acc = 0.0f;
    int k = 0;
    for (; k + 4 <= K; k += 4) {
        const uint16_t *p = w + (int64_t)k * wstep;
        const uint32_t b0 = p[0], b1 = p[wstep], b2 = p[2 * wstep], b3 = p[3 * wstep];
        const float x0 = x[k], x1 = x[k + 1], x2 = x[k + 2], x3 = x[k + 3];
        acc = fmaf(x0, __uint_as_float(b0 << 16), acc);
        acc = fmaf(x1, __uint_as_float(b1 << 16), acc);
        acc = fmaf(x2, __uint_as_float(b2 << 16), acc);
        acc = fmaf(x3, __uint_as_float(b3 << 16), acc);
    }
    for (; k < K; ++k) acc = fmaf(x[k], __uint_as_float((uint32_t)w[(int64_t)k * wstep] << 16), acc);
    return acc;
}

template <class T>
__device__ __forceinline__ const T *readlane_ptr(const T *p, int j) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, j);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), j);
    return reinterpret_cast<const T *>(((uint64_t)hi << 32) | lo);
}

// Wave-uniform: does some k have x[k] and (w == nullptr, or w[k * wstep])
// nonzero?  Contiguous rows (wstep <= 1, K <= 2^28): 16-byte buffer loads at
// the rows' own 4- and 2-byte alignments (exact on gfx950), 8 elements per
// lane per load, 4096 per round -- one round for K <= 4096.  The weight range
// ends exactly after element K-1: a load's dword that runs past it comes back
// as zeros (element K-1 itself when it shares such a dword), so element K-1
// is also read alone, 2 bytes, and nothing past the row is ever read.
// Strided columns: one element per lane per load, 64 * 32 per round.  All
// loads of a round are in flight together; the scan stops at the first round
// that finds a product.
__device__ bool wave_any_product(const float *x, const uint16_t *w, int64_t wstep, int K) {
    const int lane = threadIdx.x & 63;
    if (K <= 0) return false;
    if (wstep <= 1 && K <= (1 << 28)) {
        constexpr int U = 8;
        const uintptr_t wb = reinterpret_cast<uintptr_t>(w);
        const __amdgpu_buffer_rsrc_t xr = weight_rsrc(x, (uint32_t)K * 4u);
        const uintptr_t w0 = wb & ~(uintptr_t)3;
        const uint32_t wd = (uint32_t)(wb - w0);  // 0 or 2
        const __amdgpu_buffer_rsrc_t wr =
            weight_rsrc(reinterpret_cast<const void *>(w ? w0 : reinterpret_cast<uintptr_t>(x)),
                        w ? wd + 2u * (uint32_t)K : 0u);
        const uint32_t wl = w ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(wr, wd + 2u * (K - 1), 0, 0) : 1u;
        const uint32_t xl = __float_as_uint(x[K - 1]) & 0x7fffffffu;
        bool first = true;
        for (int k0 = 0; k0 < K; k0 += 512 * U) {
            u32x4 xa[U], xc[U], wv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t e = (uint32_t)(k0 + (u * 64 + lane) * 8);
                xa[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, e * 4u, 0, 0);
                xc[u] = __builtin_amdgcn_raw_buffer_load_b128(xr, e * 4u + 16u, 0, 0);
                wv[u] = w ? __builtin_amdgcn_raw_buffer_load_b128(wr, wd + e * 2u, 0, 0) : u32x4{~0u, ~0u, ~0u, ~0u};
            }
            uint32_t hit = first && (wl & 0x7fffu) != 0 && xl != 0 ? 1u : 0u;
            first = false;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = k0 + (u * 64 + lane) * 8;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t xv = (i < 4 ? xa[u][i] : xc[u][i - 4]) & 0x7fffffffu;
                    const uint32_t wv16 = (wv[u][i >> 1] >> (16 * (i & 1))) & 0x7fffu;
                    hit |= (e + i < K && xv != 0 && wv16 != 0) ? 1u : 0u;
                }
            }
            if (__builtin_amdgcn_ballot_w64(hit != 0) != 0) return true;
        }
        return false;
    }
    constexpr int U = 32;
    for (int k0 = 0; k0 < K; k0 += 64 * U) {
        uint32_t xb[U], wb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(k0 + u * 64 + lane, K - 1);
            xb[u] = __float_as_uint(x[k]) & 0x7fffffffu;
            wb[u] = w ? (uint32_t)w[(int64_t)k * wstep] & 0x7fffu : 1u;
        }
        uint32_t hit = 0;
#pragma unroll
        for (int u = 0; u < U; ++u) hit |= (k0 + u * 64 + lane < K && xb[u] != 0 && wb[u] != 0) ? 1u : 0u;
        if (__builtin_amdgcn_ballot_w64(hit != 0) != 0) return true;
    }
    return false;
}

// The zero rule for the outputs this wave holds, one per lane: `zero` marks a
// lane whose output s is exactly 0 and is stored; x is its activation row,
// w its first weight, wstep the elements between consecutive k.  All 64 lanes
// call it (wave-uniform control flow): rows are scanned by the whole wave,
// one output at a time, and the chains (if any) run one per lane.
__device__ float settle_zero(float s, bool zero, const float *x, const uint16_t *w, int64_t wstep, int K) {
    uint64_t pend = __builtin_amdgcn_ballot_w64(zero);
    if (pend == 0) return s;
    const int lane = threadIdx.x & 63;
    // activation rows that hold only +-0, each distinct row scanned once (a
    // lone zero output skips this: its product scan covers its row)
    bool xnz = true;
    if (pend & (pend - 1)) while (pend) {
        const int j = __builtin_ctzll(pend);
        const float *xj = readlane_ptr(x, j);
        const bool nz = wave_any_product(xj, nullptr, 0, K);
        const bool same = zero && x == xj;
        if (same) xnz = nz;
        pend &= ~__builtin_amdgcn_ballot_w64(same);
    }
    // outputs whose products all have a zero factor
    bool chain = false;
    for (uint64_t todo = __builtin_amdgcn_ballot_w64(zero && xnz); todo; todo &= todo - 1) {
        const int j = __builtin_ctzll(todo);
        const bool hit = wave_any_product(readlane_ptr(x, j), readlane_ptr(w, j), wstep, K);
        if (lane == j) chain = hit;
    }
    if (zero) s = chain ? chain_strided(w, wstep, x, K) : 0.0f;
    return s;
}

// The column-stream kernels and the row-dot kernels that keep x in registers
// settle zeros without scanning (a column-stream weight column is N elements
// apart in memory, too far to re-read cheaply; a row-dot workgroup is short
// lived, and every wave but the storing one should leave at its last
// barrier).  Each lane
// tracks whether any of its products had two nonzero factors and folds that
// into the sign of an exactly-zero partial: -0 for none, +0 otherwise.  The
// fold survives every later sum -- (-0) + (-0) = -0, (-0) + (+0) = +0, and a
// nonzero term wins -- so the final sum is -0 exactly when no product
// anywhere had two nonzero factors (the reference chain is then +0), +0 when
// the products underflowed or cancelled (the rare case: the chain itself),
// and otherwise the value.  Non-finite partials pass through unchanged.
__device__ __forceinline__ float zero_fold(float acc, bool has_product) {
    return acc == 0.0f ? (has_product ? 0.0f : -0.0f) : acc;
}

// 0x7fff in the low half when a is nonzero and in the high half when b is:
// ANDed with a dword holding two bf16 weights, nonzero exactly when one of the
// two products (a with the low weight, b with the high one) has two nonzero
// factors.  Computed once per x window; the streaming loops then track
// products with one AND-OR per weight dword, branch-free.
__device__ __forceinline__ uint32_t nonzero_pair(float a, float b) {
    return ((__float_as_uint(a) & 0x7fffffffu) != 0 ? 0x00007fffu : 0u) |
           ((__float_as_uint(b) & 0x7fffffffu) != 0 ? 0x7fff0000u : 0u);
}

// The final rule on a folded sum for one output (per lane; the chain is the
// rare path).
__device__ __forceinline__ float zero_unfold(float v, bool live, const float *x, const uint16_t *w, int64_t wstep,
                                             int K) {
    if (live && v == 0.0f) v = __builtin_signbit(v) ? 0.0f : chain_strided(w, wstep, x, K);
    return v;
}

// The zero rule for the row-dot kernel with x in LDS (one long-lived
// workgroup per CU), run after the workgroup's last barrier, with no cost in
// the streaming loop.  total(t) gives output
// t's sum (t < count).  Wave 0 alone stores every nonzero sum and notes in
// LDS (`hits[NWAVES]`) whether any sum was exactly zero; the other waves wait
// for that note at one barrier.  Only then (the rare path) do all waves
// evaluate the totals again, in the same order, so they meet the same zero
// outputs: lane_hit(t) re-reads the windows this lane summed for output t and
// says whether one of its products had two nonzero factors, and the waves'
// answers meet in LDS (`hits[0..NWAVES)`, one word per wave).  A zero output
// then gets +0 (no such product: every product was an exact zero, so the
// reference chain never leaves +0) or chain(t) (the products underflowed or
// cancelled), stored by wave 0.  `hits` holds NWAVES + 1 words.
template <int NWAVES, class Total, class Hit, class Chain, class Store>
__device__ __forceinline__ void rd_finish(int count, uint64_t *hits, Total total, Hit lane_hit, Chain chain,
                                          Store store) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave == 0) {
        uint64_t any = 0;
        for (int t0 = 0; t0 < count; t0 += 64) {
            const int t = t0 + lane;
            if (t < count) {
                const float v = total(t);
                if (v != 0.0f) store(t, v);
                else any = 1;
            }
        }
        any = __builtin_amdgcn_ballot_w64(any != 0);
        if (lane == 0) hits[NWAVES] = any;
    }
    __syncthreads();
    if (hits[NWAVES] == 0) return;
    for (int t0 = 0; t0 < count; t0 += 64) {
        const int t = t0 + lane;
        const bool live = t < count;
        const float v = live ? total(t) : 1.0f;
        const uint64_t zm = __builtin_amdgcn_ballot_w64(live && v == 0.0f);
        if (zm == 0) continue;  // the same in every wave: the barriers below are safe
        uint64_t mine = 0;
        for (uint64_t b = zm; b; b &= b - 1) {
            const int j = __builtin_ctzll(b);
            if (__builtin_amdgcn_ballot_w64(lane_hit(t0 + j)) != 0) mine |= 1ull << j;
        }
        if (lane == 0) hits[wave] = mine;
        __syncthreads();
        uint64_t has = 0;
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) has |= hits[w];
        __syncthreads();  // hits is reused by the next chunk
        if (wave == 0 && live && v == 0.0f) store(t, ((has >> lane) & 1) ? chain(t) : 0.0f);
    }
}

// Does some e have x[e] and the bf16 at half e of w nonzero?  (8 elements)
__device__ __forceinline__ bool window_hit(const float (&x)[8], const u32x4 &w) {
    bool hit = false;
#pragma unroll
    for (int e = 0; e < 8; ++e)
        hit |= (__float_as_uint(x[e]) & 0x7fffffffu) != 0 && ((w[e >> 1] >> (16 * (e & 1))) & 0x7fffu) != 0;
    return hit;
}

// ---- RD streaming: W [N,K], 16-byte aligned rows, K <= 32768 ------------------
//
// One launch serves up to kMaxGroup independent problems sharing K and M
// (a single GEMV is a group of one); each workgroup first finds its problem.
//
// The NW waves of a workgroup split k: lane `lane` of wave `wave` owns the
// KV vectors of 8 elements starting at ((j*NW + wave)*64 + lane)*8, j < KV, so
// for every j the workgroup reads NW*1 KiB of a row contiguously.  The lane
// loads its x slice (MT activation rows) into registers once, then the
// workgroup walks weight rows [rb, rb+rpw) ROWS at a time through two
// register buffers: the next ROWS rows are in flight while the current ones
// are summed.  Each (activation row, weight row) partial is reduced across
// the wave with DPP and parked in LDS; one barrier at the end, then a
// fixed-order sum over the waves.
//
// Every load is unconditional, so the compiler can count the loads in flight
// and wait only for the buffer being summed (a load under a branch makes it
// wait for all of them, which serialises the two buffers).  A lane that owns
// no element, and a row past the workgroup's last, load from offset
// kOutOfRange, beyond the buffer resource's size: the hardware returns zeros
// and reads no memory.
constexpr int kMaxRpw = 64;
constexpr uint32_t kOutOfRange = 0x80000000u;

// Kernel-argument form of RdGroup: problem g owns workgroups
// [gstart[g], gstart[g+1]) of the launch.
struct RdGroupArgs {
    const uint16_t *w[kMaxGroup];
    const float *x[kMaxGroup];
    float *y[kMaxGroup];
    int n[kMaxGroup];
    int gstart[kMaxGroup + 1];
    int count;
};

// GROUP = false: a single problem, read straight from entry 0 of the
// arguments.  GROUP = true: the problem index is counted branch-free from
// gstart (entries past the last problem hold INT32_MAX), so all of gstart
// arrives in one scalar load; a search loop would chain dependent scalar
// loads before the first weight load (measured 0.3-1 us per launch).
template <int NW, int KV, int ROWS, int MT, bool GROUP>
__global__ void __launch_bounds__(64 * NW)
gemv_rd_stream_kernel(const RdGroupArgs ga, int K, int M, int rpw) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int gi = 0;
    if constexpr (GROUP) {
#pragma unroll
        for (int g = 1; g < kMaxGroup; ++g) gi += (int)blockIdx.x >= ga.gstart[g] ? 1 : 0;
    }
    const uint16_t *__restrict__ W = ga.w[gi];
    const float *__restrict__ X = ga.x[gi];
    float *__restrict__ Y = ga.y[gi];
    const int N = ga.n[gi];
    const int64_t ldw = K, ldy = N;
    // The workgroup's rows: [rb, rb + nr).
    const int rb = ((int)blockIdx.x - ga.gstart[gi]) * rpw;
    const int nr = min(N, rb + rpw) - rb;
    const int m0 = blockIdx.y * MT;
    const int mrows = min(MT, M - m0);

    // x rows [m0, m0 + mrows): activation row m0 + m reads row min(m, mrows - 1).
    const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X + (int64_t)m0 * K, (uint32_t)mrows * (uint32_t)K * 4);
    uint32_t eoff[KV];
    bool has[KV];
    u32x4 xa[MT][KV], xb[MT][KV];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int e = ((j * NW + wave) * 64 + lane) * 8;
        has[j] = e < K;
        eoff[j] = has[j] ? (uint32_t)e * 2 : kOutOfRange;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint32_t xo = has[j] ? ((uint32_t)min(m, mrows - 1) * (uint32_t)K + (uint32_t)e) * 4 : kOutOfRange;
            xa[m][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0);
            xb[m][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 16, 0, 0);
        }
    }
    // +0.0f for a lane that owns elements (the reference's chain start,
    // jit.rs:29655), -0.0f, the additive identity, for a lane that owns none.
    const float init = (wave * 64 + lane) * 8 < K ? 0.0f : -0.0f;

    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(W + (int64_t)rb * ldw, (uint32_t)((int64_t)nr * ldw * 2));
    const uint32_t row_bytes = (uint32_t)ldw * 2;
    __shared__ float red[NW][MT][kMaxRpw];

    // Row rb + i sits at i * row_bytes; rows i >= nr fall past the
    // resource's range (the planner keeps rpw rows below 2^31 bytes).
    u32x4 ba[ROWS][KV], bb[ROWS][KV];
    auto load = [&](u32x4 (&wv)[ROWS][KV], int i0) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            const uint32_t base = (uint32_t)(i0 + q) * row_bytes;
#pragma unroll
            for (int j = 0; j < KV; ++j) wv[q][j] = load_w16(rs, eoff[j], base);
        }
    };
    load(ba, 0);
    float xr[MT][KV][8];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                xr[m][j][q] = __uint_as_float(xa[m][j][q]);
                xr[m][j][q + 4] = __uint_as_float(xb[m][j][q]);
            }
    // A vector past K reads +0 weights (past the resource's range); its x
    // becomes -0.0f, so each of its products is -0.0f, the exact additive
    // identity: it leaves any chain unchanged, a -0.0f (a product that
    // underflowed) included.  Applied once, after both weight buffers' loads
    // are in flight (the sign bit needs x to have arrived), so the loop's
    // widen stays one shift or mask per weight.
    auto pad_x = [&]() {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < KV; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    xr[m][j][e] = __uint_as_float(__float_as_uint(xr[m][j][e]) | (has[j] ? 0u : 0x80000000u));
    };

    // xm: nonzero_pair of each x dword pair, set once x has arrived.  Each
    // lane's partial is zero-folded before the wave sum (zero_fold).
    uint32_t xm[MT][KV][4];
    auto sum_rows = [&](const u32x4 (&wv)[ROWS][KV], int i0) {
        float acc[MT][ROWS];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int q = 0; q < ROWS; ++q) acc[m][q] = init;
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int q = 0; q < ROWS; ++q) {
                    const uint32_t d = wv[q][j][e >> 1];
                    const float w = (e & 1) ? widen_hi(d) : widen_lo(d);
#pragma unroll
                    for (int m = 0; m < MT; ++m) acc[m][q] = fmaf(xr[m][j][e], w, acc[m][q]);
                }
        // Value v of the step: activation row v / ROWS, weight row i0 + v % ROWS.
        float a[MT * ROWS];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                uint32_t nz = 0;
#pragma unroll
                for (int j = 0; j < KV; ++j)
#pragma unroll
                    for (int d = 0; d < 4; ++d) nz |= wv[q][j][d] & xm[m][j][d];
                a[m * ROWS + q] = zero_fold(acc[m][q], nz != 0);
            }
        wave_sums(a, [&](int v, float s) {
            if (i0 + v % ROWS < nr) red[wave][v / ROWS][i0 + v % ROWS] = s;
        });
    };
    // Rows [i0, i0 + ROWS) sit in one buffer while the next ROWS rows load
    // into the other; the first step is peeled so that pad_x follows the
    // second buffer's loads.
    load(bb, ROWS);
    __builtin_amdgcn_sched_barrier(0);  // keep pad_x's wait for x after every load above
    pad_x();
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int d = 0; d < 4; ++d) xm[m][j][d] = nonzero_pair(xr[m][j][2 * d], xr[m][j][2 * d + 1]);
    sum_rows(ba, 0);
    for (int i0 = 0; i0 + ROWS < nr; i0 += 2 * ROWS) {
        load(ba, i0 + 2 * ROWS);
        sum_rows(bb, i0 + ROWS);
        if (i0 + 2 * ROWS >= nr) break;
        load(bb, i0 + 3 * ROWS);
        sum_rows(ba, i0 + 2 * ROWS);
    }
    __syncthreads();
    // Only the waves that hold outputs stay (wave-uniform, so the rare chain's
    // loads are too); the others leave, freeing their slots for the next
    // workgroup.
    for (int t0 = wave * 64; t0 < mrows * nr; t0 += 64 * NW) {
        const int t = t0 + lane;
        const bool live = t < mrows * nr;
        const int m = live ? t / nr : 0, r = live ? t - m * nr : 0;
        float s = red[0][m][r];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w][m][r];
        s = zero_unfold(s, live, X + (int64_t)(m0 + m) * K, W + (int64_t)(rb + r) * ldw, 1, K);
        if (live) Y[(int64_t)(m0 + m) * ldy + rb + r] = s;
    }
}

// ---- RD streaming, two 8-wave halves sharing x through LDS (M = 1, long rows) ----
//
// gemv_rd_stream_kernel's layout with one 16-wave workgroup per CU in place
// of two 8-wave ones: each half walks its own rpw/2 consecutive rows exactly
// as an 8-wave workgroup does (k split over its 8 waves, two register
// buffers, unconditional loads), but x is read from L2 once per workgroup,
// into LDS, and every lane takes its windows from there.  At K = 14336 this
// halves x's L2 traffic (each 8-wave workgroup otherwise streams all 56 KiB
// of x at kernel start, 28 MiB per launch).
constexpr int kXldsMaxK = 16384;  // x in LDS: 64 KiB; KV <= 4 windows per lane

template <int KV, int ROWS>
__global__ void __launch_bounds__(1024)
gemv_rd_stream_xlds_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y,
                           int N, int K, int rpw) {
    static_assert(KV <= 4, "x windows must lie inside the LDS copy");
    constexpr int NW = 8;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wave = wid & (NW - 1), half = wid / NW;
    const int hrows = rpw / 2;
    const int rb = (int)blockIdx.x * rpw + half * hrows;  // this half's rows: [rb, rb + nr)
    const int nr = max(0, min(N, rb + hrows) - rb);
    // x in LDS as two planes: window w's first 4 elements at lo[4w], its last
    // 4 at hi[4w], so a wave reading one half of 64 consecutive windows (and
    // writing them) touches 1 KiB of consecutive bytes: no bank conflicts
    // (windows read whole at a 32-byte stride conflicted on 29% of the LDS
    // cycles, rocprof SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE).
    __shared__ __attribute__((aligned(16))) float xs[kXldsMaxK];
    constexpr int kHi = kXldsMaxK / 2;
    __shared__ float red[2][NW][kMaxRpw / 2];

    // x into registers: thread t takes windows t and t + 1024, each whole
    // (two 16-byte loads; windows past K read as zeros from past the
    // resource's range).
    const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X, (uint32_t)K * 4);
    u32x4 xp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        xp[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (threadIdx.x + (i >> 1) * 1024u) * 32u + (i & 1) * 16u, 0, 0);

    uint32_t eoff[KV];
    bool has[KV];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int e = ((j * NW + wave) * 64 + lane) * 8;
        has[j] = e < K;
        eoff[j] = has[j] ? (uint32_t)e * 2 : kOutOfRange;
    }
    const float init = (wave * 64 + lane) * 8 < K ? 0.0f : -0.0f;
    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(W + (int64_t)rb * K, (uint32_t)((int64_t)nr * K * 2));
    const uint32_t row_bytes = (uint32_t)K * 2;
    u32x4 ba[ROWS][KV], bb[ROWS][KV];
    auto load = [&](u32x4 (&wv)[ROWS][KV], int i0) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            const uint32_t base = (uint32_t)(i0 + q) * row_bytes;
#pragma unroll
            for (int j = 0; j < KV; ++j) wv[q][j] = load_w16(rs, eoff[j], base);
        }
    };
    load(ba, 0);
    load(bb, ROWS);
    __builtin_amdgcn_sched_barrier(0);  // both weight buffers in flight before the wait for x
#pragma unroll
    for (int i = 0; i < 4; ++i)
        *reinterpret_cast<u32x4 *>(&xs[(i & 1) * kHi + (threadIdx.x + (i >> 1) * 1024u) * 4u]) = xp[i];
    __syncthreads();
    // The lane's windows; a window past K (zeros in LDS) gets x = -0.0f, so
    // its products with the +0 weights read past the range are -0.0f, the
    // exact additive identity.
    float xr[KV][8];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int w = (j * NW + wave) * 64 + lane;
        const u32x4 a = *reinterpret_cast<const u32x4 *>(&xs[w * 4]);
        const u32x4 b = *reinterpret_cast<const u32x4 *>(&xs[kHi + w * 4]);
        const uint32_t sgn = has[j] ? 0u : 0x80000000u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xr[j][q] = __uint_as_float(a[q] | sgn);
            xr[j][q + 4] = __uint_as_float(b[q] | sgn);
        }
    }
    auto sum_rows = [&](const u32x4 (&wv)[ROWS][KV], int i0) {
        float acc[ROWS];
#pragma unroll
        for (int q = 0; q < ROWS; ++q) acc[q] = init;
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int q = 0; q < ROWS; ++q) {
                    const uint32_t d = wv[q][j][e >> 1];
                    acc[q] = fmaf(xr[j][e], (e & 1) ? widen_hi(d) : widen_lo(d), acc[q]);
                }
        wave_sums(acc, [&](int q, float s) {
            if (i0 + q < nr) red[half][wave][i0 + q] = s;
        });
    };
    sum_rows(ba, 0);
    for (int i0 = 0; i0 + ROWS < nr; i0 += 2 * ROWS) {
        load(ba, i0 + 2 * ROWS);
        sum_rows(bb, i0 + ROWS);
        if (i0 + 2 * ROWS >= nr) break;
        load(bb, i0 + 3 * ROWS);
        sum_rows(ba, i0 + 2 * ROWS);
    }
    __syncthreads();
    __shared__ uint64_t hits[2 * NW + 1];
    const int rows_here = max(0, min(rpw, N - (int)blockIdx.x * rpw));  // outputs t = h * hrows + r
    rd_finish<2 * NW>(
        rows_here, hits,
        [&](int t) {
            const int h = t / hrows, r = t - h * hrows;
            float s = red[h][0][r];
#pragma unroll
            for (int w = 1; w < NW; ++w) s += red[h][w][r];
            return s;
        },
        [&](int t) {  // only the waves of the half that summed row t; x from its LDS copy
            const int h = t / hrows, r = t - h * hrows;
            bool hit = false;
            if (h == half)
#pragma unroll
                for (int j = 0; j < KV; ++j) {
                    const int w = (j * NW + wave) * 64 + lane;
                    const u32x4 a = *reinterpret_cast<const u32x4 *>(&xs[w * 4]);
                    const u32x4 b = *reinterpret_cast<const u32x4 *>(&xs[kHi + w * 4]);
                    const float xw[8] = {__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]),
                                         __uint_as_float(a[3]), __uint_as_float(b[0]), __uint_as_float(b[1]),
                                         __uint_as_float(b[2]), __uint_as_float(b[3])};
                    hit |= window_hit(xw, load_w16(rs, eoff[j], (uint32_t)r * row_bytes));
                }
            return hit;
        },
        [&](int t) { return chain_strided(W + (int64_t)((int)blockIdx.x * rpw + t) * K, 1, X, K); },
        [&](int t, float v) { Y[(int)blockIdx.x * rpw + t] = v; });
}

// ---- RD streaming, one group of 14 waves (M = 1 to 4, long rows) -------------
//
// One group of NS = 14 waves splits k: lane t of the workgroup owns the KV
// 16-byte windows t + j*NT of a row (NT = 896 threads; 8 bf16 or 4 f32
// weights each), so at K = 14336 every load instruction carries data.  The
// same layout on NS = 8 waves (NT = 512, one window per lane) serves bf16
// rows of K <= 4096, three or four workgroups to a CU, and on NS = 4 rows of
// K <= 2048.  A
// window's x is the lane's alone, so each lane loads its MT activation rows'
// windows straight into registers (56 KiB of x per activation row and
// workgroup, one workgroup per CU).  The workgroup's 16 rows stream ROWS at a
// time through two register buffers with unconditional loads and no barrier
// until the end, where wave 0 sums each row's 14 partials in wave order and
// rd_finish settles exact zeros (its rare path reads x again from memory).
// Every weight load feeds all MT activation rows' fma chains.  Output
// (activation row m, weight row n) goes to Y[m * ys_act + n * ys_row].
constexpr int kX14Waves = 14;
constexpr int kX14MaxK = 2 * kX14Waves * 512;  // 14336: KV <= 2 (bf16), 4 (f32)
constexpr int kX14MaxM = 4;

__device__ float chain_f32(const float *__restrict__ w, const float *__restrict__ x, int K);

template <typename WT, int KV, int MT, int NS, int RPW_ = 16, int ROWS_ = 0>
__device__ __forceinline__ void rd_group_body(const WT *__restrict__ W, const float *__restrict__ X,
                                              float *__restrict__ Y, int N, int K, int64_t ys_act, int64_t ys_row) {
    constexpr bool F32 = sizeof(WT) == 4;
    constexpr int EW = 16 / sizeof(WT);  // weights per window
    // Rows per register buffer (a lane has 128 registers at 14 waves per CU;
    // x takes EW * KV * MT of them): bf16 4 at MT = 1, 2 at MT = 2 and 3, 1
    // at MT = 4 with two windows (122 registers in all at KV = 2, MT = 3);
    // f32 2 up to MT = 2, then 1.  On 8 waves (KV = 1) the same rows take 54
    // to 76 registers.
    constexpr int ROWS = ROWS_ ? ROWS_ : F32 ? (MT <= 2 ? 2 : 1) : MT == 1 ? 4 : MT == 4 && KV == 2 ? 1 : 2;
    constexpr int NT = 64 * NS, RPW = RPW_;
    static_assert(RPW % ROWS == 0, "rows per workgroup");
    static_assert(KV * NS * 64 * EW <= kX14MaxK, "windows");
    static_assert(MT >= 1 && MT <= kX14MaxM, "activation rows");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = (int)blockIdx.x * RPW;
    const int nr = max(0, min(N, rb + RPW) - rb);

    __shared__ float red[NS][MT * RPW];

    // The lane's x windows (EW floats: one or two 16-byte halves), issued
    // ahead of the weights.
    constexpr int XH = EW / 4;
    u32x4 xp[MT][KV][XH];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X + (int64_t)m * K, (uint32_t)K * 4);
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int h = 0; h < XH; ++h)
                xp[m][j][h] =
                    __builtin_amdgcn_raw_buffer_load_b128(xrs, (threadIdx.x + j * NT) * (4u * EW) + h * 16u, 0, 0);
    }
    uint32_t eoff[KV];
    bool has[KV];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int e = (threadIdx.x + j * NT) * EW;
        has[j] = e < K;
        eoff[j] = has[j] ? (uint32_t)e * (uint32_t)sizeof(WT) : kOutOfRange;
    }
    const float init = (int)threadIdx.x * EW < K ? 0.0f : -0.0f;
    const uint32_t row_bytes = (uint32_t)K * (uint32_t)sizeof(WT);
    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(W + (int64_t)rb * K, (uint32_t)nr * row_bytes);
    u32x4 ba[ROWS][KV], bb[ROWS][KV];
    auto load = [&](u32x4 (&wv)[ROWS][KV], int i0) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q)
#pragma unroll
            for (int j = 0; j < KV; ++j) wv[q][j] = load_w16(rs, eoff[j], (uint32_t)(i0 + q) * row_bytes);
    };
    load(ba, 0);
    if constexpr (ROWS < RPW) load(bb, ROWS);
    __builtin_amdgcn_sched_barrier(0);
    float xr[MT][KV][EW];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < KV; ++j) {
            const uint32_t sgn = has[j] ? 0u : 0x80000000u;
#pragma unroll
            for (int e = 0; e < EW; ++e) xr[m][j][e] = __uint_as_float(xp[m][j][e >> 2][e & 3] | sgn);
        }
    auto sum_rows = [&](const u32x4 (&wv)[ROWS][KV], int i0) {
        float acc[MT][ROWS];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int q = 0; q < ROWS; ++q) acc[m][q] = init;
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int e = 0; e < EW; ++e)
#pragma unroll
                for (int q = 0; q < ROWS; ++q) {
                    float wf;
                    if constexpr (F32) {
                        wf = __uint_as_float(wv[q][j][e]);
                    } else {
                        const uint32_t d = wv[q][j][e >> 1];
                        wf = (e & 1) ? widen_hi(d) : widen_lo(d);
                    }
#pragma unroll
                    for (int m = 0; m < MT; ++m) acc[m][q] = fmaf(xr[m][j][e], wf, acc[m][q]);
                }
        // Value v of the step: activation row v / ROWS, weight row i0 + v % ROWS.
        float a[MT * ROWS];
#pragma unroll
        for (int v = 0; v < MT * ROWS; ++v) a[v] = acc[v / ROWS][v % ROWS];
        wave_sums(a, [&](int v, float s) { red[wave][(v / ROWS) * RPW + i0 + v % ROWS] = s; });
    };
#pragma unroll
    for (int i0 = 0; i0 < RPW; i0 += 2 * ROWS) {
        sum_rows(ba, i0);
        if (i0 + 2 * ROWS < RPW) load(ba, i0 + 2 * ROWS);
        if (i0 + ROWS < RPW) {
            sum_rows(bb, i0 + ROWS);
            if (i0 + 3 * ROWS < RPW) load(bb, i0 + 3 * ROWS);
        }
    }
    __syncthreads();
    // Outputs t < MT * nr: activation row t / nr, weight row t % nr.
    __shared__ uint64_t hits[NS + 1];
    rd_finish<NS>(
        MT * nr, hits,
        [&](int t) {
            const int m = MT == 1 ? 0 : t / nr, r = MT == 1 ? t : t - m * nr;
            float s = red[0][m * RPW + r];
#pragma unroll
            for (int w = 1; w < NS; ++w) s += red[w][m * RPW + r];
            return s;
        },
        [&](int t) {
            const int m = MT == 1 ? 0 : t / nr, r = MT == 1 ? t : t - m * nr;
            const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X + (int64_t)m * K, (uint32_t)K * 4);
            bool hit = false;
#pragma unroll
            for (int j = 0; j < KV; ++j) {
                const uint32_t xo = (threadIdx.x + j * NT) * (4u * EW);
                const u32x4 wv = load_w16(rs, eoff[j], (uint32_t)r * row_bytes);
                if constexpr (F32) {
                    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) hit |= (a[e] & 0x7fffffffu) != 0 && (wv[e] & 0x7fffffffu) != 0;
                } else {
                    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0);
                    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 16u, 0, 0);
                    const float xw[8] = {__uint_as_float(a[0]), __uint_as_float(a[1]), __uint_as_float(a[2]),
                                         __uint_as_float(a[3]), __uint_as_float(b[0]), __uint_as_float(b[1]),
                                         __uint_as_float(b[2]), __uint_as_float(b[3])};
                    hit |= window_hit(xw, wv);
                }
            }
            return hit;
        },
        [&](int t) {
            const int m = MT == 1 ? 0 : t / nr, r = MT == 1 ? t : t - m * nr;
            if constexpr (F32)
                return chain_f32(W + (int64_t)(rb + r) * K, X + (int64_t)m * K, K);
            else
                return chain_strided(W + (int64_t)(rb + r) * K, 1, X + (int64_t)m * K, K);
        },
        [&](int t, float v) {
            const int m = MT == 1 ? 0 : t / nr, r = MT == 1 ? t : t - m * nr;
            Y[(int64_t)m * ys_act + (int64_t)(rb + r) * ys_row] = v;
        });
}

template <typename WT, int KV, int MT>
__global__ void __launch_bounds__(64 * kX14Waves)
gemv_rd_stream_x14_kernel(const WT *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N, int K,
                          int64_t ys_act, int64_t ys_row) {
    rd_group_body<WT, KV, MT, kX14Waves>(W, X, Y, N, K, ys_act, ys_row);
}

// The same on one group of 8 waves (bf16 rows of K <= 4096) or of 4 (K <=
// 2048), one window per lane.
template <int MT>
__global__ void __launch_bounds__(512)
gemv_rd_stream_x8_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                         int K, int64_t ys_act, int64_t ys_row) {
    rd_group_body<uint16_t, 1, MT, 8>(W, X, Y, N, K, ys_act, ys_row);
}

template <int MT>
__global__ void __launch_bounds__(256)
gemv_rd_stream_x4_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                         int K, int64_t ys_act, int64_t ys_row) {
    rd_group_body<uint16_t, 1, MT, 4>(W, X, Y, N, K, ys_act, ys_row);
}

template <int MT>
__global__ void __launch_bounds__(512)
gemv_rd_stream_x8f_kernel(const float *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                          int K, int64_t ys_act, int64_t ys_row) {
    rd_group_body<float, 2, MT, 8>(W, X, Y, N, K, ys_act, ys_row);
}

// One 8-wave group per CU: RPW rows per workgroup (N = RPW * CUs), ROWS per
// register buffer, MT activation rows.
template <int RPW, int ROWS, int MT = 1>
__global__ void __launch_bounds__(512)
gemv_rd_stream_x8r_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                          int K, int64_t ys_act, int64_t ys_row) {
    rd_group_body<uint16_t, 1, MT, 8, RPW, ROWS>(W, X, Y, N, K, ys_act, ys_row);
}

// ---- RD streaming, rows at any 2-byte alignment (odd K, offset views) ----------
//
// The layout of gemv_rd_stream_kernel (NW waves split k; lane l of wave w
// owns the 8-element windows p = (j*NW + w)*64 + l of every row, x windows
// in registers, two register buffers of ROWS rows, unconditional loads), for
// rows that do not start on a 16-byte boundary.
//
// Every weight load is a 128-bit buffer load at a 4-byte-aligned offset:
// rows at 2 mod 4 bytes are read from the dword boundary below them, so the
// lane's window then holds elements 8p - 1 .. 8p + 6 (a shift h = 1), and
// its x window is shifted the same way once per workgroup.  Measured on
// gfx950 at C5's size (W[11008, K]): rows at 4- or 8-byte alignment stream at
// 15.4-15.8 us, rows at 2-byte alignment read there directly 17.4-17.8 us.
// For the shift to be one per workgroup all its rows share their alignment:
// with ldw odd (rows alternate between 0 and 2 mod 4), rstep = 2 (`rsh` = 1) and
// workgroup pair (2b, 2b + 1) takes the even and the odd rows of one block of
// 2 * rpw consecutive rows; otherwise rstep = 1 and a workgroup takes rpw
// consecutive rows.
//
// The descriptor starts on the 4-byte boundary at or below the workgroup's
// first row and ends on the dword that holds its last row's last element
// (at most 2 bytes past the matrix, in the same dword and so the same page);
// the range check is per dword, so loads past it return zeros.  Elements
// outside [0, K) (the neighbouring rows' bits may be inf or NaN), whole
// windows past K included, become bf16 -0.0 (0x8000); their x is +0.0 (read
// past either end of x), so each such product is -0.0f, the exact additive
// identity, and padding never turns a -0.0f chain into +0.0f.  M == 1.
//
// Short tail: the windows cover elements [0, kmh), kmh = min(kmain, C - h)
// with C = 8 * KV * NW * 64; the 0 to 8 elements [kmh, K) past the last
// whole block of windows (K = 4097: one, or two on shifted rows) are read
// element by element per row, issued once per workgroup before the stream
// starts by lane i of the last wave for the workgroup's row i, and summed by
// that lane into a ninth partial.  A last block holding one element would
// otherwise double every lane's loads for it (K = 4097 measured 53% of peak
// that way).
template <int NW, int KV, int ROWS>
__global__ void __launch_bounds__(64 * NW)
gemv_rd_unaligned_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                         int K, int kmain, int64_t ldw, int rpw, int rsh) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The workgroup's rows: rb + rstep * i, i < nr, rstep = 1 << rsh.  (Shifts,
    // not divisions: a division is expanded on the vector unit, and every
    // value derived from it -- the loop bounds, the row offsets -- would
    // follow it into vector registers.)
    const int rstep = 1 << rsh;
    const int blk = (int)blockIdx.x >> rsh;
    const int rb = (blk << rsh) * rpw + ((int)blockIdx.x - (blk << rsh));
    // nr = 0 for the odd half of a last block with a single row: its
    // descriptor's range is then empty, so every load returns zeros, and it
    // stores nothing.  (No early return: the exit test would have to wait for
    // its kernel arguments before the other arguments are even requested.)
    const int nr = rb < N ? min(rpw, ((N - 1 - rb) >> rsh) + 1) : 0;
    const int64_t rlast = rb + (int64_t)max(nr - 1, 0) * rstep;

    const uintptr_t base = reinterpret_cast<uintptr_t>(W + (int64_t)rb * ldw) & ~(uintptr_t)3;
    const uintptr_t end = reinterpret_cast<uintptr_t>(W + rlast * ldw + K);
    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(
        reinterpret_cast<const void *>(base), nr > 0 ? (uint32_t)((end - base + 3) & ~(uintptr_t)3) : 0u);
    const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X, (uint32_t)K * 4u);

    // Row i's first element, in bytes from the descriptor's base.  No branch
    // on i < nr (a branch around a load address makes the compiler wait for
    // every load in flight): a row past the last yields offsets past the
    // range's end, which read zeros, and its sum is never stored.
    auto row_off = [&](int i) -> uint32_t {
        return (uint32_t)(reinterpret_cast<uintptr_t>(W + (rb + (int64_t)rstep * i) * ldw) - base);
    };
    const int h = (int)((row_off(0) >> 1) & 1);  // every row's shift, in elements
    const int kmh = min(kmain, KV * NW * 512 - h);

    // The short tail's weights, loaded by the last wave only (lane i for row
    // i), before any other load: the first wait covers them, so the branch
    // adds no wait of its own.  Element by element (2-byte loads), none past
    // element K-1.  Its x comes through the scalar cache.
    const int rem = K - kmh;  // 0 .. 8
    uint32_t tw[8] = {};
    if (rem > 0 && wave == NW - 1) {
        const uint32_t tbase = lane < nr ? row_off(lane) + (uint32_t)kmh * 2u : kOutOfRange;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            tw[e] = __builtin_amdgcn_raw_buffer_load_b16(rs, e < rem ? tbase + 2u * e : kOutOfRange, 0, 0);
    }

    // Window p: the 16 bytes at 16p past the row's dword boundary, elements
    // 8p - h + c (c < 8); x[8p .. 8p + 7], and x[8p - 1], which the shift
    // brings in (from the lane below, or for a wave's first lane through the
    // scalar cache: a vector load of it for every lane measured 1.2 us per
    // C5-sized launch).
    uint32_t coff[KV];
    uint32_t mask[KV][4];
    u32x4 xa[KV], xb[KV];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int p = (j * NW + wave) * 64 + lane;
        const int lo = 8 * p - h;  // element of the window's first half-word
        coff[j] = lo < kmh ? (uint32_t)p * 16u : kOutOfRange;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int e0 = lo + 2 * d, e1 = e0 + 1;
            mask[j][d] = (e0 >= 0 && e0 < kmh ? 0x0000ffffu : 0u) | (e1 >= 0 && e1 < kmh ? 0xffff0000u : 0u);
        }
        xa[j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (uint32_t)p * 32u, 0, 0);
        xb[j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (uint32_t)p * 32u + 16u, 0, 0);
    }
    const float init = 8 * (wave * 64 + lane) - h < kmh ? 0.0f : -0.0f;

    __shared__ float red[NW + 1][kMaxRpw];  // row NW: the short tail's partials
    u32x4 ba[ROWS][KV], bb[ROWS][KV];
    // Row i's dword boundary: aoff0 + i * rstride bytes.
    const uint32_t aoff0 = row_off(0) - 2u * (uint32_t)h;
    const uint32_t rstride = (uint32_t)(rstep * ldw * 2);
    auto load = [&](u32x4 (&wv)[ROWS][KV], int i0) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            const uint32_t o = aoff0 + (uint32_t)(i0 + q) * rstride;
#pragma unroll
            for (int j = 0; j < KV; ++j) wv[q][j] = load_w16(rs, coff[j], o);
        }
    };
    load(ba, 0);
    float xr[KV][8];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int p0 = (j * NW + wave) * 64;  // the wave's first window
        // x[8 p0 - 1] only where it exists: a wave whose windows all lie
        // past K (K = 2450 on 8 waves) must not read beyond x (a plain load,
        // no range check), and its masked windows need a finite x.
        const float xfirst = p0 > 0 && 8 * p0 - 1 < K ? X[8 * p0 - 1] : 0.0f;
        const float x0[8] = {__uint_as_float(xa[j][0]), __uint_as_float(xa[j][1]), __uint_as_float(xa[j][2]),
                             __uint_as_float(xa[j][3]), __uint_as_float(xb[j][0]), __uint_as_float(xb[j][1]),
                             __uint_as_float(xb[j][2]), __uint_as_float(xb[j][3])};
        const float below = __shfl_up(x0[7], 1, 64);  // x[8p - 1] for every lane but the first
        xr[j][0] = h ? (lane == 0 ? xfirst : below) : x0[0];
#pragma unroll
        for (int c = 1; c < 8; ++c) xr[j][c] = h ? x0[c - 1] : x0[c];
    }
    // hm: the window mask limited to the halves whose x is nonzero
    // (nonzero_pair); each lane's partial is zero-folded before the wave sum.
    uint32_t hm[KV][4];
#pragma unroll
    for (int j = 0; j < KV; ++j)
#pragma unroll
        for (int d = 0; d < 4; ++d) hm[j][d] = mask[j][d] & nonzero_pair(xr[j][2 * d], xr[j][2 * d + 1]);
    if (rem > 0 && wave == NW - 1) {  // the short tail's partial, ascending k from +0, zero-folded
        float t = 0.0f;
        bool hit = false;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float xv = X[kmh + min(e, rem - 1)];
            const uint32_t v = e < rem ? tw[e] : 0x8000u;  // past K: -0 against +0, the exact additive identity
            const float p = e < rem ? xv : 0.0f;
            t = fmaf(p, __uint_as_float(v << 16), t);
            hit |= p != 0.0f && (v & 0x7fffu) != 0;
        }
        if (lane < nr) red[NW][lane] = zero_fold(t, hit);
    }

    // A wave whose windows of the last block all lie past kmh skips that
    // block's arithmetic (a wave-uniform branch around arithmetic only; its
    // loads, out of range, stay unconditional).
    const bool last_block = 8 * (((KV - 1) * NW + wave) * 64) - h < kmh;
    auto sum_rows = [&](const u32x4 (&wv)[ROWS][KV], int i0) {
        float a[ROWS];
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            float acc = init;
            uint32_t nz = 0;
#pragma unroll
            for (int j = 0; j < KV; ++j) {
                if (j == KV - 1 && !last_block) break;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t v = (wv[q][j][d] & mask[j][d]) | (~mask[j][d] & 0x80008000u);
                    acc = fmaf(xr[j][2 * d], widen_lo(v), acc);
                    acc = fmaf(xr[j][2 * d + 1], widen_hi(v), acc);
                    nz |= wv[q][j][d] & hm[j][d];
                }
            }
            a[q] = zero_fold(acc, nz != 0);
        }
        wave_sums(a, [&](int q, float s) {
            if (i0 + q < nr) red[wave][i0 + q] = s;
        });
    };
    for (int i0 = 0; i0 < nr; i0 += 2 * ROWS) {
        load(bb, i0 + ROWS);
        sum_rows(ba, i0);
        if (i0 + ROWS >= nr) break;
        load(ba, i0 + 2 * ROWS);
        sum_rows(bb, i0 + ROWS);
    }
    __syncthreads();
    for (int t0 = wave * 64; t0 < nr; t0 += 64 * NW) {  // as gemv_rd_stream_kernel's
        const int t = t0 + lane;
        const bool live = t < nr;
        const int i = live ? t : 0;
        float s = red[0][i];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w][i];
        if (rem > 0) s += red[NW][i];
        const int64_t row = rb + (int64_t)rstep * i;
        s = zero_unfold(s, live, X, W + row * ldw, 1, K);
        if (live) Y[row] = s;
    }
}

// ---- RD skinny M on MFMA: W [N,K] x X [M,K], K % 64 == 0 ---------------------------
//
// From M = 2 the FMA path loses to the matrix cores (M fmas per weight element,
// MT activation rows of registers; on the LM-head shape M = 2 takes 174-183 us
// there against 161-166 here, M = 3 212-240 against 166-173), so the
// products go to v_mfma_f32_16x16x32_bf16: A = a 16-row weight tile, B = x^T
// for 16 activation rows.  x is f32, so it enters as three bf16 terms,
// x == hi + mid + lo, each taken by truncation: every residual is exact in
// f32 and keeps at most 8 significant bits, so the split is exact for
// |x| >= 2^-110 (below that the error is < 2^-133 absolute).  Measured on
// gfx950 this MFMA multiplies exactly, sums a block's 32 products and the
// accumulator with one rounding, keeps bf16/f32 subnormals, and follows IEEE
// for inf and NaN -- so each output is the exact dot product up to 3
// roundings per 32 k, more accurate than the reference's sequential fma chain.
//
// Special values keep the reference's classes (fmaf(x, w, acc) semantics):
//   x = +-inf or NaN: hi carries it (a NaN is kept quiet), mid = lo = 0;
//   x != 0 tiny: hi is never 0, so inf * x stays inf;
//   w = +-inf or NaN: multiplies hi only -- the mid and lo MFMAs see 0 there,
//     because inf * (mid == 0) would be NaN where the reference has inf.
//
// Zeros: the MFMA rounds a nonzero sum smaller than half the least f32
// subnormal to +0 whatever its sign, where the reference's fmaf gives the
// signed zero (every product underflowing negative ends at -0).  So an output
// that comes out exactly zero is settled by the reference's own rule: +0 when
// its activation row or its weight row holds only zeros (every product is an
// exact zero and the chain never leaves +0), otherwise the chain itself,
// fmaf over ascending k from +0 (rare: underflow or exact cancellation).

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma_bf16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
}

// Bits 0xffff in each 16-bit half of d whose bf16 exponent is all ones.
__device__ __forceinline__ uint32_t inf_nan_mask(uint32_t d) {
    const uint32_t t = ((d & 0x7f807f80u) + 0x00800080u) & 0x80008000u;
    return (t >> 15) * 0xffffu;
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Running per-half maximum of bf16 magnitudes: a half holding an inf or NaN
// reaches 0x7f80.  Two instructions per dword (and, packed max); the exact
// per-element mask is computed only when a wave's screen fires.
__device__ __forceinline__ uint32_t max_mag(uint32_t acc, uint32_t d) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, acc),
                                                                  __builtin_bit_cast(u16x2, d & 0x7fff7fffu)));
}

__device__ __forceinline__ bool wave_has_inf_nan(uint32_t mx) {
    const bool mine = (mx & 0xffffu) >= 0x7f80u || (mx >> 16) >= 0x7f80u;
    return __builtin_amdgcn_ballot_w64(mine) != 0;
}

// The three bf16 terms of one f32.
__device__ __forceinline__ void split3(float v, uint32_t &h, uint32_t &m, uint32_t &l) {
    // Selects, not branches: every lane of the rows16 layout splits 16 values per line.
    const uint32_t u = __float_as_uint(v);
    const bool fin = (u & 0x7f800000u) != 0x7f800000u;
    const uint32_t t = u >> 16;
    const uint32_t nan_q = !fin && (u & 0x007fffffu) ? 0x0040u : 0u;                 // NaN: stay NaN after truncation
    const uint32_t keep = fin && (t & 0x7fffu) == 0 && (u & 0x7fffffffu) != 0 ? 1u : 0u;  // |x| < 2^-133: hi nonzero
    h = t | nan_q | keep;
    const float r1 = fin ? v - __uint_as_float(h << 16) : 0.0f;
    m = __float_as_uint(r1) >> 16;
    const float r2 = r1 - __uint_as_float(m << 16);
    l = __float_as_uint(r2) >> 16;
}

// Four values at once, two per dword of each plane.  Where all four are
// finite with |x| = 0 or |x| >= 2^-133 (bf16's least subnormal), split3's
// rule is truncation alone (no NaN quieting, no kept tiny bit, no inf
// residual), taken here without its selects: 4 operations a value and the
// packing instead of about 15.  The test is two reductions over the
// magnitudes (|x| - 1 wraps 0 to the top); a lane that fails it (an inf, a
// NaN or a tiny value among its four) takes split3.
__device__ __forceinline__ void split4(const float *v, uint32_t *hi, uint32_t *mid, uint32_t *lo) {
    uint32_t amax = 0, amin1 = 0xffffffffu;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t a = __float_as_uint(v[e]) & 0x7fffffffu;
        amax = max(amax, a);
        amin1 = min(amin1, a - 1u);
    }
    if (amax < 0x7f800000u && amin1 >= 0x0000ffffu) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t u0 = __float_as_uint(v[2 * q]), u1 = __float_as_uint(v[2 * q + 1]);
            const float r10 = v[2 * q] - __uint_as_float(u0 & 0xffff0000u);
            const float r11 = v[2 * q + 1] - __uint_as_float(u1 & 0xffff0000u);
            const uint32_t b10 = __float_as_uint(r10), b11 = __float_as_uint(r11);
            const uint32_t b20 = __float_as_uint(r10 - __uint_as_float(b10 & 0xffff0000u));
            const uint32_t b21 = __float_as_uint(r11 - __uint_as_float(b11 & 0xffff0000u));
            hi[q] = (u0 >> 16) | (u1 & 0xffff0000u);
            mid[q] = (b10 >> 16) | (b11 & 0xffff0000u);
            lo[q] = (b20 >> 16) | (b21 & 0xffff0000u);
        }
        return;
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        uint32_t h0, m0, l0, h1, m1, l1;
        split3(v[2 * q], h0, m0, l0);
        split3(v[2 * q + 1], h1, m1, l1);
        hi[q] = h0 | (h1 << 16);
        mid[q] = m0 | (m1 << 16);
        lo[q] = l0 | (l1 << 16);
    }
}

// Eight values: two halves of four.
__device__ __forceinline__ void split8(const float *v, u32x4 &hi, u32x4 &mid, u32x4 &lo) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t hq[2], mq[2], lq[2];
        split4(v + 4 * h, hq, mq, lq);
        hi[2 * h] = hq[0], hi[2 * h + 1] = hq[1];
        mid[2 * h] = mq[0], mid[2 * h + 1] = mq[1];
        lo[2 * h] = lq[0], lo[2 * h + 1] = lq[1];
    }
}

// The reference chain for one output: fmaf over ascending k from +0 (K a
// multiple of 8, rows 16-byte aligned).
__device__ float reference_chain(const uint16_t *__restrict__ w, const float *__restrict__ x, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; k += 8) {
        const u32x4 wv = *reinterpret_cast<const u32x4 *>(w + k);
        const float4 xa = *reinterpret_cast<const float4 *>(x + k);
        const float4 xb = *reinterpret_cast<const float4 *>(x + k + 4);
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t bits = e & 1 ? wv[e >> 1] & 0xffff0000u : wv[e >> 1] << 16;
            acc = fmaf(xv[e], __uint_as_float(bits), acc);
        }
    }
    return acc;
}

// Tiny activation rows.  split3 is exact for |x| >= 2^-110: below that the
// third term falls under bf16's least subnormal (2^-133) and x loses its low
// bits.  That matters only when a whole activation row is that small -- then
// every product loses up to 2^-133 / |x| of itself (a row of |x| ~ 1e-37
// would be off by ~2^-10) -- while in a row with larger entries the lost
// bits are below 2^-33 of the largest one.  So each MFMA kernel keeps, per
// lane, the largest bf16 magnitude of the hi terms it split (hi keeps the
// order of |x| against 2^-100, and is nonzero for every nonzero x), takes
// the maximum per activation row over its workgroup's k range, and gives a
// row whose maximum is nonzero but below 2^-100 (bf16 0x0d80) the reference
// chain over that k range instead of its MFMA sums: bit for bit the
// reference's value when k is not split, else the slice's part of it.  Rare
// path: no real activation row is this small.
constexpr uint32_t kTinyHiBits = 0x0d80u;

__device__ __forceinline__ uint32_t hi_max(uint32_t mx) { return max(mx & 0xffffu, mx >> 16); }
__device__ __forceinline__ bool tiny_row(uint32_t mx) { return mx != 0 && mx < kTinyHiBits; }

// Wave-uniform: does the row hold an element other than +-0?  (bytes: 16 * n16)
__device__ bool wave_row_nonzero(const void *row, int n16, uint32_t mask) {
    const u32x4 *p = reinterpret_cast<const u32x4 *>(row);
    uint32_t acc = 0;
    for (int c = threadIdx.x & 63; c < n16; c += 64) {
        const u32x4 v = p[c];
        acc |= (v[0] | v[1] | v[2] | v[3]) & mask;
    }
    return __builtin_amdgcn_ballot_w64(acc != 0) != 0;
}

// One wave's outputs after the zero rule above.  Lane l holds s[t][r] for
// weight row base[t] + 4(l/16) + r of W and activation row m of X; `live`
// marks the ones it stores.  All 64 lanes call this; the rows are walked
// wave-uniformly.  Rare path: entered only when some output is exactly zero.
template <int T>
__device__ void settle_zeros(f32x4 (&s)[T], const bool (&live)[T][4], const int (&base)[T], const uint16_t *W,
                             const float *X, int K, int m) {
    const int g = (threadIdx.x & 63) >> 4;
    bool zero[T][4];
    bool any = false;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            zero[t][r] = live[t][r] && s[t][r] == 0.0f;
            any |= zero[t][r];
        }
    if (__builtin_amdgcn_ballot_w64(any) == 0) return;
    // Is this lane's activation row nonzero?  Lanes j = 0..15 hold every row
    // the wave has.
    bool xnz = false;
    for (int j = 0; j < 16; ++j) {
        const int mj = __builtin_amdgcn_readlane(m, j);
        if (__builtin_amdgcn_ballot_w64(any && m == mj) != 0) {
            const bool nz = wave_row_nonzero(X + (int64_t)mj * K, K / 4, 0x7fffffffu);
            if (m == mj) xnz = nz;
        }
    }
    // Zero outputs become +0, or the chain's value where both rows are nonzero.
    bool chain[T][4];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            chain[t][r] = false;
            if (zero[t][r]) s[t][r] = 0.0f;
            for (int gq = 0; gq < 4; ++gq) {
                const bool ask = zero[t][r] && xnz && g == gq;
                if (__builtin_amdgcn_ballot_w64(ask) == 0) continue;
                const int row = base[t] + 4 * gq + r;
                const bool nz = wave_row_nonzero(W + (int64_t)row * K, K / 8, 0x7fff7fffu);
                if (ask) chain[t][r] = nz;
            }
        }
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (chain[t][r]) s[t][r] = reference_chain(W + (int64_t)(base[t] + 4 * g + r) * K, X + (int64_t)m * K, K);
}

// Fourth MFMA layout ("wide"): what bounds the MFMA kernels on MI355X is the
// bytes every vector load moves into the CU -- activation re-reads cost as
// much as weight bytes, even from L2 -- and the MFMA operand pattern (16 rows
// x 64 bytes per load) moves them ~15% slower than whole cache lines.  So:
// 256 weight rows per workgroup (8 waves x 2 tiles, each wave owning its
// tiles: no cross-wave reduction), k in chunks of 64 so each row's chunk is
// one 128-byte line, weights loaded 8 whole lines per instruction into a
// swizzled LDS tile (writes and operand reads conflict-free), x's chunk (16 x 64)
// split once per workgroup into LDS planes.  x bytes are 1/8 of weight bytes.
// Each wave stages and consumes only its own 32 rows, so its tile needs only
// the wave's own program order (LDS executes a wave's operations in order);
// the shared x planes are double-buffered behind one barrier per chunk.
// Loads run two chunks ahead in registers.
constexpr int kWideRows = 256;
constexpr int kWidePitch = 128;

// Weight and x tiles in LDS hold rows of 128 bytes, 8 pieces of 16, back to
// back, with piece p of row r stored at position p ^ ((r / 2) mod 8).  A
// tile is written 8 rows x 128 bytes per instruction (each pair of rows then
// covers the 64 banks once) and read 16 rows x one piece (the rows' pieces
// land on 16 different groups of 4 banks).  The earlier 144-byte pitch kept
// the reads apart but let each pair of rows written together meet on 4 banks
// (11-24% of the MFMA kernels' LDS cycles lost to conflicts).
__device__ __forceinline__ int swz(int r, int p) { return r * 128 + ((p ^ ((r >> 1) & 7)) << 4); }

// Chunk order of the MFMA layouts.  A workgroup streams its weight rows
// one 128-byte column of lines (64 k) at a time; with every workgroup at
// the same k the whole device reads addresses that differ only above the
// row pitch, which for power-of-two rows (K = 4096: 8 KiB) meets a few HBM
// channels at a time.  Workgroup b therefore starts at chunk 5b mod n and
// wraps: on C4's W [128256, 4096] the read pattern alone streams in 150 us
// rotated against 178 in step (a plain read of the same bytes: 145).  The
// MFMA sums are taken in that order; the zero rule and the tiny-row chains
// recompute in k order, so only rounding inside the bound changes.
__device__ __forceinline__ int chunk_rotation(uint32_t b, int n) {
    return n > 0 ? (int)((b * 5u) % (uint32_t)n) : 0;
}
__device__ __forceinline__ int rotate_chunk(int c, int s0, int n) { return c + s0 >= n ? c + s0 - n : c + s0; }

__global__ void __launch_bounds__(512)
gemv_rd_mfma_wide_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                         int K, int M) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int row0 = blockIdx.x * kWideRows;
    const int nrows = min(kWideRows, N - row0);
    const int m0 = blockIdx.y * 16;
    const int nchunks = K / 64;

    __shared__ __attribute__((aligned(16))) uint8_t wt[kWideRows * kWidePitch];  // 32 KiB
    __shared__ u32x4 xpl[2][2][3][64];                                           // 2 x 6 KiB
    __shared__ uint32_t xmax_s[16];  // per activation row: the largest hi-term magnitude (tiny rows)
    uint8_t *const wtw = wt + wave * 32 * kWidePitch;                            // this wave's 32 rows
    if (tid < 16) xmax_s[tid] = 0;

    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(W + (int64_t)row0 * K, (uint32_t)((int64_t)nrows * K * 2));
    // Staging: load j (0..3) covers the wave's rows 8j + lane/8, bytes 16*(lane%8) of the chunk.
    const int scol = (lane & 7) * 16;
    const int slr = lane >> 3;
    uint32_t soff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        soff[j] = (uint32_t)min(wave * 32 + slr + 8 * j, nrows - 1) * (uint32_t)K * 2u + scol;
    // x items: threads 0..127 = (k-block b = tid/64, operand lane = tid%64).
    const bool xthread = tid < 128;
    const int xm = m0 + (lane & 15);
    const float *xp = X + (int64_t)min(xm, M - 1) * K + (tid >> 6) * 32 + (lane >> 4) * 8;
    const bool xlive = xthread && xm < M;

    struct Regs {
        u32x4 w[4];
        float x[8];
    };
    const int s0 = chunk_rotation(blockIdx.x, nchunks);
    auto load = [&](int c, Regs &r) {
        c = rotate_chunk(c, s0, nchunks);
#pragma unroll
        for (int j = 0; j < 4; ++j) r.w[j] = load_w16(rs, soff[j] + (uint32_t)c * 128u);
        if (xlive) {
            const float4 a = *reinterpret_cast<const float4 *>(xp + c * 64);
            const float4 b = *reinterpret_cast<const float4 *>(xp + c * 64 + 4);
            r.x[0] = a.x; r.x[1] = a.y; r.x[2] = a.z; r.x[3] = a.w;
            r.x[4] = b.x; r.x[5] = b.y; r.x[6] = b.z; r.x[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) r.x[e] = 0.0f;
        }
    };
    uint32_t xmx = 0;
    auto store = [&](const Regs &r, int xbuf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4 *>(wtw + swz(slr + 8 * j, lane & 7)) = r.w[j];
        if (xthread) {
            u32x4 hi, md, lo;
            split8(r.x, hi, md, lo);
#pragma unroll
            for (int v = 0; v < 4; ++v) xmx = max_mag(xmx, hi[v]);
            xpl[xbuf][tid >> 6][0][lane] = hi;
            xpl[xbuf][tid >> 6][1][lane] = md;
            xpl[xbuf][tid >> 6][2][lane] = lo;
        }
    };

    f32x4 acc[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
    auto compute = [&](int xbuf) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const u32x4 hi = xpl[xbuf][b][0][lane], md = xpl[xbuf][b][1][lane], lo = xpl[xbuf][b][2][lane];
            u32x4 a[2];
            uint32_t mx = 0;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                a[t] = *reinterpret_cast<const u32x4 *>(wtw + swz(t * 16 + i16, b * 4 + g));
#pragma unroll
                for (int v = 0; v < 4; ++v) mx = max_mag(mx, a[t][v]);
            }
            const bool any_special = wave_has_inf_nan(mx);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                acc[t] = mfma_bf16(a[t], hi, acc[t]);
                u32x4 a2 = a[t];
                if (any_special) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) a2[v] &= ~inf_nan_mask(a2[v]);
                }
                acc[t] = mfma_bf16(a2, md, acc[t]);
                acc[t] = mfma_bf16(a2, lo, acc[t]);
            }
        }
    };

    // Chunk c is in LDS (x planes in buffer c&1); chunk c+1 waits in one
    // register set and chunk c+2 loads into the other.
    Regs ra, rb;
    if (nchunks > 0) load(0, ra);
    if (nchunks > 1) load(1, rb);
    if (nchunks > 0) store(ra, 0);
    __syncthreads();
    auto step = [&](int c, Regs &rnext, Regs &rfree) {
        if (c + 2 < nchunks) load(c + 2, rfree);
        compute(c & 1);
        if (c + 1 < nchunks) store(rnext, (c + 1) & 1);
        __syncthreads();
    };
    for (int c = 0; c < nchunks; c += 2) {
        step(c, rb, ra);
        if (c + 1 >= nchunks) break;
        step(c + 1, ra, rb);
    }

    if (xthread) atomicMax(&xmax_s[lane & 15], hi_max(xmx));
    __syncthreads();
    const int base[2] = {wave * 32, wave * 32 + 16};
    bool live[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) live[t][r] = m0 + i16 < M && base[t] + g * 4 + r < nrows;
    const bool tiny = m0 + i16 < M && tiny_row(xmax_s[i16]);
    if (__builtin_amdgcn_ballot_w64(tiny) != 0) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (tiny && live[t][r])
                    acc[t][r] = reference_chain(W + (int64_t)(row0 + base[t] + g * 4 + r) * K,
                                                X + (int64_t)(m0 + i16) * K, K);
    }
    settle_zeros(acc, live, base, W + (int64_t)row0 * K, X + (int64_t)m0 * K, K, i16);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (live[t][r]) Y[(int64_t)(m0 + i16) * N + row0 + base[t] + g * 4 + r] = acc[t][r];
}

// Sixth MFMA layout ("gemm"), for 9 activation rows and up (prefill-sized M
// among them): the wide layout with MB tiles of 16 activation rows per
// workgroup instead of one.  Every
// weight tile a wave stages in LDS meets all 16 * MB activation rows, so W
// streams from HBM once per 16 * MB rows (the 16-row layouts stream it once
// per 16).  x arrives already split: split_x_planes_kernel writes its three
// bf16 terms once per call as planes [3][M][K], and each chunk's operands are
// copied into LDS (no per-workgroup split).  FUSE (16-row activation tiles):
// each workgroup loads its chunks of x as f32 and splits them itself on the
// way into LDS instead, which saves the split launch; at 16 activation rows
// the repeated split is a few dozen values per thread.  When 256-row by 16*MB-row tiles
// would leave the device short of workgroups, k is split over `slices`
// workgroups, each covering kc chunks of 64, whose partial sums go to
// P[slice][m][n] for gemm_sum_slices_kernel.  Numerics, special values and
// the zero rule are the wide layout's, tile by tile; with slices the zero
// rule runs after the sum.
template <int MB, bool FUSE, int NWV>
__global__ void __launch_bounds__(64 * NWV)
gemv_rd_mfma_gemm_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, const uint16_t *__restrict__ XS,
                         float *__restrict__ Y, float *__restrict__ P, int N, int K, int M, int kc, int gx, int gy,
                         int xcd) {
    static_assert(MB >= 1 && MB <= 4, "16 to 64 activation rows per workgroup");
    static_assert(NWV == 4 || NWV == 8, "32 weight rows per wave");
    constexpr int kRows = 32 * NWV;                  // weight rows per workgroup
    constexpr int kXItems = 128 * MB;                // x staging items (tile, k-block, operand lane)
    constexpr int kXPer = (kXItems + 64 * NWV - 1) / (64 * NWV);  // items per thread
    constexpr int D = 2;  // register sets of the chunk ring (3 and 4 measured no faster)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i16 = lane & 15;
    const int g = lane >> 4;
    // The tile from the linear workgroup id (a 1-D grid of gx * gy * slices).
    // With `xcd` set, workgroup L, which runs on XCD L % 8 (the dispatcher
    // deals workgroups to the 8 XCDs in turn), takes the L / 8-th tile of
    // that XCD's contiguous share, activation tiles fastest, so the
    // workgroups an XCD runs together share weight blocks through its L2
    // (C2 shapes at several activation tiles: 2-3% faster than weight blocks
    // fastest); otherwise tiles go in launch order, consecutive weight
    // blocks to different XCDs.
    uint32_t lin = blockIdx.x;
    if (xcd) {
        const uint32_t x = lin & 7u, q = gridDim.x >> 3, r = gridDim.x & 7u;
        lin = x * q + min(x, r) + (lin >> 3);
    }
    const int by = (int)(lin % (uint32_t)gy);
    const int bx = (int)(lin / (uint32_t)gy % (uint32_t)gx);
    const int bz = (int)(lin / (uint32_t)gy / (uint32_t)gx);
    const int row0 = bx * kRows;
    const int nrows = min(kRows, N - row0);
    const int m0 = by * 16 * MB;
    const int c0 = bz * kc;                              // this slice's chunks: [c0, c1)
    const int c1 = min(K / 64, c0 + kc);
    const int nchunks = max(0, c1 - c0);

    __shared__ __attribute__((aligned(16))) uint8_t wt[kRows * kWidePitch];  // 32 KiB at 8 waves
    __shared__ u32x4 xpl[2][MB][2][3][64];                                   // MB x 12 KiB
    __shared__ uint32_t xmax_s[16 * MB];  // per activation row: the largest hi-term magnitude (tiny rows)
    uint8_t *const wtw = wt + wave * 32 * kWidePitch;                            // this wave's 32 rows
    if (tid < 16 * MB) xmax_s[tid] = 0;

    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(W + (int64_t)row0 * K, (uint32_t)((int64_t)nrows * K * 2));
    // Staging: load j (0..3) covers the wave's rows 8j + lane/8, bytes 16*(lane%8) of the chunk.
    const int scol = (lane & 7) * 16;
    const int slr = lane >> 3;
    uint32_t soff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        soff[j] = (uint32_t)min(wave * 32 + slr + 8 * j, nrows - 1) * (uint32_t)K * 2u + scol;
    // x items it = tid + 64*NWV*j (j < kXPer), those below 128*MB: (tile xt =
    // it/128, k-block b = it/64 % 2, operand lane = lane): the lane's 8
    // elements of each of the three planes (FUSE: its 8 f32 values, split in
    // `store`), by unconditional buffer loads (rows past M load from past the
    // range: zeros).
    bool xthread[kXPer];
    int xt[kXPer], xb[kXPer];
    uint32_t xoff[kXPer];
    const uint32_t plane_bytes = (uint32_t)M * (uint32_t)K * 2u;
    const __amdgpu_buffer_rsrc_t xrs = FUSE ? weight_rsrc(X, 2u * plane_bytes) : weight_rsrc(XS, 3u * plane_bytes);
#pragma unroll
    for (int j = 0; j < kXPer; ++j) {
        const int it = tid + 64 * NWV * j;
        xthread[j] = it < kXItems;
        xt[j] = xthread[j] ? it >> 7 : 0;
        xb[j] = (it >> 6) & 1;
        const int xm = m0 + xt[j] * 16 + (lane & 15);
        const uint32_t xelem = (uint32_t)xm * (uint32_t)K + xb[j] * 32 + (lane >> 4) * 8;
        xoff[j] = xthread[j] && xm < M ? xelem * (FUSE ? 4u : 2u) : kOutOfRange;
    }

    constexpr int XQ = FUSE ? 2 : 3;  // x registers per item and chunk: f32 halves, or the three planes
    struct Regs {
        u32x4 w[4];
        u32x4 x[kXPer][XQ];
    };
    const int s0 = chunk_rotation(bx, nchunks);
    auto load = [&](int c, Regs &r) {
        const uint32_t cb = (uint32_t)(c0 + rotate_chunk(c, s0, nchunks)) * 128u;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.w[j] = load_w16(rs, soff[j] + cb);
#pragma unroll
        for (int j = 0; j < kXPer; ++j) {
            if constexpr (FUSE) {
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    r.x[j][q] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[j], 2u * cb + 16u * q, 0);
            } else {
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    r.x[j][q] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[j], q * plane_bytes + cb, 0);
            }
        }
    };
    uint32_t xmx[kXPer];
#pragma unroll
    for (int j = 0; j < kXPer; ++j) xmx[j] = 0;
    auto store = [&](const Regs &r, int xbuf) {
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4 *>(wtw + swz(slr + 8 * j, lane & 7)) = r.w[j];
#pragma unroll
        for (int j = 0; j < kXPer; ++j) {
            if (!xthread[j]) continue;
            if constexpr (FUSE) {
                const float v[8] = {__uint_as_float(r.x[j][0][0]), __uint_as_float(r.x[j][0][1]),
                                    __uint_as_float(r.x[j][0][2]), __uint_as_float(r.x[j][0][3]),
                                    __uint_as_float(r.x[j][1][0]), __uint_as_float(r.x[j][1][1]),
                                    __uint_as_float(r.x[j][1][2]), __uint_as_float(r.x[j][1][3])};
                u32x4 hi, md, lo;
                split8(v, hi, md, lo);
#pragma unroll
                for (int e = 0; e < 4; ++e) xmx[j] = max_mag(xmx[j], hi[e]);
                xpl[xbuf][xt[j]][xb[j]][0][lane] = hi;
                xpl[xbuf][xt[j]][xb[j]][1][lane] = md;
                xpl[xbuf][xt[j]][xb[j]][2][lane] = lo;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) xmx[j] = max_mag(xmx[j], r.x[j][0][e]);
#pragma unroll
                for (int q = 0; q < 3; ++q) xpl[xbuf][xt[j]][xb[j]][q][lane] = r.x[j][q];
            }
        }
    };

    f32x4 acc[MB][2];
#pragma unroll
    for (int mt = 0; mt < MB; ++mt) acc[mt][0] = acc[mt][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // One k-block of 32: the hi term with the raw weights, md and lo with
    // inf/NaN lanes cleared when the wave's block holds any.
    auto block = [&](const u32x4 (&a)[2], const u32x4 (&xo)[MB][3]) {
        u32x4 a2[2];
        uint32_t mx = 0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) mx = max_mag(mx, a[t][v]);
        const bool any_special = wave_has_inf_nan(mx);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            a2[t] = a[t];
            if (any_special) {
#pragma unroll
                for (int v = 0; v < 4; ++v) a2[t][v] &= ~inf_nan_mask(a2[t][v]);
            }
        }
#pragma unroll
        for (int mt = 0; mt < MB; ++mt)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                acc[mt][t] = mfma_bf16(a[t], xo[mt][0], acc[mt][t]);
                acc[mt][t] = mfma_bf16(a2[t], xo[mt][1], acc[mt][t]);
                acc[mt][t] = mfma_bf16(a2[t], xo[mt][2], acc[mt][t]);
            }
    };
    auto read_ops = [&](int xbuf, int b, u32x4 (&a)[2], u32x4 (&xo)[MB][3]) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
            a[t] = *reinterpret_cast<const u32x4 *>(wtw + swz(t * 16 + i16, b * 4 + g));
#pragma unroll
        for (int mt = 0; mt < MB; ++mt)
#pragma unroll
            for (int q = 0; q < 3; ++q) xo[mt][q] = xpl[xbuf][mt][b][q][lane];
    };
    // With 64-row tiles both k-blocks' operands are read from LDS up front,
    // so the second block's reads are in flight during the first block's
    // MFMAs (C2 up / down at m = 512: 233 / 239 us against 245 / 241).  With
    // fewer tiles the extra registers would cost a workgroup per CU (m = 64:
    // 67 / 68 us against 61 / 63), so each block's operands are read just
    // before it.
    auto compute = [&](int xbuf) {
        if constexpr (MB == 4) {
            u32x4 a[2][2], xo[2][MB][3];
            read_ops(xbuf, 0, a[0], xo[0]);
            read_ops(xbuf, 1, a[1], xo[1]);
            block(a[0], xo[0]);
            block(a[1], xo[1]);
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                u32x4 a[2], a2[2];
                uint32_t mx = 0;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    a[t] = *reinterpret_cast<const u32x4 *>(wtw + swz(t * 16 + i16, b * 4 + g));
#pragma unroll
                    for (int v = 0; v < 4; ++v) mx = max_mag(mx, a[t][v]);
                }
                const bool any_special = wave_has_inf_nan(mx);
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    a2[t] = a[t];
                    if (any_special) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) a2[t][v] &= ~inf_nan_mask(a2[t][v]);
                    }
                }
#pragma unroll
                for (int mt = 0; mt < MB; ++mt) {
                    const u32x4 hi = xpl[xbuf][mt][b][0][lane], md = xpl[xbuf][mt][b][1][lane],
                                lo = xpl[xbuf][mt][b][2][lane];
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        acc[mt][t] = mfma_bf16(a[t], hi, acc[mt][t]);
                        acc[mt][t] = mfma_bf16(a2[t], md, acc[mt][t]);
                        acc[mt][t] = mfma_bf16(a2[t], lo, acc[mt][t]);
                    }
                }
            }
        }
    };

    // A ring of D register sets: at step c chunk c is in LDS (x planes in
    // buffer c&1), chunks c+1 .. c+D-1 are in flight to their sets, and the
    // set chunk c arrived in (already in LDS) takes chunk c+D.
    Regs r[D];
#pragma unroll
    for (int u = 0; u < D; ++u)
        if (u < nchunks) load(u, r[u]);
    if (nchunks > 0) store(r[0], 0);
    __syncthreads();
    for (int cb = 0; cb < nchunks; cb += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int c = cb + u;
            if (c >= nchunks) break;
            if (c + D < nchunks) load(c + D, r[u]);
            compute(c & 1);
            if (c + 1 < nchunks) store(r[(u + 1) % D], (c + 1) & 1);
            __syncthreads();
        }
    }

#pragma unroll
    for (int j = 0; j < kXPer; ++j)
        if (xthread[j]) atomicMax(&xmax_s[xt[j] * 16 + (lane & 15)], hi_max(xmx[j]));
    __syncthreads();
    const int base[2] = {wave * 32, wave * 32 + 16};
#pragma unroll
    for (int mt = 0; mt < MB; ++mt) {
        const int m = m0 + mt * 16 + i16;
        bool live[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) live[t][rr] = m < M && base[t] + g * 4 + rr < nrows;
        const bool tiny = m < M && tiny_row(xmax_s[mt * 16 + i16]);
        if (__builtin_amdgcn_ballot_w64(tiny) != 0) {  // this slice's chain (all of k without slices)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (tiny && live[t][rr])
                        acc[mt][t][rr] = reference_chain(W + (int64_t)(row0 + base[t] + g * 4 + rr) * K + 64 * c0,
                                                         X + (int64_t)m * K + 64 * c0, 64 * nchunks);
        }
        if (P) {  // a k slice: the partial sums, for gemm_sum_slices_kernel
            float *ps = P + (int64_t)bz * M * N + (int64_t)m * N + row0;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (live[t][rr]) ps[base[t] + g * 4 + rr] = acc[mt][t][rr];
            continue;
        }
        settle_zeros(acc[mt], live, base, W + (int64_t)row0 * K, X + (int64_t)(m0 + mt * 16) * K, K, i16);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                if (live[t][rr]) Y[(int64_t)m * N + row0 + base[t] + g * 4 + rr] = acc[mt][t][rr];
    }
}

// x [M,K] f32 -> its three bf16 terms as planes XS[q][M][K] (split3 of each
// element), for the gemm layout.  count = M*K, a multiple of 8; 16-byte
// aligned.  Grid-stride.
__global__ void __launch_bounds__(256)
split_x_planes_kernel(const float *__restrict__ X, uint16_t *__restrict__ XS, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count / 8; i += (int64_t)gridDim.x * 256) {
        const float4 a = reinterpret_cast<const float4 *>(X)[2 * i];
        const float4 b = reinterpret_cast<const float4 *>(X)[2 * i + 1];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        u32x4 hi, md, lo;
        split8(v, hi, md, lo);
        reinterpret_cast<u32x4 *>(XS)[i] = hi;
        reinterpret_cast<u32x4 *>(XS + count)[i] = md;
        reinterpret_cast<u32x4 *>(XS + 2 * count)[i] = lo;
    }
}

// y[m][n] = P[0][m][n] + P[1][m][n] + ... in slice order, then the zero rule
// of settle_zeros for one output: an exact zero is +0 when the activation row
// or the weight row holds only +-0, else the reference chain's value.
__global__ void __launch_bounds__(256)
gemm_sum_slices_kernel(const float *__restrict__ P, int slices, float *__restrict__ Y, const uint16_t *__restrict__ W,
                       const float *__restrict__ X, int M, int N, int K) {
    const int64_t count = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
        float s = P[i];
#pragma unroll 8
        for (int j = 1; j < slices; ++j) s += P[j * count + i];
        if (s == 0.0f) {
            const int m = (int)(i / N), n = (int)(i - (int64_t)m * N);
            const uint32_t *xr = reinterpret_cast<const uint32_t *>(X + (int64_t)m * K);
            const uint32_t *wr = reinterpret_cast<const uint32_t *>(W + (int64_t)n * K);
            uint32_t xo = 0, wo = 0;
            for (int k = 0; k < K; ++k) xo |= xr[k] & 0x7fffffffu;
            for (int k = 0; k < K / 2; ++k) wo |= wr[k] & 0x7fff7fffu;
            s = (xo && wo) ? reference_chain(W + (int64_t)n * K, X + (int64_t)m * K, K) : 0.0f;
        }
        Y[i] = s;
    }
}

// Fifth MFMA layout ("rows16"), for a few activation rows: 16 weight rows per
// workgroup, read whole.  The rows advance in windows of 8 lines (1 KiB per
// row); wave w owns line w of every window, 64 k elements = two MFMA k-blocks.
// On MI355X the read pattern decides the rate: 16 rows x 1 KiB per window
// streams ~10% faster than the wide layout's 256 rows x 128 bytes, and a load
// instruction must cover whole lines (8 rows x 128 bytes here) -- one in the
// MFMA operand layout (16 rows x 64 bytes) streams ~15% slower still.  So each
// wave loads its 16 rows x 128 bytes as whole lines and passes them through a
// private LDS tile into the operand layout (one wave's LDS operations run in
// program order: no barrier).
//
// x: splitting f32 into three bf16 terms is the costly vector work here, and
// the B operand has 16 columns however few activation rows there are.  With
// MC = 4 or 8 activation rows per workgroup, lane l loads and splits the
// 64 MC / 64 values x[m0 + l/(64/MC)][64L + MC(l%(64/MC)), +MC) and writes the
// three terms to a private LDS tile; B columns MC..15 read a row of zeros.
// With MC = 16 each lane loads its B operand directly (lanes past M load from
// outside the buffer: zeros, no traffic) and splits 16 values.  The waves' partial sums meet once, at the
// end, in LDS in wave order.  Loads run one line ahead (two register sets);
// lines past the last load from outside the buffers.
constexpr int kRows16Pitch = 128;

template <int MC, int T>
__global__ void __launch_bounds__(512)
gemv_rd_mfma_rows16_kernel(const uint16_t *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y,
                           int N, int K, int M, int lpk, float *__restrict__ P) {
    static_assert(MC == 4 || MC == 8 || MC == 16, "activation rows per workgroup");
    static_assert(T == 1 || T == 2 || T == 4, "16-row blocks per workgroup");
    constexpr bool kCompact = MC < 16;
    constexpr int kLanesPerRow = 64 / MC;  // compact x: lanes per activation row
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i16 = lane & 15;
    const int g = lane >> 4;
    const int m0 = blockIdx.y * MC;
    const int mrows = min(MC, M - m0);
    // k slice blockIdx.z: lines [l0, l1) of 64 elements (lpk per slice; one
    // slice unless P, the slices' partial sums, is given)
    const int l0 = (int)blockIdx.z * lpk;
    const int l1 = min(K >> 6, l0 + lpk);

    // LDS: the waves' weight tiles and x planes while streaming, then the
    // partial sums (T x 8 KiB) in the same bytes.
    constexpr int kXRows = kCompact ? MC + 1 : 1;  // MC x rows and a zero row
    constexpr int kTileBytes = 16 * kRows16Pitch;
    constexpr int kXBytes = kCompact ? 3 * kXRows * kRows16Pitch : 0;
    constexpr int kStreamBytes = 8 * (kTileBytes + kXBytes);
    constexpr int kRedBytes = 8 * T * 64 * 16;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kStreamBytes > kRedBytes ? kStreamBytes : kRedBytes];
    __shared__ uint32_t xmax_s[16];  // per activation row: the largest hi-term magnitude (tiny rows)
    uint8_t *const tile = lds + wave * kTileBytes;
    uint8_t *const xt = lds + 8 * kTileBytes + wave * kXBytes;  // [3][kXRows][pitch]
    f32x4 *const red = reinterpret_cast<f32x4 *>(lds);         // [8][T][64]
    if (threadIdx.x < 16) xmax_s[threadIdx.x] = 0;

    // Block t of this workgroup: weight rows 16 (blockIdx.x + t gridDim.x) + 0..15.
    __amdgpu_buffer_rsrc_t rs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int r0 = min(N, (int)(blockIdx.x + t * gridDim.x) * 16);
        rs[t] = weight_rsrc(W + (int64_t)r0 * K, (uint32_t)((int64_t)min(16, N - r0) * K * 2));
    }
    const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X + (int64_t)m0 * K, (uint32_t)((int64_t)mrows * K * 4));
    // Whole-line staging: load j (0, 1) covers rows 8j + lane/8, bytes 16*(lane%8) of the line; rows
    // past a block's end lie outside its buffer resource and read zeros.
    const int srow = lane >> 3, scol = (lane & 7) * 16;
    const uint32_t woff0 = (uint32_t)srow * (uint32_t)K * 2u + scol;
    const uint32_t woff1 = (uint32_t)(srow + 8) * (uint32_t)K * 2u + scol;
    // x offsets.  MC = 16: lane (j, g) takes x[m0 + j][64L + 32b + 8g, +8) for k-block b.
    // MC = 4, 8: lane l takes x[m0 + l/(64/MC)][64L + MC(l%(64/MC)), +MC).
    const int xm = kCompact ? lane / kLanesPerRow : i16;
    const int xq = lane % kLanesPerRow;
    const uint32_t xoff =
        xm < mrows ? ((uint32_t)xm * (uint32_t)K + (kCompact ? (uint32_t)(MC * xq) : 8u * g)) * 4u : kOutOfRange;
    if (kCompact) {
#pragma unroll
        for (int p = 0; p < 3; ++p)
            if (lane < kRows16Pitch / 16)
                *reinterpret_cast<u32x4 *>(xt + p * kXRows * kRows16Pitch + swz(MC, lane)) = u32x4{0, 0, 0, 0};
    }

    struct Line {
        u32x4 w0[T], w1[T];    // weight rows srow, srow + 8 of each block
        u32x4 x0, x1, x2, x3;  // MC = 16: x for k-block 0 (x0, x1) and 1 (x2, x3); MC = 4: x0; MC = 8: x0, x1
    };
    // Line L's loads; lines past the end read zeros from outside the buffers.
    auto load = [&](Line &r, int L) {
        const bool live = L < l1;
        const uint32_t lw = (uint32_t)L * 128u, lx = (uint32_t)L * 256u;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            r.w0[t] = load_w16(rs[t], live ? woff0 : kOutOfRange, lw);
            r.w1[t] = load_w16(rs[t], live ? woff1 : kOutOfRange, lw);
        }
        const uint32_t xo = live ? xoff : kOutOfRange;
        r.x0 = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, lx, 0);
        if (MC == 8) r.x1 = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 16u, lx, 0);
        if (MC == 16) {
            r.x1 = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 16u, lx, 0);
            r.x2 = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 128u, lx, 0);
            r.x3 = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 144u, lx, 0);
        }
    };

    // A wave that owns no line adds -0, the identity that keeps a -0 sum.
    const float z = l0 + wave < l1 ? 0.0f : -0.0f;
    f32x4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f32x4{z, z, z, z};
    uint32_t xmx = 0;  // the largest hi-term magnitude this lane split (its activation row xm, or i16)
    auto compute = [&](const Line &r) {
        // x: the three bf16 terms in the B operand layout.
        u32x4 h0, md0, lo0, h1, md1, lo1;
        if (MC == 4) {
            uint32_t hq[2], mq[2], lq[2];
            const float xv[4] = {__uint_as_float(r.x0[0]), __uint_as_float(r.x0[1]), __uint_as_float(r.x0[2]),
                                 __uint_as_float(r.x0[3])};
            split4(xv, hq, mq, lq);
#pragma unroll
            for (int q = 0; q < 2; ++q) xmx = max_mag(xmx, hq[q]);
            uint8_t *const xr = xt + swz(xm, xq >> 1) + (xq & 1) * 8;
            *reinterpret_cast<uint2 *>(xr) = uint2{hq[0], hq[1]};
            *reinterpret_cast<uint2 *>(xr + kXRows * kRows16Pitch) = uint2{mq[0], mq[1]};
            *reinterpret_cast<uint2 *>(xr + 2 * kXRows * kRows16Pitch) = uint2{lq[0], lq[1]};
        } else if (MC == 8) {
            float xv[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                xv[e] = __uint_as_float(r.x0[e]);
                xv[4 + e] = __uint_as_float(r.x1[e]);
            }
            u32x4 hq, mq, lq;
            split8(xv, hq, mq, lq);
#pragma unroll
            for (int v = 0; v < 4; ++v) xmx = max_mag(xmx, hq[v]);
            uint8_t *const xr = xt + swz(xm, xq);
            *reinterpret_cast<u32x4 *>(xr) = hq;
            *reinterpret_cast<u32x4 *>(xr + kXRows * kRows16Pitch) = mq;
            *reinterpret_cast<u32x4 *>(xr + 2 * kXRows * kRows16Pitch) = lq;
        }
        if (kCompact) {
            __builtin_amdgcn_wave_barrier();
            const int xrow = i16 < MC ? i16 : MC;
            const uint8_t *const xr0 = xt + swz(xrow, g), *const xr1 = xt + swz(xrow, 4 + g);
            h0 = *reinterpret_cast<const u32x4 *>(xr0);
            md0 = *reinterpret_cast<const u32x4 *>(xr0 + kXRows * kRows16Pitch);
            lo0 = *reinterpret_cast<const u32x4 *>(xr0 + 2 * kXRows * kRows16Pitch);
            h1 = *reinterpret_cast<const u32x4 *>(xr1);
            md1 = *reinterpret_cast<const u32x4 *>(xr1 + kXRows * kRows16Pitch);
            lo1 = *reinterpret_cast<const u32x4 *>(xr1 + 2 * kXRows * kRows16Pitch);
        } else {
            float xv[16];
            const u32x4 xs[4] = {r.x0, r.x1, r.x2, r.x3};
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[4 * q + e] = __uint_as_float(xs[q][e]);
            split8(xv, h0, md0, lo0);
            split8(xv + 8, h1, md1, lo1);
#pragma unroll
            for (int v = 0; v < 4; ++v) xmx = max_mag(max_mag(xmx, h0[v]), h1[v]);
        }
        // Weights: each block through the wave's tile in turn.
#pragma unroll
        for (int t = 0; t < T; ++t) {
            __builtin_amdgcn_wave_barrier();
            *reinterpret_cast<u32x4 *>(tile + swz(srow, lane & 7)) = r.w0[t];
            *reinterpret_cast<u32x4 *>(tile + swz(srow + 8, lane & 7)) = r.w1[t];
            __builtin_amdgcn_wave_barrier();
            const u32x4 a0 = *reinterpret_cast<const u32x4 *>(tile + swz(i16, g));
            const u32x4 a1 = *reinterpret_cast<const u32x4 *>(tile + swz(i16, 4 + g));
            uint32_t mx = 0;
#pragma unroll
            for (int v = 0; v < 4; ++v) mx = max_mag(max_mag(mx, a0[v]), a1[v]);
            const bool any_special = wave_has_inf_nan(mx);
            u32x4 a0m = a0, a1m = a1;
            if (any_special) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    a0m[v] &= ~inf_nan_mask(a0m[v]);
                    a1m[v] &= ~inf_nan_mask(a1m[v]);
                }
            }
            acc[t] = mfma_bf16(a0, h0, acc[t]);
            acc[t] = mfma_bf16(a0m, md0, acc[t]);
            acc[t] = mfma_bf16(a0m, lo0, acc[t]);
            acc[t] = mfma_bf16(a1, h1, acc[t]);
            acc[t] = mfma_bf16(a1m, md1, acc[t]);
            acc[t] = mfma_bf16(a1m, lo1, acc[t]);
        }
        __builtin_amdgcn_wave_barrier();
    };

    Line la, lb;
    load(la, l0 + wave);
    for (int L = l0 + wave; L < l1; L += 16) {
        load(lb, L + 8);
        compute(la);
        if (L + 8 >= l1) break;
        load(la, L + 16);
        compute(lb);
    }

    // acc[t] of lane l holds weight rows 4(l/16) + r of block t, activation row m0 + l%16.
    __syncthreads();  // every wave is done with its tile and x planes
#pragma unroll
    for (int t = 0; t < T; ++t) red[(wave * T + t) * 64 + lane] = acc[t];
    atomicMax(&xmax_s[kCompact ? xm : i16], hi_max(xmx));
    __syncthreads();
    if (wave < T) {
        const int t = wave;
        const int row0 = (int)(blockIdx.x + t * gridDim.x) * 16;
        if (row0 < N) {
            const int nrows = min(16, N - row0);
            f32x4 s[1] = {red[t * 64 + lane]};
#pragma unroll
            for (int w = 1; w < 8; ++w) s[0] += red[(w * T + t) * 64 + lane];
            const int base[1] = {0};
            bool live[1][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) live[0][r] = i16 < mrows && g * 4 + r < nrows;
            const bool tiny = i16 < mrows && tiny_row(xmax_s[i16]);
            if (__builtin_amdgcn_ballot_w64(tiny) != 0) {  // this slice's chain (all of k without slices)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (tiny && live[0][r])
                        s[0][r] = reference_chain(W + (int64_t)(row0 + g * 4 + r) * K + 64 * l0,
                                                  X + (int64_t)(m0 + i16) * K + 64 * l0, 64 * max(0, l1 - l0));
            }
            if (P) {  // a k slice: its partial sums, for gemm_sum_slices_kernel (which settles zeros)
                float *ps = P + (int64_t)blockIdx.z * M * N + (int64_t)(m0 + i16) * N + row0 + g * 4;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (live[0][r]) ps[r] = s[0][r];
            } else {
                settle_zeros(s, live, base, W + (int64_t)row0 * K, X + (int64_t)m0 * K, K, i16);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (live[0][r]) Y[(int64_t)(m0 + i16) * N + row0 + g * 4 + r] = s[0][r];
            }
        }
    }
}

// ---- RD general: W [N,K], any alignment ----------------------------------------
//
// Workgroup (blockIdx.x, blockIdx.y) computes y[m0 .. m0+MT) x [n0 .. n0+ROWS).
// K is cut into chunks of 64*VEC elements; chunk c belongs to wave c % 4 and
// lane l reads elements [c*64*VEC + l*VEC, +VEC) of each of the ROWS rows.
// Rows past N and activation rows past M are clamped to valid addresses and
// their results discarded.
template <int VEC, int ROWS, int MT>
__global__ void __launch_bounds__(kThreads)
gemv_rd_kernel(const uint16_t *__restrict__ W, int64_t ldw, const float *__restrict__ X,
               int64_t ldx, float *__restrict__ Y, int64_t ldy, int N, int K, int M) {
    constexpr int CH = 64 * VEC;
    constexpr int U = (ROWS * MT <= 8) ? 2 : 1;  // chunks in flight per wave
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * ROWS;
    const int m0 = blockIdx.y * MT;

    const uint16_t *wrow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
        wrow[r] = W + (int64_t)min(n0 + r, N - 1) * ldw + lane * VEC;
    const float *xrow[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) xrow[m] = X + (int64_t)min(m0 + m, M - 1) * ldx + lane * VEC;

    // A lane with at least one element starts its chain at +0.0f, like the
    // reference (jit.rs:29655).  A lane with none starts at -0.0f, the exact
    // additive identity, so idle lanes cannot turn a -0.0f result (a product
    // that underflowed) into +0.0f in the reduction.  K == 0 writes +0.0f.
    const float init = (wave * CH + lane * VEC < K || K == 0) ? 0.0f : -0.0f;
    float acc[MT][ROWS];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[m][r] = init;

    auto consume = [&](const WVec<VEC> (&wv)[ROWS], int koff) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float xv[VEC];
            load_x<VEC>(xrow[m] + koff, xv);
#pragma unroll
            for (int e = 0; e < VEC; ++e)
#pragma unroll
                for (int r = 0; r < ROWS; ++r) acc[m][r] = fmaf(xv[e], widen<VEC>(wv[r], e), acc[m][r]);
        }
    };

    const int nfull = K / CH;
    int c = wave;
    for (; c + (U - 1) * kWaves < nfull; c += U * kWaves) {
        WVec<VEC> wv[U][ROWS];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < ROWS; ++r) wv[u][r].load(wrow[r] + (int64_t)(c + u * kWaves) * CH);
#pragma unroll
        for (int u = 0; u < U; ++u) consume(wv[u], (c + u * kWaves) * CH);
    }
    for (; c < nfull; c += kWaves) {
        WVec<VEC> wv[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) wv[r].load(wrow[r] + (int64_t)c * CH);
        consume(wv, c * CH);
    }
    // Partial last chunk: VEC divides K, so a lane's vector is wholly in or out.
    if (nfull * CH < K && wave == nfull % kWaves && nfull * CH + lane * VEC < K) {
        WVec<VEC> wv[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) wv[r].load(wrow[r] + (int64_t)nfull * CH);
        consume(wv, nfull * CH);
    }

    __shared__ float red[kWaves][MT * ROWS];
    {
        float a[MT * ROWS];
#pragma unroll
        for (int v = 0; v < MT * ROWS; ++v) a[v] = acc[v / ROWS][v % ROWS];
        wave_sums(a, [&](int v, float s) { red[wave][v] = s; });
    }
    __syncthreads();
    for (int i0 = wave * 64; i0 < MT * ROWS; i0 += kThreads) {  // wave-uniform: settle_zero needs whole waves
        const int i = i0 + lane < MT * ROWS ? i0 + lane : 0;
        const int m = i / ROWS, r = i % ROWS;
        float s = red[0][i];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) s += red[w][i];
        const bool store = i0 + lane < MT * ROWS && n0 + r < N && m0 + m < M;
        s = settle_zero(s, store && s == 0.0f, X + (int64_t)(store ? m0 + m : 0) * ldx,
                        W + (int64_t)(store ? n0 + r : 0) * ldw, 1, K);
        if (store) Y[(int64_t)(m0 + m) * ldy + n0 + r] = s;
    }
}

// ---- CS: W [K,N] ----------------------------------------------------------
//
// Workgroup (bx, slice, z) computes partial sums of columns [bx*CB, +CB) over
// k in [slice*kslice, +kslice) for batch slice z.  A wave-wide load covers RW
// consecutive k rows x LPR lanes x VEC columns; lane (g, cl) takes k row
// g of each group and columns cl*VEC .. +VEC.  Waves interleave row groups.
// Columns past N are clamped to column 0 and discarded.
template <int VEC, int RW, int MT>
__global__ void __launch_bounds__(kThreads)
gemv_cs_kernel(const uint16_t *__restrict__ W, int64_t rs, const float *__restrict__ X, int64_t ls,
               float *__restrict__ P, int64_t p_slice, int64_t p_z, int N, int K, int M, int kslice) {
    constexpr int LPR = 64 / RW;
    constexpr int CB = LPR * VEC;
    constexpr int STEP = kWaves * RW;
    constexpr int U = (MT <= 2) ? 4 : 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane / LPR;
    const int cl = lane % LPR;
    const int col = blockIdx.x * CB + cl * VEC;
    const int slice = blockIdx.y;
    const int64_t z = blockIdx.z;
    const int kbeg = slice * kslice;
    const int kend = min(K, kbeg + kslice);

    const uint16_t *wz = W + z * rs + (col < N ? col : 0);
    const float *xz = X + z * ls;
    float *pz = P + (int64_t)slice * p_slice + z * p_z;

    // +0.0f for a lane that owns k rows, -0.0f (the additive identity) for an
    // idle one; see gemv_rd_kernel.
    const float init = (kbeg + wave * RW + g < kend || K == 0) ? 0.0f : -0.0f;
    float acc[MT][VEC];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[m][e] = init;

    // nz: the lane's columns that met a product with two nonzero factors (zero_fold)
    uint32_t nz[MT][(VEC + 1) / 2] = {};
    auto consume = [&](const WVec<VEC> &wv, int k) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float xv = xz[(int64_t)min(m, M - 1) * K + k];
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[m][e] = fmaf(xv, widen<VEC>(wv, e), acc[m][e]);
            const uint32_t xm = xv != 0.0f ? 0x7fff7fffu : 0u;
#pragma unroll
            for (int d = 0; d < (VEC + 1) / 2; ++d) nz[m][d] |= wv.d[d] & xm;
        }
    };

    int k = kbeg + wave * RW + g;
    for (; k + (U - 1) * STEP < kend; k += U * STEP) {
        WVec<VEC> wv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u].load(wz + (int64_t)(k + u * STEP) * N);
#pragma unroll
        for (int u = 0; u < U; ++u) consume(wv[u], k + u * STEP);
    }
    for (; k < kend; k += STEP) {
        WVec<VEC> wv;
        wv.load(wz + (int64_t)k * N);
        consume(wv, k);
    }

    // Fold, then sum the RW row groups of the wave: lanes cl, cl+LPR, cl+2*LPR, ...
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const uint32_t half = VEC == 1 ? nz[m][0] : nz[m][e >> 1] >> (16 * (e & 1));
            acc[m][e] = zero_fold(acc[m][e], (half & 0x7fffu) != 0);
#pragma unroll
            for (int o = LPR; o < 64; o <<= 1) acc[m][e] += __shfl_xor(acc[m][e], o, 64);
        }

    __shared__ float red[kWaves][MT][CB];
    if (g == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int e = 0; e < VEC; ++e) red[wave][m][cl * VEC + e] = acc[m][e];
    }
    __syncthreads();
    // With one k slice P is y itself and the zero rule applies here;
    // otherwise sum_slices_kernel applies it to the slices' (folded) sum.
    const bool final_out = kslice >= K;
    for (int i = threadIdx.x; i < MT * CB; i += kThreads) {
        const int m = i / CB, c = i % CB;
        const int n = blockIdx.x * CB + c;
        float s = red[0][m][c];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) s += red[w][m][c];
        const bool store = n < N && m < M;
        if (final_out) s = zero_unfold(s, store, xz + (int64_t)(store ? m : 0) * K, W + z * rs + (store ? n : 0), N, K);
        if (store) pz[(int64_t)m * N + n] = s;
    }
}

// ---- CS streaming: W [K,N], N % 8 == 0, 16-byte aligned rows ------------------
//
// Workgroup (cb, s, z) owns output columns [cb*512, +512) of batch slice z and
// k rows [s*kslice, +kslice).  Lane l owns columns cb*512 + 8l .. +8 and loads
// them 16 bytes at a time (nontemporal); the NW waves take contiguous chunks
// of the workgroup's k rows, so x[m][k] is the same for the whole wave and
// comes through the scalar cache.  The waves' partials meet in LDS in a fixed
// order; with one k slice the workgroup writes y, otherwise its partial goes
// to P[s] and sum_slices_stream_kernel adds the slices in a fixed order.
// (Finishing inside the same launch needs device-scope fences, which on a
// multi-XCD part write back and invalidate the whole L2 per workgroup:
// measured 5x slower than the second launch.)
//
// UN: rows at any 2-byte alignment (odd N, offset views).  Buffer loads take
// 2-byte-aligned offsets exactly, and the hardware range check is per dword
// of the load: a dword that runs past the range's end comes back as zeros.
// A row's last chunk runs into the next row, which is in range except after
// the workgroup's last row; there the range extends 2 bytes, so the dword
// holding element N-1 is whole.  Those 2 bytes belong to the next row, which
// exists because the matrix's last row is left out: the slice pass applies it
// as the chain's final fma (sum_slices_stream_kernel).  Columns past N read
// the next row's first elements and are never stored.
constexpr int kCsCols = 512;

//
// G > 1 (narrow N, e.g. per-head projections with N = 64..256): the wave's
// lanes form G row groups of 64/G lanes; group g walks rows r0 + g, r0 + g +
// G, ... of the wave's range over 512/G columns, so one load instruction still
// covers 1 KiB (G rows of 1024/G bytes) where at G = 1 most lanes would sit
// past N.  x is then per lane (its row's value), loaded with the weights.  The
// groups' folded partials meet in LDS with the waves', in a fixed order.
template <int NW, int MT, bool UN, int G>
__global__ void __launch_bounds__(64 * NW)
gemv_cs_stream_kernel(const uint16_t *__restrict__ W, int64_t rs, const float *__restrict__ X, int64_t ls,
                      float *__restrict__ Y, float *__restrict__ P, int64_t z_stride, int64_t p_slice, int N,
                      int K, int M, int kslice, int slices) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "row groups per wave");
    static_assert(G == 1 || !UN, "row groups serve aligned rows");
    constexpr int CB = kCsCols / G;  // columns per workgroup
    constexpr int CL = 64 / G;       // lanes per row group
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = lane / CL;        // this lane's row group
    const int cb = blockIdx.x;
    const int s = blockIdx.y;
    const int64_t z = blockIdx.z;
    const int col = cb * CB + (lane % CL) * 8;
    const bool live = col < N;

    const int kb = s * kslice;
    const int ke = min(UN ? K - 1 : K, kb + kslice);
    const int per = (ke - kb + NW - 1) / NW;
    const int r0 = min(ke, kb + wave * per);
    const int r1 = min(ke, r0 + per);

    const float *xz = X + z * ls;
    const uint16_t *const w0 = W + z * rs + (int64_t)r0 * N;
    const uint32_t delta = UN ? (uint32_t)(reinterpret_cast<uintptr_t>(w0) & 3) : 0;  // 0 or 2
    const uint32_t range = (uint32_t)((int64_t)(r1 - r0) * N * 2) + (UN ? (delta + 2 + 3) & ~3u : 0);
    const __amdgpu_buffer_rsrc_t rsw = weight_rsrc(reinterpret_cast<const char *>(w0) - delta, range);
    const uint32_t row_bytes = (uint32_t)N * 2;
    const uint32_t lane_off = delta + (uint32_t)col * 2 + (uint32_t)rg * row_bytes;

    // +0.0f when this lane sums at least one product (or K == 0, which must
    // write +0.0f), -0.0f, the additive identity, otherwise.
    const float init = ((r0 + rg < r1 && live) || K == 0) ? 0.0f : -0.0f;
    float acc[MT][8];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][e] = init;

    // nz: the bf16 halves of the lane's columns that met a nonzero weight
    // where x is nonzero (any product with two nonzero factors; zero_fold).
    uint32_t nz[MT][4] = {};
    // xg: at G > 1 the lane's own x values, loaded with its rows' weights.
    auto consume = [&](const u32x4 &wv, int k, const float *xg) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float xv = G == 1 ? xz[(int64_t)min(m, M - 1) * K + k] : xg[m];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t d = wv[e >> 1];
                acc[m][e] = fmaf(xv, (e & 1) ? widen_hi(d) : widen_lo(d), acc[m][e]);
            }
            const uint32_t xm = xv != 0.0f ? 0x7fff7fffu : 0u;  // wave-uniform
#pragma unroll
            for (int d = 0; d < 4; ++d) nz[m][d] |= wv[d] & xm;
        }
    };

    // Two register buffers of U rows: the next U rows are in flight while the
    // current ones are summed.  Loads are unconditional (a dead lane, and a
    // row past this wave's range, read from past the buffer's end and get
    // zeros without touching memory), so the compiler waits only for the
    // buffer it sums; the row guard sits on the arithmetic, which also keeps
    // x[k] in range.
    constexpr int U = MT <= 2 ? 8 : 4;
    constexpr int XU = G == 1 ? 1 : U;  // per-lane x registers (G > 1)
    const uint32_t loff = live ? lane_off : kOutOfRange;
    u32x4 ba[U], bb[U];
    float xa[XU][MT], xb[XU][MT];
    // Buffer u holds row r + u*G + rg of each lane.
    auto load = [&](u32x4 (&b)[U], float (&xv)[XU][MT], int r) {
#pragma unroll
        for (int u = 0; u < U; ++u) b[u] = load_w16(rsw, loff, (uint32_t)(r - r0 + u * G) * row_bytes);
        if constexpr (G > 1) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = r + u * G + rg;
#pragma unroll
                for (int m = 0; m < MT; ++m) xv[u][m] = k < r1 ? xz[(int64_t)min(m, M - 1) * K + k] : 0.0f;
            }
        }
    };
    auto sum_rows = [&](const u32x4 (&b)[U], const float (&xv)[XU][MT], int r) {
        if (r + U * G <= r1) {
#pragma unroll
            for (int u = 0; u < U; ++u) consume(b[u], r + u * G + rg, xv[G == 1 ? 0 : u]);
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (r + u * G + rg < r1) consume(b[u], r + u * G + rg, xv[G == 1 ? 0 : u]);
        }
    };
    load(ba, xa, r0);
    for (int r = r0; r < r1; r += 2 * U * G) {
        load(bb, xb, r + U * G);
        sum_rows(ba, xa, r);
        if (r + U * G >= r1) break;
        load(ba, xa, r + 2 * U * G);
        sum_rows(bb, xb, r + U * G);
    }

    // The partials in LDS as two half-planes: a lane's columns 8l .. 8l+3 go
    // to the first at words 4l .. 4l+3, columns 8l+4 .. 8l+7 to the second,
    // so each 16-byte write covers consecutive words across the lanes; they
    // are read back in address order (word a of a half-plane row is column
    // (a % 4CL) / 4 * 8 + (a / 4CL) * 4 + a % 4).  Every LDS access here
    // moves consecutive words (32-byte windows written at a 32-byte stride
    // lost a third of the LDS cycles to conflicts); the price is y's stores in
    // 16-byte runs 32 bytes apart within a wave, once per workgroup.  Rows
    // are 16 words longer than their data, so two waves' words of one column
    // never share a bank (reads that fetch both at once stay whole).
    constexpr int kRow = MT * CB + 16;
    __shared__ __attribute__((aligned(16))) float red[NW * G][kRow];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float4 f;
            f.x = zero_fold(acc[m][4 * h + 0], ((nz[m][2 * h] >> 0) & 0x7fffu) != 0);
            f.y = zero_fold(acc[m][4 * h + 1], ((nz[m][2 * h] >> 16) & 0x7fffu) != 0);
            f.z = zero_fold(acc[m][4 * h + 2], ((nz[m][2 * h + 1] >> 0) & 0x7fffu) != 0);
            f.w = zero_fold(acc[m][4 * h + 3], ((nz[m][2 * h + 1] >> 16) & 0x7fffu) != 0);
            *reinterpret_cast<float4 *>(&red[wave * G + rg][m * CB + h * 4 * CL + (lane % CL) * 4]) = f;
        }
    __syncthreads();

    const int c0 = cb * CB;
    const int ncol = min(CB, N - c0);
    // With one k slice (and every row in it) the workgroup writes y and the
    // zero rule applies here; otherwise the folded partial goes to P and
    // sum_slices_stream_kernel applies it.
    const bool final_out = slices == 1 && !UN;
    float *out = final_out ? Y + z * z_stride : P + z * z_stride + (int64_t)s * p_slice;
    for (int t = threadIdx.x; t < MT * CB; t += 64 * NW) {
        const int m = t / CB, a = t - m * CB;
        const int c = (a % (4 * CL)) / 4 * 8 + (a / (4 * CL)) * 4 + a % 4;
        const bool store = m < M && c < ncol;
        float v = red[0][t];
#pragma unroll
        for (int w = 1; w < NW * G; ++w) v += red[w][t];
        if (final_out)
            v = zero_unfold(v, store, xz + (int64_t)(store ? m : 0) * K, W + z * rs + (store ? c0 + c : 0), N, K);
        if (store) out[(int64_t)m * N + c0 + c] = v;
    }
}

// Second pass of the column-stream kernels: y[i] = sum over slices of
// P[j][i] in ascending j (partials folded by zero_fold), then the zero rule
// (zero_unfold).  `src` names the
// problem, so an output's activation row and weight column can be found:
// output i of the launch is (slice z, activation row m, column n) =
// (i / (M*N), (i / N) % M, i % N), its activation row x + z*ls + m*K, its
// weights w + z*rs + n, N elements apart.
struct CsSrc {
    const uint16_t *w;
    const float *x;
    int64_t rs, ls, K, N, M;
    bool last_row;  // the UN streaming kernel left out row K-1 (below)
};

__device__ __forceinline__ float cs_unfold(float v, bool live, int64_t i, const CsSrc &src) {
    const int64_t mn = src.M * src.N;
    const int64_t z = live ? i / mn : 0, r = live ? i - z * mn : 0;
    const int64_t m = r / src.N, n = r - m * src.N;
    return zero_unfold(v, live, src.x + z * src.ls + m * src.K, src.w + z * src.rs + n, src.N, (int)src.K);
}

// The streaming kernel's pass.  A workgroup owns 64 consecutive outputs; its
// NWS waves take slices j = w, w+NWS, ... (coalesced 256-byte reads), and the
// NWS partial sums meet in LDS in wave order.  Every element's order is fixed.
// 16 waves when there are at least 16 slices, so that each lane has at most a
// few partials to fetch and they are all in flight at once (the pass is
// latency-bound: the partials were just written through other XCDs' L2s).
// With `last_row` set (the UN streaming kernel left out the matrix's last
// row): y[i] = fmaf(x[z][m][K-1], w[z][K-1][n], that sum), the chain's final
// step; wave 0 fetches those two operands before the partials.
template <int NWS>
__global__ void __launch_bounds__(64 * NWS)
sum_slices_stream_kernel(const float *__restrict__ P, int64_t p_slice, int slices, float *__restrict__ Y,
                         int64_t count, const CsSrc src) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + lane;
    const bool live = i < count;
    float xv = 0.0f;
    uint32_t wb = 0;
    if (src.last_row && wave == 0 && live) {
        const int64_t mn = src.M * src.N;
        const int64_t z = i / mn, r = i - z * mn;
        const int64_t m = r / src.N, n = r - m * src.N;
        xv = src.x[z * src.ls + m * src.K + (src.K - 1)];
        wb = src.w[z * src.rs + (src.K - 1) * src.N + n];
    }
    float s = -0.0f;
    bool first = true;
    if (live) {
#pragma unroll 4
        for (int j = wave; j < slices; j += NWS) {
            const float v = P[(int64_t)j * p_slice + i];
            s = first ? v : s + v;
            first = false;
        }
    }
    __shared__ float part[NWS][64];
    part[wave][lane] = s;
    __syncthreads();
    if (wave == 0) {
        float v = part[0][lane];
#pragma unroll
        for (int w = 1; w < NWS; ++w) v += part[w][lane];
        if (src.last_row && live)
            v = zero_fold(fmaf(xv, __uint_as_float(wb << 16), v),
                          !(v == 0.0f && __builtin_signbit(v)) || (xv != 0.0f && (wb & 0x7fffu) != 0));
        v = cs_unfold(v, live, i, src);
        if (live) Y[i] = v;
    }
}

// The general kernel's pass: y[i] = sum over slices in ascending order of
// P[s][i], then the zero rule.
__global__ void __launch_bounds__(kThreads)
sum_slices_kernel(const float *__restrict__ P, int64_t p_slice, int slices, float *__restrict__ Y,
                  int64_t count, const CsSrc src) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const bool live = i < count;
    float s = 0.0f;
    if (live) {
        s = P[i];
        for (int j = 1; j < slices; ++j) s += P[(int64_t)j * p_slice + i];
    }
    s = cs_unfold(s, live, i, src);
    if (live) Y[i] = s;
}

// ---- staging copies --------------------------------------------------------------
//
// Words between any two device-visible ranges, one small grid (16 bytes per
// thread where aligned, else 4): x from pinned host staging into device
// memory (DMC_HIP_X_KERNEL), and the deferred calls' outputs from device
// memory into pinned host staging.
__global__ void __launch_bounds__(256)
copy_words_kernel(uint32_t *__restrict__ dst, const uint32_t *__restrict__ src, int64_t words, bool v4) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    if (v4) {
        const int64_t n4 = words / 4;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
            reinterpret_cast<uint4 *>(dst)[i] = reinterpret_cast<const uint4 *>(src)[i];
        for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += stride) dst[i] = src[i];
    } else {
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += stride) dst[i] = src[i];
    }
}

// ---- measurement probe -------------------------------------------------------
//
// Read-bandwidth ceiling: workgroup b streams its contiguous share of the
// buffer in 16-byte nontemporal loads, 8 in flight per lane, and folds them
// into one word that lane 0 stores to sink[b] (so the loads are live).
constexpr int kProbeGroups = 16384;

__global__ void __launch_bounds__(kThreads)
probe_read_kernel(const uint8_t *__restrict__ src, uint64_t n16, uint32_t *__restrict__ sink) {
    const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t b = (uint64_t)blockIdx.x * per;
    const uint64_t e = min(n16, b + per);
    uint32_t acc = 0;
    if (b < e) {
        const __amdgpu_buffer_rsrc_t rs = weight_rsrc(src + b * 16, (uint32_t)((e - b) * 16));
        const uint32_t cnt = (uint32_t)(e - b);
        constexpr int U = 8;
        uint32_t i = threadIdx.x;
        for (; i + (U - 1) * kThreads < cnt; i += U * kThreads) {
            u32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) v[u] = load_w16(rs, (i + u * kThreads) * 16);
#pragma unroll
            for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
        }
        for (; i < cnt; i += kThreads) {
            const u32x4 v = load_w16(rs, i * 16);
            acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
        }
    }
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

// Synthetic weights: dst[i] = table[splitmix64((offset + i) ^ key) >> 48].
// Integer-only, so a host regenerates any element bit for bit.
__global__ void __launch_bounds__(kThreads)
fill_counter_bf16_kernel(uint16_t *__restrict__ dst, uint64_t count, uint64_t offset, uint64_t key,
                         const uint16_t *__restrict__ table) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * kThreads) {
        uint64_t z = ((offset + i) ^ key) + 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        dst[i] = table[z >> 48];
    }
}

// Weight layout change for residency: dst [cols, rows] = src [rows, cols]^T,
// bf16 bit patterns moved unchanged.  64 x 64 tiles through LDS (the row
// pitch of 66 halves spreads a tile column over the banks); both grid
// dimensions stride, so any shape fits the 65535-workgroup limit.
constexpr int kTile = 64;

__global__ void __launch_bounds__(kThreads)
transpose_bf16_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst, int64_t rows, int64_t cols) {
    __shared__ uint16_t tile[kTile][kTile + 2];
    const int tx = threadIdx.x & (kTile - 1);
    const int ty = threadIdx.x / kTile;  // 0..3
    for (int64_t r0 = (int64_t)blockIdx.y * kTile; r0 < rows; r0 += (int64_t)gridDim.y * kTile) {
        for (int64_t c0 = (int64_t)blockIdx.x * kTile; c0 < cols; c0 += (int64_t)gridDim.x * kTile) {
            for (int i = ty; i < kTile; i += kThreads / kTile) {
                const int64_t r = r0 + i, c = c0 + tx;
                if (r < rows && c < cols) tile[i][tx] = src[r * cols + c];
            }
            __syncthreads();
            for (int i = ty; i < kTile; i += kThreads / kTile) {
                const int64_t c = c0 + i, r = r0 + tx;
                if (c < cols && r < rows) dst[c * rows + r] = tile[tx][i];
            }
            __syncthreads();
        }
    }
}

// The same transpose with 16-byte accesses, for rows and cols that are
// multiples of 8 on 16-byte-aligned bases (every weight shape of the decode
// workloads).  A 64 x 64 tile: thread t loads source row r0 + t/8 (+32),
// elements c0 + 8(t%8), +8; after the barrier it gathers destination row
// c0 + t/4 (a source column), elements r0 + 16(t%4), +16, and stores them as
// two 16-byte pieces -- four threads per 128-byte line, so a wave stores 16
// whole lines.  Workgroups stride over the tiles.
constexpr int kTvPitch = 72;  // halves per tile row: 144 bytes keeps 16-byte rows

// Column of element (r, c) in the tile: its 16-byte piece c/8 is XORed with
// 2 * (r / 16 mod 4).  Rows 16 apart sit on the same banks at any 16-byte
// pitch, and the gather reads one column from rows 16 apart in the four
// threads of a quad; the XOR sends them to four different pieces.  (Without
// it two thirds of the kernel's LDS cycles were bank conflicts, rocprof
// SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.)
__device__ __forceinline__ int tv_swz(int r, int c) { return (((c >> 3) ^ (((r >> 4) & 3) << 1)) << 3) | (c & 7); }

__global__ void __launch_bounds__(256)
transpose_bf16_v8_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst, int64_t rows, int64_t cols,
                         int64_t tiles_c, int64_t ntiles) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kTile][kTvPitch];
    const int t = threadIdx.x;
    for (int64_t tl = blockIdx.x; tl < ntiles; tl += gridDim.x) {
        const int64_t r0 = (tl / tiles_c) * kTile, c0 = (tl % tiles_c) * kTile;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int lr = t / 8 + 32 * h, lc = 8 * (t % 8);
            const int64_t r = r0 + lr, c = c0 + lc;
            u32x4 v = {0, 0, 0, 0};
            if (r < rows && c < cols) v = *reinterpret_cast<const u32x4 *>(src + r * cols + c);
            *reinterpret_cast<u32x4 *>(&tile[lr][tv_swz(lr, lc)]) = v;
        }
        __syncthreads();
        const int i = t / 4, jq = t % 4;
        const int ci = tv_swz(16 * jq, i);  // the same for the 16 rows this thread reads
        uint32_t o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            o[e] = (uint32_t)tile[16 * jq + 2 * e][ci] | ((uint32_t)tile[16 * jq + 2 * e + 1][ci] << 16);
        const int64_t dr = c0 + i;
        if (dr < cols) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int64_t dc = r0 + 16 * jq + 8 * h;
                if (dc < rows)
                    *reinterpret_cast<u32x4 *>(dst + dr * rows + dc) =
                        u32x4{o[4 * h], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]};
            }
        }
        __syncthreads();
    }
}

// ---- f32 weights, row-dot: the f32 path of `W @ x` -----------------------------
//
// The reference's f32 `@` keeps the bf16 kernels' closed form with the weight
// read as f32: per output, acc = +0, then acc = fma(l[i][k], r[k][j], acc)
// over ascending k (scalar_matmul, jit.rs:20715-20802, which an f32 `W @ x`
// takes, jit.rs:20806-20831; dmc_matmul_par's matmul_tile, jit.rs:29448-29466,
// bit-identical by jit.rs:29404-29408).  Here W [N,K] f32 is the weight (rows
// are output rows) and X [M,K] the activation rows, as in the bf16 row-dot
// kernels; the caller orients its [m, n] result through the output strides:
// output (activation row a, weight row n) goes to Y[a * ys_act + n * ys_row].

// The reference chain of one f32 output (the zero rule's rare path).
__device__ float chain_f32(const float *__restrict__ w, const float *__restrict__ x, int K) {
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) acc = fmaf(x[k], w[k], acc);
    return acc;
}

__device__ __forceinline__ float zero_unfold_f32(float v, bool live, const float *x, const float *w, int K) {
    if (live && v == 0.0f) v = __builtin_signbit(v) ? 0.0f : chain_f32(w, x, K);
    return v;
}

// Streaming: gemv_rd_stream_kernel's layout with four f32 weights per 16-byte
// load.  Lane `lane` of wave `wave` owns the KV vectors of 4 elements starting
// at ((j*NW + wave)*64 + lane)*4, so for every j the workgroup reads NW KiB of
// a row contiguously; x's slice stays in registers; the workgroup walks weight
// rows [rb, rb + rpw) ROWS at a time through two register buffers (the next
// rows in flight while the current ones are summed), every load
// unconditional (past K or past the last row: offsets beyond the buffer
// resource, which read zeros).  Rows 16-byte aligned (K % 4 == 0).  Zero rule:
// the FMA kernels' fold (zero_fold), x's nonzero mask per element.
template <int NW, int KV, int ROWS, int MT>
__global__ void __launch_bounds__(64 * NW)
gemv_rd_f32_stream_kernel(const float *__restrict__ W, const float *__restrict__ X, float *__restrict__ Y, int N,
                          int K, int M, int rpw, int64_t ys_act, int64_t ys_row) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rb = (int)blockIdx.x * rpw;
    const int nr = min(N, rb + rpw) - rb;
    const int m0 = blockIdx.y * MT;
    const int mrows = min(MT, M - m0);

    const __amdgpu_buffer_rsrc_t xrs = weight_rsrc(X + (int64_t)m0 * K, (uint32_t)mrows * (uint32_t)K * 4);
    uint32_t eoff[KV];
    bool has[KV];
    u32x4 xv[MT][KV];
#pragma unroll
    for (int j = 0; j < KV; ++j) {
        const int e = ((j * NW + wave) * 64 + lane) * 4;
        has[j] = e < K;
        eoff[j] = has[j] ? (uint32_t)e * 4 : kOutOfRange;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint32_t xo = has[j] ? ((uint32_t)min(m, mrows - 1) * (uint32_t)K + (uint32_t)e) * 4 : kOutOfRange;
            xv[m][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0);
        }
    }
    // +0 for a lane that owns elements (the chain's start), -0 (the additive
    // identity) for one that owns none.
    const float init = (wave * 64 + lane) * 4 < K ? 0.0f : -0.0f;

    const __amdgpu_buffer_rsrc_t rs = weight_rsrc(W + (int64_t)rb * K, (uint32_t)((int64_t)nr * K * 4));
    const uint32_t row_bytes = (uint32_t)K * 4;
    __shared__ float red[NW][MT][kMaxRpw];

    u32x4 ba[ROWS][KV], bb[ROWS][KV];
    auto load = [&](u32x4 (&wv)[ROWS][KV], int i0) {
#pragma unroll
        for (int q = 0; q < ROWS; ++q) {
            const uint32_t base = (uint32_t)(i0 + q) * row_bytes;
#pragma unroll
            for (int j = 0; j < KV; ++j) wv[q][j] = load_w16(rs, eoff[j], base);
        }
    };
    load(ba, 0);
    float xr[MT][KV][4];
    uint32_t xm[MT][KV][4];
    auto sum_rows = [&](const u32x4 (&wv)[ROWS][KV], int i0) {
        float acc[MT][ROWS];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int q = 0; q < ROWS; ++q) acc[m][q] = init;
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int q = 0; q < ROWS; ++q) {
                    const float w = __uint_as_float(wv[q][j][e]);
#pragma unroll
                    for (int m = 0; m < MT; ++m) acc[m][q] = fmaf(xr[m][j][e], w, acc[m][q]);
                }
        // Value v of the step: activation row v / ROWS, weight row i0 + v % ROWS.
        float a[MT * ROWS];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int q = 0; q < ROWS; ++q) {
                uint32_t nz = 0;
#pragma unroll
                for (int j = 0; j < KV; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) nz |= wv[q][j][e] & xm[m][j][e];
                a[m * ROWS + q] = zero_fold(acc[m][q], nz != 0);
            }
        wave_sums(a, [&](int v, float s) {
            if (i0 + v % ROWS < nr) red[wave][v / ROWS][i0 + v % ROWS] = s;
        });
    };
    load(bb, ROWS);
    __builtin_amdgcn_sched_barrier(0);  // x's wait below comes after every load above
    // A vector past K reads +0 weights; its x becomes -0, so each of its
    // products is -0, the exact additive identity.
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < KV; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t b = xv[m][j][e] | (has[j] ? 0u : 0x80000000u);
                xr[m][j][e] = __uint_as_float(b);
                xm[m][j][e] = (b & 0x7fffffffu) != 0 ? 0x7fffffffu : 0u;
            }
    sum_rows(ba, 0);
    for (int i0 = 0; i0 + ROWS < nr; i0 += 2 * ROWS) {
        load(ba, i0 + 2 * ROWS);
        sum_rows(bb, i0 + ROWS);
        if (i0 + 2 * ROWS >= nr) break;
        load(bb, i0 + 3 * ROWS);
        sum_rows(ba, i0 + 2 * ROWS);
    }
    __syncthreads();
    for (int t0 = wave * 64; t0 < mrows * nr; t0 += 64 * NW) {
        const int t = t0 + lane;
        const bool live = t < mrows * nr;
        const int m = live ? t / nr : 0, r = live ? t - m * nr : 0;
        float s = red[0][m][r];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w][m][r];
        s = zero_unfold_f32(s, live, X + (int64_t)(m0 + m) * K, W + (int64_t)(rb + r) * K, K);
        if (live) Y[(int64_t)(m0 + m) * ys_act + (int64_t)(rb + r) * ys_row] = s;
    }
}

// General: any K (0 included), 4-byte alignment, row strides ldw and ldx.
// Four waves, one weight row each; lane `lane` takes k = lane + 64 i, four
// loads in flight; MT activation rows per workgroup (x from the caches).
template <int MT>
__global__ void __launch_bounds__(256)
gemv_rd_f32_kernel(const float *__restrict__ W, int64_t ldw, const float *__restrict__ X, int64_t ldx,
                   float *__restrict__ Y, int N, int K, int M, int64_t ys_act, int64_t ys_row) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = (int)blockIdx.x * 4 + wave;
    const int m0 = blockIdx.y * MT;
    const int mrows = min(MT, M - m0);
    if (n >= N) return;  // wave-uniform; no barrier follows
    const float *__restrict__ w = W + (int64_t)n * ldw;
    const float *__restrict__ x = X + (int64_t)m0 * ldx;
    const float init = lane < K ? 0.0f : -0.0f;
    float acc[MT];
    uint32_t nz[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        acc[m] = init;
        nz[m] = 0;
    }
    for (int k0 = 0; k0 < K; k0 += 256) {
        float wv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int k = k0 + 64 * u + lane;
            wv[u] = k < K ? w[k] : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mrows) {  // wave-uniform
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int k = k0 + 64 * u + lane;
                    if (k < K) {
                        const float xk = x[(int64_t)m * ldx + k];
                        acc[m] = fmaf(xk, wv[u], acc[m]);
                        nz[m] |= (__float_as_uint(xk) & 0x7fffffffu) != 0 &&
                                         (__float_as_uint(wv[u]) & 0x7fffffffu) != 0
                                     ? 1u
                                     : 0u;
                    }
                }
            }
        }
    }
    float a[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) a[m] = m < mrows ? zero_fold(acc[m], nz[m] != 0) : 0.0f;
    wave_sums(a, [&](int m, float s) {
        if (m < mrows) {
            s = zero_unfold_f32(s, true, x + (int64_t)m * ldx, w, K);
            Y[(int64_t)(m0 + m) * ys_act + (int64_t)n * ys_row] = s;
        }
    });
}

// dst [cols, rows] = src [rows, cols]^T for 4-byte elements (the resident
// transposed copy of an f32 `x @ W` weight): 64 x 64 tiles through LDS, one
// padded column per tile row so the transposed reads spread over the banks.
constexpr int kTileF = 64;

__global__ void __launch_bounds__(256)
transpose_f32_kernel(const float *__restrict__ src, float *__restrict__ dst, int64_t rows, int64_t cols,
                     int64_t tiles_c, int64_t ntiles) {
    __shared__ float tile[kTileF][kTileF + 1];
    const int t = threadIdx.x;
    const int lc = t & 63, lr0 = t >> 6;
    for (int64_t tl = blockIdx.x; tl < ntiles; tl += gridDim.x) {
        const int64_t r0 = (tl / tiles_c) * kTileF, c0 = (tl % tiles_c) * kTileF;
#pragma unroll
        for (int i = 0; i < kTileF / 4; ++i) {
            const int lr = lr0 + 4 * i;
            const int64_t r = r0 + lr, c = c0 + lc;
            tile[lr][lc] = r < rows && c < cols ? src[r * cols + c] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kTileF / 4; ++i) {
            const int lr = lr0 + 4 * i;
            const int64_t dr = c0 + lr, dc = r0 + lc;
            if (dr < cols && dc < rows) dst[dr * rows + dc] = tile[lc][lr];
        }
        __syncthreads();
    }
}

// IEEE binary16 bits (in the low 16 bits of h) to binary32 bits, exactly, by
// integer steps: the f16_bits_to_f32 of compiler/src/jit.rs:29231-29257
// (subnormals normalized, NaN payloads and the signalling bit kept, which a
// hardware conversion may quiet).
__device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu;
    if (exp == 0) {
        if (mant == 0) return sign;
        const int s = __clz((int)mant) - 21;  // shifts that bring the leading 1 to bit 10
        return sign | ((uint32_t)(113 - s) << 23) | (((mant << s) & 0x3ffu) << 13);
    }
    if (exp == 0x1f) return sign | 0x7f800000u | (mant << 13);
    return sign | ((exp + 112u) << 23) | (mant << 13);
}

// dst[i] = widen of the 16-bit pattern src[i] to f32: bf16 (F16 = false,
// bits << 16; NaN payloads, infinities and subnormals kept) or IEEE f16
// (F16 = true); and dst[i] = src[i]'s bits >> 16 (truncation, the inverse of
// the bf16 widen on bf16-representable values).  VEC = 8: 8 elements per
// thread per step (16-byte-aligned bases, count a multiple of 8 in the vector
// part; the remainder runs one element per thread).  Grid-stride.
template <bool F16>
__device__ __forceinline__ uint32_t widen16(uint32_t h) {
    if constexpr (F16) return f16_bits_to_f32_bits(h);
    return h << 16;
}

template <int VEC, bool F16>
__global__ void __launch_bounds__(256)
bf16_upconvert_kernel(const uint16_t *__restrict__ src, float *__restrict__ dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC == 8) {
        for (; i < n / 8; i += stride) {
            const u32x4 v = reinterpret_cast<const u32x4 *>(src)[i];
            u32x4 lo, hi;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                lo[2 * q] = widen16<F16>(v[q] & 0xffffu);
                lo[2 * q + 1] = F16 ? widen16<F16>(v[q] >> 16) : v[q] & 0xffff0000u;
                hi[2 * q] = widen16<F16>(v[q + 2] & 0xffffu);
                hi[2 * q + 1] = F16 ? widen16<F16>(v[q + 2] >> 16) : v[q + 2] & 0xffff0000u;
            }
            reinterpret_cast<u32x4 *>(dst)[2 * i] = lo;
            reinterpret_cast<u32x4 *>(dst)[2 * i + 1] = hi;
        }
        i = (n / 8) * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    }
    for (; i < n; i += stride) dst[i] = __uint_as_float(widen16<F16>((uint32_t)src[i]));
}

template <int VEC>
__global__ void __launch_bounds__(256)
f32_to_bf16_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC == 8) {
        for (; i < n / 8; i += stride) {
            const u32x4 a = reinterpret_cast<const u32x4 *>(src)[2 * i];
            const u32x4 b = reinterpret_cast<const u32x4 *>(src)[2 * i + 1];
            reinterpret_cast<u32x4 *>(dst)[i] =
                u32x4{(a[0] >> 16) | (a[1] & 0xffff0000u), (a[2] >> 16) | (a[3] & 0xffff0000u),
                      (b[0] >> 16) | (b[1] & 0xffff0000u), (b[2] >> 16) | (b[3] & 0xffff0000u)};
        }
        i = (n / 8) * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    }
    for (; i < n; i += stride) dst[i] = (uint16_t)(__float_as_uint(src[i]) >> 16);
}

// ---- dispatch -------------------------------------------------------------

int mt_for(int64_t m) {
    if (m <= 1) return 1;
    if (m <= 2) return 2;
    if (m <= 4) return 4;
    if (m <= 8) return 8;
    return 16;
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    return (v && *v) ? atoi(v) : dflt;
}

template <int VEC, int ROWS, int MT>
hipError_t rd_go(const RdProblem &p, const RdPlan &pl, hipStream_t s) {
    hipLaunchKernelGGL((gemv_rd_kernel<VEC, ROWS, MT>), dim3((unsigned)pl.grid_x, (unsigned)pl.grid_y),
                       dim3(kThreads), 0, s, p.w, p.ldw, p.x, p.ldx, p.y, p.ldy, (int)p.n, (int)p.k,
                       (int)p.m);
    return hipGetLastError();
}

template <int VEC, int ROWS>
hipError_t rd_mt(const RdProblem &p, const RdPlan &pl, hipStream_t s) {
    switch (pl.mt) {
    case 1: return rd_go<VEC, ROWS, 1>(p, pl, s);
    case 2: return rd_go<VEC, ROWS, 2>(p, pl, s);
    case 4: return rd_go<VEC, ROWS, 4>(p, pl, s);
    case 8: return rd_go<VEC, ROWS, 8>(p, pl, s);
    case 16: return rd_go<VEC, ROWS, 16>(p, pl, s);
    }
    return hipErrorInvalidValue;
}

template <int VEC>
hipError_t rd_rows(const RdProblem &p, const RdPlan &pl, hipStream_t s) {
    switch (pl.rows) {
    case 1: return rd_mt<VEC, 1>(p, pl, s);
    case 2: return rd_mt<VEC, 2>(p, pl, s);
    case 4: return rd_mt<VEC, 4>(p, pl, s);
    case 8: return rd_mt<VEC, 8>(p, pl, s);
    }
    return hipErrorInvalidValue;
}

template <int NW, int KV, int ROWS, int MT>
hipError_t rs_go(const RdGroupArgs &ga, const RdGroup &g, const RdPlan &pl, hipStream_t s) {
    static_assert(MT * KV <= 8 && ROWS * KV <= 8, "register budget");
    const dim3 grid((unsigned)ga.gstart[ga.count], (unsigned)pl.grid_y);
    if (ga.count == 1)
        hipLaunchKernelGGL((gemv_rd_stream_kernel<NW, KV, ROWS, MT, false>), grid, dim3(64 * NW), 0, s, ga,
                           (int)g.k, (int)g.m, pl.rpw);
    else
        hipLaunchKernelGGL((gemv_rd_stream_kernel<NW, KV, ROWS, MT, true>), grid, dim3(64 * NW), 0, s, ga,
                           (int)g.k, (int)g.m, pl.rpw);
    return hipGetLastError();
}

// The streaming variants that are built: MT * KV <= 8 and ROWS * KV <= 8 keep
// x and the two weight buffers within ~128 VGPRs.
template <int NW, int KV, int ROWS>
hipError_t rs_mt(const RdGroupArgs &ga, const RdGroup &g, const RdPlan &pl, hipStream_t s) {
    switch (pl.mt) {
    case 1: return rs_go<NW, KV, ROWS, 1>(ga, g, pl, s);
    case 2: if constexpr (KV <= 4) return rs_go<NW, KV, ROWS, 2>(ga, g, pl, s); break;
    case 4: if constexpr (KV <= 2) return rs_go<NW, KV, ROWS, 4>(ga, g, pl, s); break;
    case 8: if constexpr (KV <= 1) return rs_go<NW, KV, ROWS, 8>(ga, g, pl, s); break;
    }
    return hipErrorInvalidValue;
}

template <int NW, int KV>
hipError_t rs_rows(const RdGroupArgs &ga, const RdGroup &g, const RdPlan &pl, hipStream_t s) {
    switch (pl.rows) {
    case 1: return rs_mt<NW, KV, 1>(ga, g, pl, s);
    case 2: if constexpr (KV <= 4) return rs_mt<NW, KV, 2>(ga, g, pl, s); break;
    case 4: if constexpr (KV <= 2) return rs_mt<NW, KV, 4>(ga, g, pl, s); break;
    }
    return hipErrorInvalidValue;
}

template <int NW, int KV>
hipError_t rd_unaligned_go(const RdProblem &p, const RdPlan &pl, hipStream_t s) {
    // one row per step for KV = 2 and KV > 4: the compiler keeps the other
    // buffer's loads in flight there (two rows of KV = 2 made it drain them)
    constexpr int ROWS = (KV <= 4 && KV != 2) ? 2 : 1;
    if (pl.rows != ROWS) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_rd_unaligned_kernel<NW, KV, ROWS>), dim3((unsigned)pl.grid_x), dim3(64 * NW), 0, s, p.w,
                       p.x, p.y, (int)p.n, (int)p.k, (int)(pl.kmain > 0 ? pl.kmain : p.k), p.ldw, pl.rpw,
                       pl.rstep == 2 ? 1 : 0);
    return hipGetLastError();
}

hipError_t rd_unaligned_dispatch(const RdProblem &p, const RdPlan &pl, hipStream_t s) {
    if (pl.mt != 1) return hipErrorInvalidValue;
    if (pl.waves == 8) {
        switch (pl.kvec) {
        case 1: return rd_unaligned_go<8, 1>(p, pl, s);
        case 2: return rd_unaligned_go<8, 2>(p, pl, s);
        case 3: return rd_unaligned_go<8, 3>(p, pl, s);
        case 4: return rd_unaligned_go<8, 4>(p, pl, s);
        case 5: return rd_unaligned_go<8, 5>(p, pl, s);
        case 6: return rd_unaligned_go<8, 6>(p, pl, s);
        case 7: return rd_unaligned_go<8, 7>(p, pl, s);
        }
        return hipErrorInvalidValue;
    }
    if (pl.kvec != 1) return hipErrorInvalidValue;
    switch (pl.waves) {
    case 1: return rd_unaligned_go<1, 1>(p, pl, s);
    case 2: return rd_unaligned_go<2, 1>(p, pl, s);
    case 4: return rd_unaligned_go<4, 1>(p, pl, s);
    }
    return hipErrorInvalidValue;
}

hipError_t rs_dispatch(const RdGroupArgs &ga, const RdGroup &g, const RdPlan &pl, hipStream_t s) {
    if (pl.waves == 8) {
        switch (pl.kvec) {
        case 1: return rs_rows<8, 1>(ga, g, pl, s);
        case 2: return rs_rows<8, 2>(ga, g, pl, s);
        case 3: return rs_rows<8, 3>(ga, g, pl, s);
        case 4: return rs_rows<8, 4>(ga, g, pl, s);
        case 5: return rs_rows<8, 5>(ga, g, pl, s);
        case 6: return rs_rows<8, 6>(ga, g, pl, s);
        case 7: return rs_rows<8, 7>(ga, g, pl, s);
        case 8: return rs_rows<8, 8>(ga, g, pl, s);
        }
        return hipErrorInvalidValue;
    }
    if (pl.kvec != 1) return hipErrorInvalidValue;
    switch (pl.waves) {
    case 1: return rs_rows<1, 1>(ga, g, pl, s);
    case 2: return rs_rows<2, 1>(ga, g, pl, s);
    case 4: return rs_rows<4, 1>(ga, g, pl, s);
    }
    return hipErrorInvalidValue;
}

// One launch: batch slices [z0, z0+nz), activation rows [m0, m0+mc).
template <int VEC, int RW, int MT>
hipError_t cs_go(const CsProblem &p, const CsPlan &pl, float *P, int64_t p_slice, int64_t z0,
                 int64_t nz, int64_t m0, int64_t mc, hipStream_t s) {
    const int64_t p_z = p.m * p.n;
    hipLaunchKernelGGL((gemv_cs_kernel<VEC, RW, MT>), dim3((unsigned)pl.grid_x, (unsigned)pl.slices,
                       (unsigned)nz), dim3(kThreads), 0, s, p.w + z0 * p.rs, p.rs,
                       p.x + z0 * p.ls + m0 * p.k, p.ls, P + z0 * p_z + m0 * p.n, p_slice, p_z,
                       (int)p.n, (int)p.k, (int)mc, (int)pl.kslice);
    return hipGetLastError();
}

template <int VEC, int RW>
hipError_t cs_mt(const CsProblem &p, const CsPlan &pl, float *P, int64_t ps, int64_t z0, int64_t nz,
                 int64_t m0, int64_t mc, hipStream_t s) {
    switch (pl.mt) {
    case 1: return cs_go<VEC, RW, 1>(p, pl, P, ps, z0, nz, m0, mc, s);
    case 2: return cs_go<VEC, RW, 2>(p, pl, P, ps, z0, nz, m0, mc, s);
    case 4: return cs_go<VEC, RW, 4>(p, pl, P, ps, z0, nz, m0, mc, s);
    case 8: return cs_go<VEC, RW, 8>(p, pl, P, ps, z0, nz, m0, mc, s);
    case 16: return cs_go<VEC, RW, 16>(p, pl, P, ps, z0, nz, m0, mc, s);
    }
    return hipErrorInvalidValue;
}

template <int NW, int MT, int G>
hipError_t css_go(const CsProblem &p, const CsPlan &pl, float *P, int64_t z0, int64_t nz, int64_t m0,
                  int64_t mc, hipStream_t s) {
    const int64_t zs = p.m * p.n;
    const dim3 grid((unsigned)pl.grid_x, (unsigned)pl.slices, (unsigned)nz);
    if (pl.cb != kCsCols / G || pl.grid_x * pl.cb < p.n) return hipErrorInvalidValue;
    if (pl.unaligned) {
        if (G != 1) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gemv_cs_stream_kernel<NW, MT, true, 1>), grid, dim3(64 * NW), 0, s, p.w + z0 * p.rs,
                           p.rs, p.x + z0 * p.ls + m0 * p.k, p.ls, p.y + z0 * zs + m0 * p.n, P + z0 * zs + m0 * p.n,
                           zs, p.batch * zs, (int)p.n, (int)p.k, (int)mc, (int)pl.kslice, (int)pl.slices);
    } else {
        hipLaunchKernelGGL((gemv_cs_stream_kernel<NW, MT, false, G>), grid, dim3(64 * NW), 0, s, p.w + z0 * p.rs,
                           p.rs, p.x + z0 * p.ls + m0 * p.k, p.ls, p.y + z0 * zs + m0 * p.n,
                           P ? P + z0 * zs + m0 * p.n : nullptr, zs, p.batch * zs, (int)p.n, (int)p.k, (int)mc,
                           (int)pl.kslice, (int)pl.slices);
    }
    return hipGetLastError();
}

hipError_t css_dispatch(const CsProblem &p, const CsPlan &pl, float *P, int64_t z0, int64_t nz, int64_t m0,
                        int64_t mc, hipStream_t s) {
#define DMC_CSS(NW, G)                                                 \
    switch (pl.mt) {                                                   \
    case 1: return css_go<NW, 1, G>(p, pl, P, z0, nz, m0, mc, s);      \
    case 2: return css_go<NW, 2, G>(p, pl, P, z0, nz, m0, mc, s);      \
    case 4: return css_go<NW, 4, G>(p, pl, P, z0, nz, m0, mc, s);      \
    }                                                                  \
    return hipErrorInvalidValue;
    if (pl.waves == 4 && pl.rw == 2) { DMC_CSS(4, 2) }
    if (pl.waves == 4 && pl.rw == 4) { DMC_CSS(4, 4) }
    if (pl.waves == 4 && pl.rw == 8) { DMC_CSS(4, 8) }
    if (pl.rw > 1) return hipErrorInvalidValue;
    switch (pl.waves) {
    case 2: DMC_CSS(2, 1)
    case 4: DMC_CSS(4, 1)
    case 8: DMC_CSS(8, 1)
    }
#undef DMC_CSS
    return hipErrorInvalidValue;
}

hipError_t cs_dispatch(const CsProblem &p, const CsPlan &pl, float *P, int64_t ps, int64_t z0,
                       int64_t nz, int64_t m0, int64_t mc, hipStream_t s) {
    if (pl.vec == 8 && pl.rw == 4) return cs_mt<8, 4>(p, pl, P, ps, z0, nz, m0, mc, s);
    if (pl.vec == 8 && pl.rw == 1) return cs_mt<8, 1>(p, pl, P, ps, z0, nz, m0, mc, s);
    if (pl.vec == 4 && pl.rw == 1) return cs_mt<4, 1>(p, pl, P, ps, z0, nz, m0, mc, s);
    if (pl.vec == 2 && pl.rw == 1) return cs_mt<2, 1>(p, pl, P, ps, z0, nz, m0, mc, s);
    if (pl.vec == 1 && pl.rw == 1) return cs_mt<1, 1>(p, pl, P, ps, z0, nz, m0, mc, s);
    return hipErrorInvalidValue;
}

}  // namespace

namespace {

// Streaming plan for `count` packed problems of n[i] rows sharing m and k.
// False when k is outside the kernel's register budget.
bool plan_stream(int64_t m, int64_t k, const int64_t *n, int count, int64_t cus, RdPlan &pl) {
    if (k < 1 || k > 32768 || env_int("DMC_HIP_RD_STREAM", 1) == 0) return false;
    const int nw = k <= 512 ? 1 : k <= 1024 ? 2 : k <= 2048 ? 4 : 8;
    const int kv = (int)((k + nw * 512 - 1) / (nw * 512));
    const int mt_cap = kv == 1 ? 8 : kv == 2 ? 4 : kv <= 4 ? 2 : 1;
    const int mt = std::min(mt_for(m), mt_cap);
    const int64_t gy = (m + mt - 1) / mt;
    auto blocks = [&](int64_t r) {
        int64_t b = 0;
        for (int i = 0; i < count; ++i) b += (n[i] + r - 1) / r;
        return b;
    };
    // Rows per register buffer: 2, or 1 for rows of 3 or more vectors per
    // lane (same box, 1 / 2 rows per step, us: W[4097,11008] 15.6 / 15.85,
    // W[4097,14336] 19.2 / 20.95; at 2 vectors even or behind: [4097,8192]
    // 11.82 / 11.77, [6000,6144] 13.15 / 12.98) and for 2 vectors at two or
    // more activation rows (C2 down at m = 2: 21.4-21.5 us against
    // 22.0-22.2 with 2).  At one activation row
    // and one window per lane, 4 rows in one step while 4-row workgroups
    // number at most 8 per CU: every load of a short-lived workgroup in
    // flight at once (same box, 4 / 2 rows per step, us: [1024,4096] 3.56 /
    // 3.62, [1792,4096] 4.54 / 4.84, [2048,4096] 4.66 / 5.06, C1 6.98 /
    // 7.12, [8192,4096] 11.54 / 11.68, [4096,2048] 4.89 / 4.99); on larger
    // grids 2 rows stay ahead (C2 up 18.3 against 18.5, C4 141.9 against
    // 143.4).
    const int rows_default =
        kv >= 3 || (kv == 2 && mt >= 2) ? 1 : mt == 1 && kv == 1 && blocks(4) * gy <= 8 * cus ? 4 : 2;
    int rows = env_int("DMC_HIP_RD_ROWS", rows_default);
    if (!(rows == 1 || rows == 2 || (rows == 4 && kv <= 2))) rows = rows_default;
    // Rows per workgroup, measured on MI355X: 4 for short rows (k <= 4096
    // per 8 waves: up/gate 18.1 us, 8 rows 18.5), fewer when that would leave
    // under 4 workgroups per CU; 8 for long ones (down, k = 14336: 19.0 us,
    // 4 rows 19.8), fewer when that would leave under 2 per CU.  With two or
    // more activation rows each weight row's x reads weigh more: 16 short
    // rows (C2 up at m = 2, capped to 8 by the grid: 19.6 us against 21.8 at
    // 4; C4: 146.6 against 172.1 at 4 and 148.8 at 8).
    const int rpw_default = mt >= 2 && kv == 1 ? 16 : kv >= 2 ? 8 : 4;
    const int64_t min_blocks = (kv >= 2 ? 2 : 4) * cus;
    int rpw = env_int("DMC_HIP_RD_RPW", rpw_default);
    if (rpw < 1) rpw = rpw_default;
    while (rpw > rows && blocks(rpw) * gy < min_blocks) rpw >>= 1;
    rpw = std::max(rows, std::min(kMaxRpw, (rpw + rows - 1) / rows * rows));
    if ((int64_t)rpw * k * 2 > INT32_MAX || blocks(rpw) > INT32_MAX || gy > 65535) return false;
    pl.vec = 8;
    pl.rows = rows;
    pl.mt = mt;
    pl.waves = nw;
    pl.kvec = kv;
    pl.rpw = rpw;
    pl.grid_x = blocks(rpw);
    pl.grid_y = gy;
    return true;
}

}  // namespace

// Streaming over rows at any 2-byte alignment (odd K, offset views), or over
// aligned rows with a short tail: M == 1, x 16-byte aligned.
static bool plan_unaligned(const RdProblem &p, int vec, int64_t cus, RdPlan &sp) {
    if (!(p.m == 1 && p.k >= 1 && p.k <= 32768 && p.ldw >= p.k && aligned(p.x, 16) &&
          env_int("DMC_HIP_RD_UNALIGNED", 1) != 0))
        return false;
    const int nw = p.k <= 512 ? 1 : p.k <= 1024 ? 2 : p.k <= 2048 ? 4 : 8;
    const int64_t block = (int64_t)nw * 512;
    // Rows read from the dword below them (ldw odd, or W at 2 mod 4) have
    // windows shifted by one element, which leaves one more element to the
    // short tail (at most 8 in all).
    const bool shifted = (p.ldw & 1) != 0 || !aligned(p.w, 4);
    const int64_t over = p.k % block;
    // 1..8 elements past whole blocks of windows (k = 4097) go to each row's
    // short tail, read element by element; otherwise the last block of
    // windows holds the rest.
    const bool short_tail = p.k > block && over >= 1 && over <= (shifted ? 7 : 8) &&
                            env_int("DMC_HIP_RD_SHORT_TAIL", 1) != 0;
    const int kv = short_tail ? (int)(p.k / block) : (int)((p.k + block - 1) / block);
    // ldw odd: rows alternate between 0 and 2 mod 4 bytes, and a workgroup
    // takes every other row of a block of 2 * rpw, so all its rows share one
    // alignment (see the kernel).
    const int rstep = (p.ldw & 1) ? 2 : 1;
    const int rpw_default = kv >= 2 ? 8 : 4;
    const int64_t min_blocks = (kv >= 2 ? 2 : 4) * cus;
    auto groups = [&](int r) { return (p.n + (int64_t)rstep * r - 1) / ((int64_t)rstep * r) * rstep; };
    int rpw = rpw_default;
    while (rpw > 2 && groups(rpw) < min_blocks) rpw >>= 1;
    // Only when the last block of windows is at least half full, or the
    // rest is a short tail: measured on MI355X against the general
    // kernel, k = 4095 67% vs 57% of peak, 11007 64% vs 60%, 14335 64% vs
    // 56%, but k = 4097 as a one-element last block 53% vs 61%.
    // KV = 8 (k above 28,680) would need more than 256 VGPRs with the
    // product masks: the general kernel takes it.
    if (!(kv <= 7 && (short_tail || p.k - (kv - 1) * block >= block / 2) &&
          ((int64_t)rstep * rpw * p.ldw + 8) * 2 <= INT32_MAX && groups(rpw) <= INT32_MAX))
        return false;
    sp = RdPlan{};
    sp.vec = vec;
    sp.rows = (kv <= 4 && kv != 2) ? 2 : 1;
    sp.mt = 1;
    sp.waves = nw;
    sp.kvec = kv;
    sp.rpw = rpw;
    sp.any_align = true;
    sp.rstep = rstep;
    sp.grid_x = groups(rpw);
    sp.grid_y = 1;
    sp.kmain = short_tail ? kv * block : p.k;
    return true;
}

RdPlan plan_rd(const RdProblem &p, int num_cus) {
    RdPlan pl{};
    // Widest load the row alignment allows: every row start, every activation
    // row start and the base pointers must be aligned to the vector size.
    for (int v : {8, 4, 2, 1}) {
        if (p.k % v == 0 && p.ldw % v == 0 && p.ldx % v == 0 && aligned(p.w, 2 * v) &&
            aligned(p.x, 4 * v)) {
            pl.vec = v;
            break;
        }
    }
    const int64_t cus = num_cus > 0 ? num_cus : 256;

    // One to four activation rows on rows of 1024 < K <= 4096: the 14-wave
    // kernel's layout on one group of 8 waves, or of 4 for K <= 2048 (a
    // window per lane, x in registers, 16 rows per workgroup, zeros settled
    // after the stream; 3 or 4 workgroups share a CU at 8 waves).  Same
    // boxes, group / default, us:
    // - M = 1, where the groups spread evenly over at most two rounds: C1
    //   6.66 / 6.88, [8192,4096] 11.36 / 11.61, [4096,3072] 5.47 / 6.34; on 4
    //   waves TP = 8 down [4096,1792] 4.07 / 4.51, [8192,2048] 6.69 / 7.17,
    //   [4096,1536] 3.86 / 4.30; elsewhere the 4-row streaming workgroups win
    //   ([5120,4096] 9.09 / 8.03, [28672,4096] 34.65 / 33.77, [1024,4096] 4.62
    //   / 3.32, [2048,2048] 3.73 / 3.55);
    // - 8 waves, M = 2 from 3/4 of a round: C2 up 19.41-19.46 / 20.03-20.08,
    //   C1 7.11 / 7.97, [12288,4096] 16.38 / 17.50 ([5120,4096] the loss, 9.85
    //   / 9.41);
    // - 8 waves, M = 3 everywhere: C2 up 20.10-20.29 / 20.82-20.91 (rows16),
    //   [1024,4096] 5.95 / 6.99, [12288,4096] 16.96 / 19.85;
    // - 8 waves, M = 4 except between one and two rounds of resident groups
    //   (three per CU): [12288,4096] 17.90 / 19.88, TP = 8 gate/up
    //   [1792,4096] 6.56 / 7.25, C4 150.6 / 153.1, [28672,4096] 37.2-37.7 /
    //   38.0-38.2; C2 up's 896 groups leave a short second round (21.14-21.47
    //   / 20.83-20.86).  C4 at M = 2 / 3: 145.4 / 146.4 against 146.5 / 154.2;
    // - 4 waves, M = 2 to 4 on full windows (K > 1792) from two rounds:
    //   [8192,2048] 6.95 / 7.63 / 7.30 against 7.88 / 9.06 / 9.10, [14336,2048]
    //   11.30 / 11.94 / 12.46 against 11.37 / 12.57 / 12.61 (TP = 8 down at
    //   one round: 5.12 / 5.47 / 5.67 against 5.04 / 5.42 / 5.44).
    // At K = 2048 on 8 waves, or 1024 on 4, half the lanes would hold no
    // window ([4096,2048] and [16384,1024] lost at every M).  DMC_HIP_RD_X8:
    // 0 never, 2 wherever it applies (K <= 4096, 4 waves for K <= 2048);
    // explicit MFMA, rows16 or rows-per-step settings keep their kernels.
    const int x8 = env_int("DMC_HIP_RD_X8", 1);
    const int64_t g16x = (p.n + 15) / 16;
    const int gw = p.k <= 4 * 512 ? 4 : 8;  // waves per group
    const bool x8_env_ok = env_int("DMC_HIP_RD_XLDS", 1) != 2 && env_int("DMC_HIP_RD_MFMA_KIND", 0) == 0 &&
                           env_int("DMC_HIP_RD_MFMA_MIN_M", -1) < 0 && env_int("DMC_HIP_RD_ROWS", 0) == 0 &&
                           env_int("DMC_HIP_RD_R16_TILES", 0) == 0 && env_int("DMC_HIP_RD_R16_SPLIT", -1) < 0;
    const bool even = g16x % cus == 0 && g16x <= 2 * cus;
    // N = r * CUs rows, r = 4, 6, 7, 8, 10, 12 or 14 (8 waves): one group of
    // r rows per CU.  Same box, group / default, us: one activation row,
    // [1024,4096] 3.30 / 3.46 (the drop-in's stacked k/v heads), [1536,4096]
    // 3.93 / 4.39, TP = 8 gate/up [1792,4096] 4.20 / 4.54, [2048,4096] 4.40 /
    // 4.70, [2560,4096] 5.07 / 5.60, [3072,4096] 5.52 / 5.80, [3584,4096] 6.09
    // / 6.71, [1792,3072] 3.78 / 4.33 (16-row groups there: 4.38-5.13); two to
    // four rows up to r = 12, m = 2 / 3 / 4: [1024,4096] 3.67 / 3.93 / 4.24
    // against 4.09 / 6.03 / 6.42, TP = 8 gate/up 4.51 / 5.01 / 5.39 against
    // 5.80 / 6.29 / 6.64, [3072,4096] 5.86 / 6.51 / 7.00 against 6.03 / 6.83 /
    // 7.15 (r = 14 lost: [3584,4096] 6.58 / 7.32 / 7.83 against 6.39 / 7.05 /
    // 7.37).
    const int64_t rpc = p.n % cus == 0 ? p.n / cus : 0;
    const bool per_cu = gw == 8 && (rpc == 4 || rpc == 6 || rpc == 7 || rpc == 8 || rpc == 10 || rpc == 12 || rpc == 14) &&
                        (p.m == 1 || (p.m <= 4 && rpc <= 12));
    const bool x8_auto =
        x8 == 1 && x8_env_ok &&
        (gw == 8 ? (p.m == 1   ? even || per_cu
                    : per_cu   ? true
                    : p.m == 2 ? 4 * g16x >= 3 * cus
                    : p.m == 3 ? true
                               : g16x <= 3 * cus || g16x >= 6 * cus)
                 : p.k > 1024 && (p.m == 1 ? even : p.k > 1792 && g16x >= 2 * cus));
    if ((x8 == 2 || x8_auto) && p.m >= 1 && p.m <= kX14MaxM && pl.vec == 8 && p.ldw == p.k && p.ldx == p.k &&
        p.ldy == p.n && p.k > 0 && p.k <= 8 * 512) {
        RdPlan xp{};
        xp.vec = 8;
        xp.waves = gw;
        xp.xreg8 = true;
        xp.kvec = 1;
        xp.rows = 4;
        xp.rpw = 16;
        xp.mt = (int)p.m;
        xp.grid_x = g16x;
        xp.grid_y = 1;
        if (per_cu) {
            xp.rpw = (int)rpc;
            xp.rows = rpc <= 8 ? (int)rpc : (int)rpc / 2;
            xp.grid_x = cus;
        }
        return xp;
    }

    // Three or four activation rows on long rows (4096 < K <= 14336, packed
    // 128-bit rows, 16-row workgroups in whole rounds of one per CU, as at
    // M = 1 and 2 below): the 14-wave streaming kernel with every activation
    // row's x in registers, W read once and no x split.  Same box, C2 down,
    // 14-wave / rows16: m = 3 20.1-20.2 / 21.8 us, m = 4 21.3-21.4 / 21.9
    // (DMC_HIP_RD_X14_MAX_M: 2 leaves both to rows16, 3 keeps M = 4 there).
    // An explicit DMC_HIP_RD_MFMA_KIND keeps the MFMA layout it names;
    // DMC_HIP_RD_XLDS=2 takes the kernel wherever it applies.
    {
        const int64_t g16 = (p.n + 15) / 16;
        const int xl = env_int("DMC_HIP_RD_XLDS", 1);
        if (p.m >= 3 && p.m <= std::min(kX14MaxM, env_int("DMC_HIP_RD_X14_MAX_M", kX14MaxM)) && pl.vec == 8 &&
            p.ldw == p.k && p.ldx == p.k && p.ldy == p.n && p.k > 0 && p.k <= kX14MaxK && xl != 0 &&
            env_int("DMC_HIP_RD_X14", 1) != 0 && env_int("DMC_HIP_RD_MFMA_KIND", 0) == 0 &&
            (xl == 2 || (p.k > 4096 && g16 >= cus && (g16 % cus == 0 || g16 >= 4 * cus)))) {
            RdPlan xp{};
            xp.vec = 8;
            xp.waves = kX14Waves;
            xp.kvec = (int)((p.k + kX14Waves * 512 - 1) / (kX14Waves * 512));
            xp.rows = 4;
            xp.rpw = 16;
            xp.mt = (int)p.m;
            xp.grid_x = g16;
            xp.grid_y = 1;
            return xp;
        }
    }

    // MFMA kernels for skinny M >= 2: packed rows, k a multiple of 64.  The
    // layout, by measurement on MI355X: rows16 with compact x for M <= 5 (C4
    // m = 2..4: 152-156 us against 158-160 for the gemm and wide layouts) and
    // up to M = 8 on matrices up to 256 MiB; from there the gemm layout or,
    // on matrices it streams fast enough, rows16 (below).  The wide layout is
    // kept for DMC_HIP_RD_MFMA_KIND=6.
    // (A third layout, 16-row tiles with k split over the waves, measured
    // 1.2-2.7x slower than rows16 on every shape and was removed.)
    // From 3 activation rows, or from 2 where the streaming kernel does not
    // take both in one pass (rows too long for its registers at m = 2: it
    // would stream W once per activation row; [32768,28672] 521 us against
    // 269 on rows16).  Elsewhere at m = 2 the streaming kernel is as fast or
    // faster (same box, streaming / rows16, us: C2 up 20.6 / 20.5, down 22.3 /
    // 22.0, [1024,4096] 4.4 / 7.1, [4096,11008] 17.9 / 21.3, [11008,4096]
    // 17.4 / 18.7, C4 147.1 / 154.0; C1 9.3 / 8.4 the one loss); at m = 3 and
    // 4 it is 7-80% slower everywhere.
    RdPlan sfit{};
    const bool stream_fits = plan_stream(p.m, p.k, &p.n, 1, num_cus > 0 ? num_cus : 256, sfit) && sfit.mt >= p.m;
    const int mfma_min_m = env_int("DMC_HIP_RD_MFMA_MIN_M", stream_fits ? 3 : 2);
    if (mfma_min_m > 0 && p.m >= mfma_min_m && p.k >= 64 && p.k % 64 == 0 && p.k <= INT32_MAX / 2 &&
        aligned(p.w, 16) && aligned(p.x, 16) && p.ldw == p.k && p.ldx == p.k && p.ldy == p.n &&
        (int64_t)16 * 4 * p.k <= INT32_MAX && (p.m + 15) / 16 <= 65535) {  // rows16: 16 x rows of f32
        RdPlan mp{};
        mp.mfma = true;
        mp.vec = 8;
        mp.rows = 16;
        mp.mt = 16;
        mp.kvec = 0;
        const int64_t gy = (p.m + 15) / 16;
        // From 9 activation rows, the gemm layout (16 * MB rows per workgroup:
        // W streams once per 16, 32 or 64 rows; at 16-row tiles it splits x
        // in the kernel), except where rows16 (which streams W once per 16
        // activation rows and needs no extra launch unless k is split) is
        // faster.  Measured, rows16 / gemm in us:
        // - up to 16 activation rows on matrices up to 112 MiB: [8192,4096]
        //   at m = 9 / 12 / 16 16.8 / 16.8 / 18.1 against 21.5 / 21.8 / 22.5;
        //   C2 up 27.1 / 27.8 / 29.3 against 29.1 / 30.7 / 31.6, down 25.9 /
        //   26.8 / 28.2 against 29.5 / 30.2 / 31.6 (two blocks per workgroup
        //   on up; four measured faster still).  At 224 MiB they tie
        //   ([28672,4096] m = 16: 49.8 / 49.2 on four blocks), at 392 MiB
        //   and C4 gemm wins ([14336,14336] m = 16: 83.1 / 73.3; C4 m = 12 /
        //   16: 193.7 / 203.3 against 175.8 / 162.4).
        // - small matrices while the weights streamed total at most 128 MiB
        //   (matrix up to 32 MiB) or 80 MiB: C1 at m = 32 / 64 17.2 / 30.1
        //   against 25.8 / 35.0 (m = 80, 160 MiB: 39.6 / 35.5); [4096,2048] at
        //   m = 128 30.7 / 34.5 (m = 192: 41.7 / 40.3); [1024,4096] at m = 128
        //   16.3 / 32.4; [8192,4096] at m = 24 (128 MiB) 29.6 / 27.9.
        const int64_t wbytes = (int64_t)2 * p.n * p.k;
        const int64_t small_cap = wbytes <= ((int64_t)32 << 20) ? ((int64_t)128 << 20) : ((int64_t)80 << 20);
        const bool small = gy * wbytes <= small_cap;
        const bool r16_mid = p.m <= 16 && wbytes <= (int64_t)env_int("DMC_HIP_RD_R16_MID_MIB", 128) << 20;
        // From 6 activation rows on matrices above 256 MiB the gemm layout
        // (its k order rotated per workgroup, chunk_rotation) beats rows16
        // (same box, rows16 / gemm, us: C4 m = 6 / 8 160.8 / 165.3 against
        // 159.7 / 160.5; [14336,14336] m = 6 / 8 75.2 / 77.6 against 67.6 /
        // 68.3); at 224 MiB it does not ([28672,4096] m = 6 / 8 41.1 / 41.6
        // against 47.1 / 48.0: 112 row blocks, so the gemm layout splits k),
        // nor at m = 4 / 5 on C4 (156.5 / 158.0 against 160.1 / 159.2).
        const int gemm_min_m = env_int("DMC_HIP_RD_GEMM_MIN_M", wbytes > ((int64_t)256 << 20) ? 6 : 9);
        const int kind = env_int("DMC_HIP_RD_MFMA_KIND", p.m < gemm_min_m || small || r16_mid ? 7 : 8);
        const bool rows256_fit = (int64_t)kWideRows * p.k * 2 <= INT32_MAX;  // 256-row buffer range
        const bool planes_fit = (int64_t)6 * p.m * p.k <= INT32_MAX;          // x planes' buffer range
        mp.mkind = (kind == 6 || (kind == 8 && planes_fit)) && rows256_fit ? kind : 7;
        mp.waves = 8;
        if (mp.mkind == 8) {
            // 16 activation rows per workgroup up to m = 16 (no half-empty
            // MFMA tiles: C1 at m = 12 / 16, 20.0 / 21.3 us against 20.5 /
            // 22.5 with 32-row tiles, C2 within 0.5 us), 32 up to m = 32, 64
            // above (C2 up / down: m = 48 50 / 55 us against 60 / 66 on 32-row
            // tiles, m = 128 80 / 79 against 94 / 94, m = 256 124 / 125
            // against 152 / 158).
            const int gmt = env_int("DMC_HIP_GEMM_MT", p.m <= 16 ? 16 : p.m <= 32 ? 32 : 64);
            mp.mt = gmt == 16 ? 16 : gmt == 32 ? 32 : 64;
            // 8 waves (256 weight rows) per workgroup, or 4 (128 rows, two
            // workgroups per CU) with 32-row tiles where 256-row tiles would
            // not fill the device without a k split.  Same box, 8 / 4 waves,
            // us: C2 up m = 17 / 24 / 32 36.7 / 38.8 / 42.2 against 30.9 /
            // 33.9 / 38.3, down 37.2 / 40.2 / 44.1 against 32.7 / 36.9 / 40.9;
            // [28672,4096] m = 17 / 32 61.6 / 70.2 against 53.9 / 61.5.  C4
            // (501 tiles of 256 rows) loses with 4 (m = 17 / 32 182 / 196
            // against 206 / 225), and so do 64-row tiles everywhere (C2 up /
            // down m = 64 55 / 57 against 61 / 61, m = 512 232 / 236 against
            // 268 / 300: each workgroup stages x for half the rows).
            const int64_t tiles8 = ((p.n + 255) / 256) * ((p.m + mp.mt - 1) / mp.mt);
            const int gw = env_int("DMC_HIP_GEMM_WAVES", 0);
            mp.waves = (gw == 4 || (gw != 8 && mp.mt == 32 && tiles8 < cus)) && mp.mt >= 32 ? 4 : 8;
            mp.rpw = 32 * mp.waves;
            // Split k while the grid fits one workgroup per CU (16-row tiles:
            // two), kchunks chunks of 64 per slice; when that leaves a lone
            // round under 70% full, fill two rounds instead.  Measured on C2's
            // shapes: one workgroup per CU beats two for 32- and 64-row tiles
            // at every m from 32 to 512 (m = 128: 80 / 79 us against 89 / 88;
            // m = 256: 124 / 125 against 140 / 135), except up at m = 192,
            // whose 168 tiles leave a third of the CUs idle (112 us on three
            // slices against 124 on one).
            const int64_t tiles = ((p.n + mp.rpw - 1) / mp.rpw) * ((p.m + mp.mt - 1) / mp.mt);
            const int64_t nchunks = p.k / 64;
            const int64_t per_cu =
                std::max(1, env_int("DMC_HIP_GEMM_PER_CU", mp.mt == 16 || mp.waves == 4 ? 2 : 1));
            int64_t want = std::max<int64_t>(1, per_cu * cus / tiles);
            if (tiles < cus && tiles * want * 10 < cus * 7) want = std::max<int64_t>(1, 2 * per_cu * cus / tiles);
            // A slice of fewer than 8 chunks pays its pipeline fill and output
            // too often: halve the split (C2 down at m = 12 / 16 on 16-row
            // tiles: 35.0 / 37.2 us on 16 slices of 14 chunks against 37.3 /
            // 40.4 on 32 of 7).
            const int64_t min_chunks = std::max(1, env_int("DMC_HIP_GEMM_MIN_CHUNKS", 8));
            while (want > 1 && (nchunks + want - 1) / want < min_chunks) want = (want + 1) / 2;
            want = std::min<int64_t>({want, nchunks, (int64_t)env_int("DMC_HIP_GEMM_MAX_SLICES", 64)});
            want = std::max<int64_t>(want, 1);
            mp.kchunks = (int)((nchunks + want - 1) / want);
            mp.kslices = (int)((nchunks + mp.kchunks - 1) / mp.kchunks);
            // Workgroups split their own chunks of x (no planes, no split
            // launch) at 16-row tiles (C2 down at m = 16: the split launch cost
            // 3-4 us of 37), and at 32 and 64 while the repeated split stays
            // small: each of the gx column blocks splits all of x, so while gx
            // * m <= 8192.  Same box, planes / fused, us: C2 down m = 32 / 64 /
            // 128 / 256 / 512 41.0 / 56.6 / 79.3 / 125.7 / 235.8 against 35.5 /
            // 50.7 / 75.1 / 120.1 / 218.7 (16 column blocks); up m = 32 / 64 /
            // 128 37.9 / 55.4 / 80.0 against 36.2 / 51.1 / 79.4, but m = 256 /
            // 512 122.2 / 230.8 against 126.0 / 248.0 (56 column blocks).
            const int fenv = env_int("DMC_HIP_GEMM_FUSE", 1);  // 0: never; 2: always
            const int64_t gx = (p.n + mp.rpw - 1) / mp.rpw;
            mp.xfuse = fenv == 2 || (fenv == 1 && (mp.mt == 16 || gx * p.m <= 8192));
            const size_t planes = mp.xfuse ? 0 : ((size_t)3 * p.m * p.k * 2 + 255) / 256 * 256;
            mp.workspace_bytes = planes + (mp.kslices > 1 ? (size_t)mp.kslices * p.m * p.n * 4 : 0);
        } else if (mp.mkind == 6) {
            mp.rpw = kWideRows;
        } else {
            // rows16: T 16-row blocks per workgroup, gridDim.x apart, while
            // the grid keeps >= 1 workgroup per CU.  At MC = 4 and 8 two blocks
            // share each x split (C4 m = 8: 165 us against 195 with one block
            // and 174 on the wide layout; C2 up m = 3 / 4 / 6 / 8: 20.4 / 20.5
            // / 22.5 / 22.8 us against 21.2 / 21.7 / 26.4 / 26.4 with one; C2
            // down and C1, 256 blocks, keep one unless k is split, below).
            mp.mt = p.m <= 4 ? 4 : p.m <= 8 ? 8 : 16;
            // At MC = 16 the x split is as many values as one block's weights,
            // so up to four blocks share it, on a grid of at least 7/8 of the
            // CUs: C2 up/gate (896 blocks, 224 workgroups) m = 9 / 12 / 16 23.8
            // / 24.8 / 26.2 us against 26.9 / 27.9 / 30.2 on two blocks (448);
            // C1 at m = 64 22.3 against 28.8; [4096,2048] at m = 64 / 128 14.1 /
            // 26.0 against 17.0 / 29.1.  At MC = 4 and 8 four blocks tie with
            // two on C2 (m = 4 21.4 / 21.1, m = 8 23.2 / 23.8) and lose on C4.
            // At MC = 16 (one workgroup per CU at four blocks: 148 VGPRs), among
            // the block counts whose grid meets that floor, the one with the
            // least rounds x (T + 1) (a workgroup's time: T blocks of weights
            // and one x split as costly as one block): [2048,2048] at m = 160
            // takes two blocks (640 workgroups, 21.6 us) over four (320: a
            // second round a quarter full, 24.9 us).  At MC = 4 and 8, where
            // several workgroups share a CU, the most blocks that meet it.
            const int tenv = env_int("DMC_HIP_RD_R16_TILES", 0);
            const int want = tenv == 1 || tenv == 2 || tenv == 4 ? tenv : mp.mt == 16 ? 4 : 2;
            const int64_t blocks16 = (p.n + 15) / 16;
            const int mwenv = env_int("DMC_HIP_RD_R16_MIN_WG_PER_CU", -1);
            const int64_t min_wg = mwenv >= 0 ? (int64_t)mwenv * cus : mp.mt == 16 ? cus * 7 / 8 : cus;
            int tiles = 1;
            double best = -1;
            for (int t = want; t >= 1; t >>= 1) {  // ties keep the larger T
                const int64_t wg = (blocks16 + t - 1) / t * gy;
                if (t > 1 && wg < min_wg) continue;
                if (mp.mt < 16) {
                    tiles = t;
                    break;
                }
                const double cost = (double)((wg + cus - 1) / cus) * (t + 1);
                if (best < 0 || cost < best) best = cost, tiles = t;
            }
            // Where the grid would take fewer blocks per workgroup than wanted
            // (C2 down: 256 16-row blocks), keep them (at MC = 16, four) and
            // split k instead, into the fewest slices that fill the grid: the
            // x bytes per weight byte stay those of the wanted blocks, and a
            // slice-sum launch (gemm_sum_slices_kernel, which settles zeros)
            // follows.  Measured on C2 down: m = 3 / 4 / 6 / 8, 22.9 / 23.1 /
            // 28.6 / 27.9 us -> 22.0 / 22.0 / 23.9 / 23.9 on two blocks and two
            // slices; m = 12 / 16, 26.7 / 27.7 us on four blocks and four slices
            // (27.8 / 30.3 on two and two, 30.6 / 31.8 on the gemm layout).  On
            // a matrix of 32 MiB (C1) the extra launch costs more than the
            // bytes save (8.3-10.3 us -> 10.9-11.7), so only from 64 MiB of
            // weights; and each slice keeps >= 48 lines of 64 k (C2 up, 64
            // lines: four blocks on two or four slices ran 26-39 us against
            // 21-29 on two blocks and one).
            const int64_t nl = p.k / 64;
            const int ksenv = env_int("DMC_HIP_RD_R16_SPLIT", -1);  // k slices; 0 or 1: never split
            const int st = want;
            int ks = ksenv;
            if (ks < 0)
                for (ks = 2; ks < 8 && (blocks16 + st - 1) / st * gy * ks < min_wg;) ks *= 2;
            if (tiles < want && ks >= 2 && ks <= 8 && nl >= (ksenv < 0 ? 48 : 1) * ks &&
                wbytes >= ((int64_t)64 << 20) && (blocks16 + st - 1) / st * gy * ks >= min_wg) {
                tiles = st;
                mp.kchunks = (int)((nl + ks - 1) / ks);
                mp.kslices = (int)((nl + mp.kchunks - 1) / mp.kchunks);
                mp.workspace_bytes = (size_t)mp.kslices * p.m * p.n * 4;
            }
            mp.rpw = 16 * tiles;
        }
        mp.grid_x = (p.n + mp.rpw - 1) / mp.rpw;
        mp.grid_y = (p.m + mp.mt - 1) / mp.mt;
        return mp;
    }

    // Streaming kernel: packed 128-bit rows and k within the register budget.
    if (pl.vec == 8 && p.ldw == p.k && p.ldx == p.k && p.ldy == p.n) {
        RdPlan sp{};
        if (plan_stream(p.m, p.k, &p.n, 1, cus, sp)) {
            // Long rows at M = 1 (2 to 4 windows per lane): workgroups of 16
            // rows that share one LDS copy of x.  One fills a CU, so only when
            // they come in whole rounds of one per CU (or enough rounds that
            // a partial last one costs little): C5's N = 4097 would leave a
            // 257th workgroup to start after the others (17.3 us against 15.7
            // on 8-wave workgroups).  K up to 14336 takes one group of 14
            // waves splitting k (every load carries data at K = 14336: C2 down
            // 19.10 -> 18.97 us, same box), longer rows two 8-wave halves
            // (DMC_HIP_RD_X14=0 keeps the halves everywhere).
            const int64_t g16 = (p.n + 15) / 16;
            const int xl = env_int("DMC_HIP_RD_XLDS", 1);  // 0: never; 2: wherever the kernel applies
            const bool x14 = env_int("DMC_HIP_RD_X14", 1) != 0 && p.k <= kX14MaxK;
            // Two activation rows on the 14-wave group too: the 8-wave
            // streaming kernel would hold 4 windows of both rows' x in
            // registers, one weight row per buffer.
            const bool x14_m2 = p.m == 2 && sp.mt == 2 && sp.waves == 8 && sp.kvec >= 2 && sp.kvec <= 4 &&
                                env_int("DMC_HIP_RD_X14_M2", 1) != 0;
            // (DMC_HIP_RD_ROWS names the 8-wave kernel's rows per step: set, it
            // keeps that kernel at M = 1.)
            const bool rows_auto = env_int("DMC_HIP_RD_ROWS", 0) == 0;
            if ((p.m == 1 ? sp.waves == 8 && sp.kvec >= (xl == 2 ? 1 : 2) && sp.kvec <= 4 && rows_auto : x14_m2) &&
                p.k <= kXldsMaxK && (xl == 2 || (g16 >= cus && (g16 % cus == 0 || g16 >= 4 * cus))) && xl != 0 &&
                x14) {
                sp.waves = kX14Waves;
                sp.kvec = (int)((p.k + kX14Waves * 512 - 1) / (kX14Waves * 512));
                sp.rows = 4;
                sp.rpw = 16;
                sp.mt = (int)p.m;
                sp.grid_x = (p.n + 15) / 16;
                sp.grid_y = 1;
            } else if (p.m == 1 && sp.waves == 8 && sp.kvec >= (xl == 2 ? 1 : 2) && sp.kvec <= 4 && rows_auto &&
                       p.k <= kXldsMaxK && (xl == 2 || (g16 >= cus && (g16 % cus == 0 || g16 >= 4 * cus))) &&
                       xl != 0) {
                int rpw = env_int("DMC_HIP_RD_XLDS_RPW", 16);
                if (rpw != 8 && rpw != 16 && rpw != 32) rpw = 16;
                sp.waves = 16;
                sp.rows = 2;  // the halves walk their rows 2 at a time
                sp.rpw = rpw;
                sp.grid_x = (p.n + rpw - 1) / rpw;
            }
            // A last block of windows holding 1..8 elements (k = 4104) costs
            // the streaming kernel a whole extra block of loads; the unaligned
            // kernel's short tail reads them element by element (W[11008, 4104]:
            // 17.5 us streaming, W[11008, 4100] 15.8 us with the short tail).
            RdPlan up{};
            if (p.m == 1 && plan_unaligned(p, pl.vec, cus, up) && up.kmain < p.k) return up;
            return sp;
        }
    }

    if (pl.vec < 8) {
        RdPlan up{};
        if (plan_unaligned(p, pl.vec, cus, up)) return up;
    }

    // General kernel.
    pl.mt = mt_for(p.m);
    // Rows per workgroup: 4 keeps >= 4 workgroups per CU at the decode
    // shapes (N = 4096 .. 128256) with 8 KiB of weight loads in flight per
    // wave; skinny tiles trade rows for activation registers.
    int rows = pl.mt == 1 ? 4 : (pl.mt <= 4 ? 2 : 1);
    const int64_t min_groups = 2 * cus;
    while (rows > 1 && (p.n + rows - 1) / rows < min_groups) rows >>= 1;
    pl.rows = rows;
    pl.waves = kWaves;
    pl.kvec = 0;
    pl.rpw = rows;
    pl.grid_x = (p.n + rows - 1) / rows;
    pl.grid_y = (p.m + pl.mt - 1) / pl.mt;
    return pl;
}

RdPlan plan_rd_group(const RdGroup &g, int num_cus) {
    RdPlan pl{};
    if (g.count < 1 || g.count > kMaxGroup || g.k % 8 != 0) return pl;
    for (int i = 0; i < g.count; ++i)
        if (!aligned(g.w[i], 16) || !aligned(g.x[i], 32) || g.n[i] < 0) return pl;
    RdPlan sp{};
    if (plan_stream(g.m, g.k, g.n, g.count, num_cus > 0 ? num_cus : 256, sp)) return sp;
    return pl;
}

CsPlan plan_cs(const CsProblem &p, int num_cus) {
    CsPlan pl{};
    for (int v : {8, 4, 2, 1}) {
        if (p.n % v == 0 && (p.batch <= 1 || p.rs % v == 0) && aligned(p.w, 2 * v)) {
            pl.vec = v;
            break;
        }
    }
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    const int64_t batch = std::max<int64_t>(p.batch, 1);
    const int64_t kmax = std::max<int64_t>(p.k, 1);

    // Streaming kernel: 128-bit column vectors; rows at any 2-byte alignment
    // (UN: the matrix's last row goes to the slice pass) from N = 8 and K = 2.
    const bool un = pl.vec < 8 && p.n >= 8 && p.k >= 2 && env_int("DMC_HIP_CS_UNALIGNED", 1) != 0;
    if ((pl.vec == 8 || un) && env_int("DMC_HIP_CS_STREAM", 1) != 0) {
        int nw = env_int("DMC_HIP_CS_WAVES", 4);
        if (nw != 2 && nw != 4 && nw != 8) nw = 4;
        pl.stream = true;
        pl.unaligned = un;
        pl.waves = nw;
        pl.rw = 0;
        pl.mt = std::min(mt_for(p.m), 4);
        // Row groups per wave: 512/G columns per workgroup, as few as still
        // cover N (N = 128: 4 groups of 16 lanes), on aligned rows with 4
        // waves.  Batched per-head W [32,4096,128], one broadcast x: 12.5 us
        // with one group (three quarters of the lanes past N).
        int g = 1;
        if (!un && nw == 4) {
            const int genv = env_int("DMC_HIP_CS_ROW_GROUPS", 0);
            if (genv == 1 || genv == 2 || genv == 4 || genv == 8)
                g = genv;
            else
                while (g < 8 && (int64_t)(kCsCols / (2 * g)) >= p.n) g *= 2;
        }
        pl.rw = g > 1 ? g : 0;  // 0: one group (the plan's long-standing value)
        pl.cb = kCsCols / g;
        pl.grid_x = (p.n + pl.cb - 1) / pl.cb;
        // Split k so the launch has ~4 workgroups per CU; 2 with at most 16
        // column blocks, 3 with at most 24 (env-tunable); each wave with at
        // least 8 rows.  Measured with one activation row (shapes as the
        // logical [N,K]): C2 down [4096,14336] (8 column blocks) 21.2 us at 2
        // per CU against 22.3 at 4, C1 9.4 against 10.9, C5 [4097,11008]
        // (9 blocks) 23.0-23.4 against 24.0-24.1; C5 [11008,4097] (22
        // blocks) 18.2 at 3 against 19.6 at 4; C2 up (28 blocks) 22.5 at 4
        // against 24.9 at 3.
        const int64_t groups = pl.grid_x * std::min<int64_t>(batch, 32768) * ((p.m + pl.mt - 1) / pl.mt);
        const int gpc = pl.grid_x <= 16 ? 2 : pl.grid_x <= 24 ? 3 : 4;
        const int64_t target = (int64_t)env_int("DMC_HIP_CS_GROUPS_PER_CU", gpc) * cus;
        // No split where the column blocks alone give every CU a workgroup:
        // the slice pass's launch costs more than the balance it buys
        // (per-head x, W [32,128,4096]: 10.1 us on 2 slices, 7.2 on one).
        // Row groups (narrow N) keep >= 128 k rows per slice (k/v heads
        // W [8,4096,128]: 6.9 us on 64 slices of 64 rows, 6.6 on 32).
        const int64_t want = groups >= cus ? 1 : std::max<int64_t>(1, (target + groups - 1) / groups);
        const int64_t krows = un ? kmax - 1 : kmax;  // rows the streaming kernel covers
        int64_t kslice = (krows + want - 1) / want;
        kslice = std::max<int64_t>(kslice, g > 1 ? 128 : 8 * nw);
        kslice = (kslice + nw - 1) / nw * nw;
        kslice = std::max<int64_t>(nw, env_int("DMC_HIP_CS_KSLICE", (int)std::min<int64_t>(kslice, INT32_MAX)));
        pl.kslice = kslice;
        pl.slices = (krows + kslice - 1) / kslice;
        // A wave's rows, plus the 16 rows its last loads run past them, must
        // fit a 31-bit buffer offset; the grid's y extent is limited to 65535.
        const int64_t per_wave = (kslice + nw - 1) / nw;
        if (pl.slices <= 65535 && (per_wave + 16 * g) * p.n * 2 <= INT32_MAX) {
            pl.workspace_bytes = pl.slices > 1 || un ? (size_t)pl.slices * batch * p.m * p.n * 4 : 0;
            return pl;
        }
        const int vec = pl.vec;
        pl = CsPlan{};
        pl.vec = vec;
    }

    // General kernel with a second summation pass.
    pl.stream = false;
    pl.waves = kWaves;
    pl.rw = pl.vec == 8 ? 4 : 1;
    const int rw = env_int("DMC_HIP_CS_RW", pl.rw);
    if (pl.vec == 8 && (rw == 1 || rw == 4)) pl.rw = rw;
    pl.mt = mt_for(p.m);
    pl.cb = (64 / pl.rw) * pl.vec;
    pl.grid_x = (p.n + pl.cb - 1) / pl.cb;
    // Split k so the launch has ~8 workgroups per CU, with at least 64 k rows
    // per workgroup (a multiple of the 4*RW rows one workgroup step covers).
    const int64_t step = (int64_t)kWaves * pl.rw;
    const int64_t groups = pl.grid_x * batch;
    int64_t want = (8 * cus + groups - 1) / groups;
    int64_t kslice = (kmax + want - 1) / want;
    kslice = std::max<int64_t>(kslice, 64);
    kslice = (kslice + step - 1) / step * step;
    pl.kslice = kslice;
    pl.slices = (kmax + kslice - 1) / kslice;
    if (pl.slices > 65535) {  // grid.y limit
        pl.slices = 65535;
        pl.kslice = (kmax + pl.slices - 1) / pl.slices;
        pl.kslice = (pl.kslice + step - 1) / step * step;
        pl.slices = (kmax + pl.kslice - 1) / pl.kslice;
    }
    pl.workspace_bytes = pl.slices > 1 ? (size_t)pl.slices * batch * p.m * p.n * 4 : 0;
    return pl;
}

hipError_t launch_rd_group(const RdGroup &g, const RdPlan &pl, hipStream_t s) {
    if (g.m <= 0 || g.count <= 0) return hipSuccess;
    if (pl.kvec <= 0 || g.count > kMaxGroup) return hipErrorInvalidValue;
    RdGroupArgs ga{};
    int64_t acc = 0;
    for (int i = 0; i < g.count; ++i) {
        ga.w[i] = g.w[i];
        ga.x[i] = g.x[i];
        ga.y[i] = g.y[i];
        ga.n[i] = (int)g.n[i];
        ga.gstart[i] = (int)acc;
        acc += (g.n[i] + pl.rpw - 1) / pl.rpw;
    }
    ga.gstart[g.count] = (int)acc;
    for (int i = g.count + 1; i <= kMaxGroup; ++i) ga.gstart[i] = INT32_MAX;
    ga.count = g.count;
    if (acc == 0) return hipSuccess;
    return rs_dispatch(ga, g, pl, s);
}

unsigned stride_grid(int64_t work_items);

hipError_t launch_rd(const RdProblem &p, const RdPlan &pl, void *workspace, hipStream_t s) {
    if (p.m <= 0 || p.n <= 0) return hipSuccess;
    if (pl.mfma) {
        const dim3 grid((unsigned)pl.grid_x, (unsigned)pl.grid_y);
        if (pl.mkind == 6) {
            hipLaunchKernelGGL(gemv_rd_mfma_wide_kernel, grid, dim3(512), 0, s, p.w, p.x, p.y, (int)p.n, (int)p.k,
                               (int)p.m);
            return hipGetLastError();
        }
        if (pl.mkind == 8) {
            // The workspace holds x's planes (unless the kernel splits x
            // itself) and the slice partials (when k is split): a fused
            // single-slice plan needs none and may be given none.
            const bool needs_ws = !pl.xfuse || pl.kslices > 1;
            if ((needs_ws && !workspace) || (pl.mt != 16 && pl.mt != 32 && pl.mt != 64) || pl.kslices < 1 ||
                pl.kslices > 65535 || (int64_t)pl.kslices * pl.kchunks < p.k / 64 || pl.rpw != 32 * pl.waves)
                return hipErrorInvalidValue;
            uint16_t *xs = pl.xfuse ? nullptr : static_cast<uint16_t *>(workspace);
            const size_t planes = pl.xfuse ? 0 : ((size_t)3 * p.m * p.k * 2 + 255) / 256 * 256;
            float *part = pl.kslices > 1 ? reinterpret_cast<float *>(static_cast<char *>(workspace) + planes) : nullptr;
            const int64_t count = p.m * p.k;
            if (!pl.xfuse)
                hipLaunchKernelGGL(split_x_planes_kernel, dim3(stride_grid((count / 8 + 255) / 256)), dim3(256), 0,
                                   s, p.x, xs, count);
            const int64_t wgs = pl.grid_x * pl.grid_y * (int64_t)pl.kslices;
            if (wgs > INT32_MAX) return hipErrorInvalidValue;
            // The XCD-grouped tile order where activation tiles share weight
            // blocks (DMC_HIP_GEMM_XCD: 0 never, 2 always).
            const int xenv = env_int("DMC_HIP_GEMM_XCD", 1);
            const int xcd = xenv == 2 || (xenv == 1 && pl.grid_y > 1) ? 1 : 0;
#define DMC_GEMM(MB, F, NW)                                                                                  \
    if (pl.mt == 16 * MB && pl.xfuse == F && pl.waves == NW)                                                 \
        hipLaunchKernelGGL((gemv_rd_mfma_gemm_kernel<MB, F, NW>), dim3((unsigned)wgs), dim3(64 * NW), 0, s, p.w,  \
                           p.x, xs, p.y, part, (int)p.n, (int)p.k, (int)p.m, pl.kchunks, (int)pl.grid_x,          \
                           (int)pl.grid_y, xcd);                                                              \
    else
            DMC_GEMM(1, true, 8) DMC_GEMM(1, false, 8) DMC_GEMM(2, false, 8) DMC_GEMM(4, false, 8)
            DMC_GEMM(2, false, 4) DMC_GEMM(4, false, 4) DMC_GEMM(2, true, 8) DMC_GEMM(4, true, 8)
            DMC_GEMM(2, true, 4) DMC_GEMM(4, true, 4) return hipErrorInvalidValue;
#undef DMC_GEMM
            if (pl.kslices > 1)
                hipLaunchKernelGGL(gemm_sum_slices_kernel, dim3(stride_grid((p.m * p.n + 255) / 256)), dim3(256), 0,
                                   s, part, pl.kslices, p.y, p.w, p.x, (int)p.m, (int)p.n, (int)p.k);
            return hipGetLastError();
        }
        if (pl.mkind == 7) {
            const int tiles = pl.rpw / 16;
            const int ks = pl.kslices;
            const int lpk = ks > 1 ? pl.kchunks : (int)(p.k / 64);
            if (ks < 1 || ks > 8 || (ks > 1 && (!workspace || lpk < 1 || (int64_t)ks * lpk < p.k / 64)))
                return hipErrorInvalidValue;
            float *part = ks > 1 ? static_cast<float *>(workspace) : nullptr;
            const dim3 grid3((unsigned)pl.grid_x, (unsigned)pl.grid_y, (unsigned)ks);
#define DMC_R16(MC, T)                                                                                       \
    if (pl.mt == MC && tiles == T) {                                                                         \
        hipLaunchKernelGGL((gemv_rd_mfma_rows16_kernel<MC, T>), grid3, dim3(512), 0, s, p.w, p.x, p.y, (int)p.n, \
                           (int)p.k, (int)p.m, lpk, part);                                                   \
    } else
            DMC_R16(4, 1) DMC_R16(4, 2) DMC_R16(4, 4) DMC_R16(8, 1) DMC_R16(8, 2) DMC_R16(8, 4)
            DMC_R16(16, 1) DMC_R16(16, 2) DMC_R16(16, 4) return hipErrorInvalidValue;
#undef DMC_R16
            if (ks > 1)
                hipLaunchKernelGGL(gemm_sum_slices_kernel, dim3(stride_grid((p.m * p.n + 255) / 256)), dim3(256), 0,
                                   s, part, ks, p.y, p.w, p.x, (int)p.m, (int)p.n, (int)p.k);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    if (pl.kvec > 0 && pl.xreg8 && pl.waves == 8 && pl.rpw != 16) {
        if (p.m < 1 || p.m > 4 || p.m != pl.mt || pl.kvec != 1 || p.k > 8 * 512 || p.k < 1)
            return hipErrorInvalidValue;
#define DMC_X8R(R, Q)                                                                                         \
    do switch ((int)p.m) {                                                                                    \
    case 1: hipLaunchKernelGGL((gemv_rd_stream_x8r_kernel<R, Q, 1>), dim3((unsigned)pl.grid_x), dim3(512), 0, s, \
                               p.w, p.x, p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1); break;          \
    case 2: hipLaunchKernelGGL((gemv_rd_stream_x8r_kernel<R, Q, 2>), dim3((unsigned)pl.grid_x), dim3(512), 0, s, \
                               p.w, p.x, p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1); break;          \
    case 3: hipLaunchKernelGGL((gemv_rd_stream_x8r_kernel<R, Q, 3>), dim3((unsigned)pl.grid_x), dim3(512), 0, s, \
                               p.w, p.x, p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1); break;          \
    default: hipLaunchKernelGGL((gemv_rd_stream_x8r_kernel<R, Q, 4>), dim3((unsigned)pl.grid_x), dim3(512), 0, \
                               s, p.w, p.x, p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1); break;       \
    } while (0)
        if (pl.rpw == 4 && pl.rows == 4) DMC_X8R(4, 4);
        else if (pl.rpw == 6 && pl.rows == 6) DMC_X8R(6, 6);
        else if (pl.rpw == 7 && pl.rows == 7) DMC_X8R(7, 7);
        else if (pl.rpw == 8 && pl.rows == 8) DMC_X8R(8, 8);
        else if (pl.rpw == 10 && pl.rows == 5) DMC_X8R(10, 5);
        else if (pl.rpw == 12 && pl.rows == 6) DMC_X8R(12, 6);
        else if (pl.rpw == 14 && pl.rows == 7) DMC_X8R(14, 7);
        else return hipErrorInvalidValue;
#undef DMC_X8R
        return hipGetLastError();
    }
    if (pl.kvec > 0 && pl.xreg8 && pl.waves == 4) {
        if (pl.rpw != 16 || p.m != pl.mt || p.m < 1 || p.m > kX14MaxM || pl.kvec != 1 || p.k > 4 * 512 || p.k < 1)
            return hipErrorInvalidValue;
#define DMC_X4(MT)                                                                                           \
    hipLaunchKernelGGL((gemv_rd_stream_x4_kernel<MT>), dim3((unsigned)pl.grid_x), dim3(256), 0, s, p.w, p.x,  \
                       p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1)
        switch ((int)p.m) {
        case 1: DMC_X4(1); break;
        case 2: DMC_X4(2); break;
        case 3: DMC_X4(3); break;
        case 4: DMC_X4(4); break;
        default: return hipErrorInvalidValue;
        }
#undef DMC_X4
        return hipGetLastError();
    }
    if (pl.kvec > 0 && pl.xreg8) {
        if (pl.rpw != 16 || p.m != pl.mt || p.m < 1 || p.m > kX14MaxM || pl.kvec != 1 || pl.waves != 8 ||
            p.k > 8 * 512 || p.k < 1)
            return hipErrorInvalidValue;
#define DMC_X8(MT)                                                                                           \
    hipLaunchKernelGGL((gemv_rd_stream_x8_kernel<MT>), dim3((unsigned)pl.grid_x), dim3(512),                 \
                       0, s, p.w, p.x, p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1)
        switch ((int)p.m) {
        case 1: DMC_X8(1); break;
        case 2: DMC_X8(2); break;
        case 3: DMC_X8(3); break;
        case 4: DMC_X8(4); break;
        default: return hipErrorInvalidValue;
        }
#undef DMC_X8
        return hipGetLastError();
    }
    if (pl.kvec > 0 && pl.any_align) return rd_unaligned_dispatch(p, pl, s);
    if (pl.kvec > 0 && pl.waves == kX14Waves && pl.rows == 4) {
        if (pl.rpw != 16 || p.m != pl.mt || p.m < 1 || p.m > kX14MaxM || pl.kvec < 1 || pl.kvec > 2 ||
            (int64_t)pl.kvec * kX14Waves * 512 < p.k || p.k > kX14MaxK || (int64_t)16 * p.k * 2 > INT32_MAX)
            return hipErrorInvalidValue;
#define DMC_X14(KV, MT)                                                                                      \
    hipLaunchKernelGGL((gemv_rd_stream_x14_kernel<uint16_t, KV, MT>), dim3((unsigned)pl.grid_x),               \
                       dim3(64 * kX14Waves), 0, s, p.w, p.x, p.y, (int)p.n, (int)p.k, (int64_t)p.ldy, (int64_t)1)
        switch (pl.kvec * 10 + (int)p.m) {
        case 11: DMC_X14(1, 1); break;
        case 21: DMC_X14(2, 1); break;
        case 12: DMC_X14(1, 2); break;
        case 22: DMC_X14(2, 2); break;
        case 13: DMC_X14(1, 3); break;
        case 23: DMC_X14(2, 3); break;
        case 14: DMC_X14(1, 4); break;
        case 24: DMC_X14(2, 4); break;
        default: return hipErrorInvalidValue;
        }
#undef DMC_X14
        return hipGetLastError();
    }
    if (pl.kvec > 0 && pl.waves == 16) {
        if (pl.rows != 2 || (pl.rpw != 8 && pl.rpw != 16 && pl.rpw != 32) || p.m != 1 || p.k > kXldsMaxK)
            return hipErrorInvalidValue;
#define DMC_XLDS(KV)                                                                                          \
    case KV:                                                                                                  \
        hipLaunchKernelGGL((gemv_rd_stream_xlds_kernel<KV, 2>), dim3((unsigned)pl.grid_x), dim3(1024), 0, s, p.w, \
                           p.x, p.y, (int)p.n, (int)p.k, pl.rpw);                                             \
        return hipGetLastError();
        switch (pl.kvec) { DMC_XLDS(1) DMC_XLDS(2) DMC_XLDS(3) DMC_XLDS(4) }
#undef DMC_XLDS
        return hipErrorInvalidValue;
    }
    if (pl.kvec > 0) {
        RdGroup g{};
        g.w[0] = p.w;
        g.x[0] = p.x;
        g.y[0] = p.y;
        g.n[0] = p.n;
        g.count = 1;
        g.m = p.m;
        g.k = p.k;
        return launch_rd_group(g, pl, s);
    }
    switch (pl.vec) {
    case 8: return rd_rows<8>(p, pl, s);
    case 4: return rd_rows<4>(p, pl, s);
    case 2: return rd_rows<2>(p, pl, s);
    case 1: return rd_rows<1>(p, pl, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_cs(const CsProblem &p, const CsPlan &pl, void *workspace, hipStream_t s) {
    if (p.m <= 0 || p.n <= 0 || p.batch <= 0) return hipSuccess;
    const int64_t zmax_s = 32768;  // grid.z limit, with margin
    if (pl.stream) {
        float *P = pl.slices > 1 || pl.unaligned ? static_cast<float *>(workspace) : nullptr;
        for (int64_t z0 = 0; z0 < p.batch; z0 += zmax_s) {
            const int64_t nz = std::min(zmax_s, p.batch - z0);
            for (int64_t m0 = 0; m0 < p.m; m0 += pl.mt) {
                const int64_t mc = std::min<int64_t>(pl.mt, p.m - m0);
                hipError_t e = css_dispatch(p, pl, P, z0, nz, m0, mc, s);
                if (e != hipSuccess) return e;
            }
        }
        if (pl.slices > 1 || pl.unaligned) {
            const int64_t total = p.m * p.n * p.batch;
            const CsSrc src{p.w, p.x, p.rs, p.ls, p.k, p.n, p.m, pl.unaligned};
            if (pl.slices >= 16)
                hipLaunchKernelGGL(sum_slices_stream_kernel<16>, dim3((unsigned)((total + 63) / 64)), dim3(1024), 0,
                                   s, P, total, (int)pl.slices, p.y, total, src);
            else
                hipLaunchKernelGGL(sum_slices_stream_kernel<4>, dim3((unsigned)((total + 63) / 64)), dim3(256), 0, s,
                                   P, total, (int)pl.slices, p.y, total, src);
            return hipGetLastError();
        }
        return hipSuccess;
    }
    const int64_t per_z = p.m * p.n;
    const int64_t total = per_z * p.batch;
    float *P = pl.slices > 1 ? static_cast<float *>(workspace) : p.y;
    const int64_t p_slice = pl.slices > 1 ? total : 0;
    const int64_t zmax = 32768;  // grid.z limit, with margin
    for (int64_t z0 = 0; z0 < p.batch; z0 += zmax) {
        const int64_t nz = std::min(zmax, p.batch - z0);
        for (int64_t m0 = 0; m0 < p.m; m0 += pl.mt) {
            const int64_t mc = std::min<int64_t>(pl.mt, p.m - m0);
            hipError_t e = cs_dispatch(p, pl, P, p_slice, z0, nz, m0, mc, s);
            if (e != hipSuccess) return e;
        }
    }
    if (pl.slices > 1) {
        const int64_t blocks = (total + kThreads - 1) / kThreads;
        const CsSrc src{p.w, p.x, p.rs, p.ls, p.k, p.n, p.m, false};
        hipLaunchKernelGGL(sum_slices_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, P, p_slice,
                           (int)pl.slices, p.y, total, src);
        return hipGetLastError();
    }
    return hipSuccess;
}

// ---- f32 weights, row-dot ------------------------------------------------------

F32Plan plan_f32(const F32Problem &p, int num_cus) {
    F32Plan pl{};
    const int64_t cus = num_cus > 0 ? num_cus : 256;
    // Two to four activation rows on long rows (4096 < K <= 14336, 16-byte
    // rows, 16-row workgroups in whole rounds of one per CU) that the 8-wave
    // streaming kernel below would take in more than one pass over W: the
    // 14-wave kernel of the bf16 path with 4 f32 weights per window, every
    // activation row's x in registers, W read once.  Same box, 8-wave /
    // 14-wave, us: W[4096,14336] m = 2 / 3 / 4 68.0 / 100.2 / 132.2 against
    // 35.5 / 36.3 / 36.5; [4096,11008] m = 2 53.1 against 29.1; [4096,8192]
    // m = 3 42.0 against 24.7; where one pass suffices the 8-wave kernel is as
    // fast or faster ([4096,8192] m = 1 / 2 23.0 / 23.4 against 25.8 / 26.1;
    // [4096,11008] m = 1 28.3 against 29.1).  DMC_HIP_F32_X14: 0 never, 2
    // wherever the kernel applies.
    {
        const int xf = env_int("DMC_HIP_F32_X14", 1);
        const int64_t g16 = (p.n + 15) / 16;
        const int kv8 = (int)((p.k + 8 * 256 - 1) / (8 * 256));  // the 8-wave kernel's vectors per lane
        const int64_t cap8 = kv8 <= 2 ? 4 : kv8 <= 4 ? 2 : 1;    // ... and its activation rows per pass
        if (xf != 0 && p.m >= 1 && p.m <= kX14MaxM && p.k > (xf == 2 ? 3584 : 4096) && p.k <= kX14MaxK &&
            p.k % 4 == 0 && p.ldw == p.k && p.ldx == p.k && aligned(p.w, 16) && aligned(p.x, 16) &&
            (xf == 2 || (p.m > cap8 && g16 >= cus && (g16 % cus == 0 || g16 >= 4 * cus)))) {
            pl.waves = kX14Waves;
            pl.kvec = (int)((p.k + kX14Waves * 256 - 1) / (kX14Waves * 256));
            pl.rows = p.m <= 2 ? 2 : 1;
            pl.mt = (int)p.m;
            pl.rpw = 16;
            pl.grid_x = g16;
            pl.grid_y = 1;
            return pl;
        }
    }
    // One group of 8 waves for 2048 < K <= 4096 (two windows of 4 weights per
    // lane, x in registers, zeros settled after the stream): at 3 or 4
    // activation rows, and where the 8-wave streaming kernel's last window
    // would be partly empty (K not a multiple of 2048).  Same box, group /
    // streaming, us: W[14336,4096] m = 3 / 4 38.4 / 38.5 against 42.2 / 43.0,
    // [4096,4096] 12.0 / 12.2 against 14.5 / 14.9, [1792,4096] 8.8 / 9.0
    // against 9.7 / 10.0; [8192,3072] m = 1 / 2 / 3 / 4 16.1 / 16.3 / 17.2 /
    // 17.4 against 17.0 / 19.2 / 23.1 / 23.3; at K = 4096 and one or two rows
    // the streaming kernel wins ([14336,4096] 35.9 / 37.3 against 38.8 /
    // 40.3).  DMC_HIP_F32_X8: 0 never, 2 wherever it applies.
    const int xf8 = env_int("DMC_HIP_F32_X8", 1);
    if (xf8 != 0 && p.m >= 1 && p.m <= kX14MaxM && p.k > 2048 && p.k <= 4096 && p.k % 4 == 0 && p.ldw == p.k &&
        p.ldx == p.k && aligned(p.w, 16) && aligned(p.x, 16) &&
        (xf8 == 2 || p.m >= 3 || p.k % 2048 != 0) && env_int("DMC_HIP_F32_STREAM", 1) != 0) {
        pl.waves = 8;
        pl.kvec = 2;
        pl.rows = p.m <= 2 ? 2 : 1;
        pl.mt = (int)p.m;
        pl.rpw = 16;
        pl.grid_x = (p.n + 15) / 16;
        pl.grid_y = 1;
        return pl;
    }
    // Streaming: 16-byte rows, x rows alike, K within 8 vectors of 4 per lane
    // over 8 waves.  Waves as for bf16 by bytes per row (1 KiB per wave per
    // vector); activation rows per workgroup within the register budget; rows
    // per workgroup as for bf16 rows of the same byte length (4, 8 for long
    // rows), fewer while that leaves under 4 (2 for long rows) workgroups per CU.
    if (p.k >= 4 && p.k % 4 == 0 && p.k <= 16384 && p.ldw == p.k && p.ldx == p.k && aligned(p.w, 16) &&
        aligned(p.x, 16) && env_int("DMC_HIP_F32_STREAM", 1) != 0) {
        const int nw = p.k <= 256 ? 1 : p.k <= 512 ? 2 : p.k <= 1024 ? 4 : 8;
        const int kv = (int)((p.k + nw * 256 - 1) / (nw * 256));
        const int mt = std::min(p.m <= 1 ? 1 : p.m <= 2 ? 2 : 4, kv <= 2 ? 4 : kv <= 4 ? 2 : 1);
        const int rows = kv <= 2 ? 2 : 1;
        const int64_t gy = (p.m + mt - 1) / mt;
        int rpw = kv >= 3 ? 8 : 4;
        const int64_t min_blocks = (kv >= 2 ? 2 : 4) * cus;
        while (rpw > rows && (p.n + rpw - 1) / rpw * gy < min_blocks) rpw >>= 1;
        rpw = std::max(rows, rpw / rows * rows);
        const int64_t gx = (p.n + rpw - 1) / rpw;
        if ((int64_t)(rpw + 4 * rows) * p.k * 4 <= INT32_MAX && gy <= 65535 && gx <= INT32_MAX) {
            pl.waves = nw;
            pl.kvec = kv;
            pl.rows = rows;
            pl.mt = mt;
            pl.rpw = rpw;
            pl.grid_x = gx;
            pl.grid_y = gy;
            return pl;
        }
    }
    pl.mt = p.m <= 1 ? 1 : p.m <= 4 ? 4 : 16;
    pl.waves = 4;
    pl.kvec = 0;
    pl.rows = 1;
    pl.rpw = 4;
    pl.grid_x = (p.n + 3) / 4;
    pl.grid_y = (p.m + pl.mt - 1) / pl.mt;
    return pl;
}

namespace {

template <int NW, int KV, int ROWS, int MT>
hipError_t f32s_go(const F32Problem &p, const F32Plan &pl, hipStream_t s) {
    static_assert((MT * KV <= 8 && ROWS * KV <= 8) || KV == 1, "register budget");
    hipLaunchKernelGGL((gemv_rd_f32_stream_kernel<NW, KV, ROWS, MT>), dim3((unsigned)pl.grid_x, (unsigned)pl.grid_y),
                       dim3(64 * NW), 0, s, p.w, p.x, p.y, (int)p.n, (int)p.k, (int)p.m, pl.rpw, p.ys_act,
                       p.ys_row);
    return hipGetLastError();
}

template <int NW, int KV, int ROWS>
hipError_t f32s_mt(const F32Problem &p, const F32Plan &pl, hipStream_t s) {
    switch (pl.mt) {
    case 1: return f32s_go<NW, KV, ROWS, 1>(p, pl, s);
    case 2:
        if constexpr (KV <= 4) return f32s_go<NW, KV, ROWS, 2>(p, pl, s);
        break;
    case 4:
        if constexpr (KV <= 2) return f32s_go<NW, KV, ROWS, 4>(p, pl, s);
        break;
    }
    return hipErrorInvalidValue;
}

template <int MT>
hipError_t f32g_go(const F32Problem &p, const F32Plan &pl, hipStream_t s) {
    hipLaunchKernelGGL((gemv_rd_f32_kernel<MT>), dim3((unsigned)pl.grid_x, (unsigned)pl.grid_y), dim3(256), 0, s,
                       p.w, p.ldw, p.x, p.ldx, p.y, (int)p.n, (int)p.k, (int)p.m, p.ys_act, p.ys_row);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_f32(const F32Problem &p, const F32Plan &pl, hipStream_t s) {
    if (p.m <= 0 || p.n <= 0) return hipSuccess;
    if (p.k < 0 || p.m > INT32_MAX || p.n > INT32_MAX || p.k > INT32_MAX || pl.grid_x < 1 || pl.grid_y < 1 ||
        pl.grid_y > 65535 || pl.grid_x > INT32_MAX || pl.grid_x * pl.rpw < p.n || pl.grid_y * pl.mt < p.m)
        return hipErrorInvalidValue;
    if (pl.kvec == 2 && pl.waves == 8 && pl.rpw == 16) {
        if (pl.mt != p.m || p.m < 1 || p.m > kX14MaxM || p.k > 4096 || p.k < 1 || p.k % 4 != 0 || p.ldw != p.k ||
            p.ldx != p.k || !aligned(p.w, 16) || !aligned(p.x, 16) || pl.grid_x != (p.n + 15) / 16 || pl.grid_y != 1)
            return hipErrorInvalidValue;
#define DMC_F32X8(MT)                                                                                        \
    hipLaunchKernelGGL((gemv_rd_stream_x8f_kernel<MT>), dim3((unsigned)pl.grid_x), dim3(512), 0, s, p.w, p.x, \
                       p.y, (int)p.n, (int)p.k, p.ys_act, p.ys_row)
        switch ((int)p.m) {
        case 1: DMC_F32X8(1); break;
        case 2: DMC_F32X8(2); break;
        case 3: DMC_F32X8(3); break;
        default: DMC_F32X8(4); break;
        }
#undef DMC_F32X8
        return hipGetLastError();
    }
    if (pl.kvec > 0 && pl.waves == kX14Waves) {
        // The 14-wave kernel: 16 rows per workgroup, x straight into registers.
        if (pl.rpw != 16 || pl.mt != p.m || p.m < 1 || p.m > kX14MaxM || pl.kvec < 2 || pl.kvec > 4 ||
            (int64_t)pl.kvec * kX14Waves * 256 < p.k || p.k > kX14MaxK || p.k % 4 != 0 || p.ldw != p.k ||
            p.ldx != p.k || !aligned(p.w, 16) || !aligned(p.x, 16) || pl.grid_x != (p.n + 15) / 16 || pl.grid_y != 1)
            return hipErrorInvalidValue;
#define DMC_F32X14(KV, MT)                                                                                  \
    hipLaunchKernelGGL((gemv_rd_stream_x14_kernel<float, KV, MT>), dim3((unsigned)pl.grid_x),              \
                       dim3(64 * kX14Waves), 0, s, p.w, p.x, p.y, (int)p.n, (int)p.k, p.ys_act, p.ys_row)
        switch (pl.kvec * 10 + (int)p.m) {
        case 21: DMC_F32X14(2, 1); break;
        case 22: DMC_F32X14(2, 2); break;
        case 23: DMC_F32X14(2, 3); break;
        case 24: DMC_F32X14(2, 4); break;
        case 31: DMC_F32X14(3, 1); break;
        case 32: DMC_F32X14(3, 2); break;
        case 33: DMC_F32X14(3, 3); break;
        case 34: DMC_F32X14(3, 4); break;
        case 41: DMC_F32X14(4, 1); break;
        case 42: DMC_F32X14(4, 2); break;
        case 43: DMC_F32X14(4, 3); break;
        case 44: DMC_F32X14(4, 4); break;
        default: return hipErrorInvalidValue;
        }
#undef DMC_F32X14
        return hipGetLastError();
    }
    if (pl.kvec > 0) {
        // The shapes the streaming kernel assumes (plan_f32's conditions).
        if (p.k % 4 != 0 || p.ldw != p.k || p.ldx != p.k || !aligned(p.w, 16) || !aligned(p.x, 16) ||
            (int64_t)pl.kvec * pl.waves * 256 < p.k || pl.rpw < pl.rows || pl.rpw > kMaxRpw ||
            pl.rows != (pl.kvec <= 2 ? 2 : 1) || (int64_t)(pl.rpw + 4 * pl.rows) * p.k * 4 > INT32_MAX)
            return hipErrorInvalidValue;
        if (pl.waves == 8) {
            switch (pl.kvec) {
            case 1: return f32s_mt<8, 1, 2>(p, pl, s);
            case 2: return f32s_mt<8, 2, 2>(p, pl, s);
            case 3: return f32s_mt<8, 3, 1>(p, pl, s);
            case 4: return f32s_mt<8, 4, 1>(p, pl, s);
            case 5: return f32s_mt<8, 5, 1>(p, pl, s);
            case 6: return f32s_mt<8, 6, 1>(p, pl, s);
            case 7: return f32s_mt<8, 7, 1>(p, pl, s);
            case 8: return f32s_mt<8, 8, 1>(p, pl, s);
            }
        } else if (pl.kvec == 1) {
            switch (pl.waves) {
            case 1: return f32s_mt<1, 1, 2>(p, pl, s);
            case 2: return f32s_mt<2, 1, 2>(p, pl, s);
            case 4: return f32s_mt<4, 1, 2>(p, pl, s);
            }
        }
        return hipErrorInvalidValue;
    }
    if (pl.rpw != 4 || (p.k > 0 && (!aligned(p.w, 4) || !aligned(p.x, 4) || p.ldw < p.k || p.ldx < p.k)))
        return hipErrorInvalidValue;
    switch (pl.mt) {
    case 1: return f32g_go<1>(p, pl, s);
    case 4: return f32g_go<4>(p, pl, s);
    case 16: return f32g_go<16>(p, pl, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_transpose_f32(const float *src, float *dst, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const int64_t tiles_c = (cols + kTileF - 1) / kTileF;
    const int64_t ntiles = tiles_c * ((rows + kTileF - 1) / kTileF);
    hipLaunchKernelGGL(transpose_f32_kernel, dim3(stride_grid(ntiles)), dim3(256), 0, s, src, dst, rows, cols, tiles_c,
                       ntiles);
    return hipGetLastError();
}

size_t probe_sink_bytes() { return (size_t)kProbeGroups * 4; }

// Split-k partial sums of dmc_hip_gemv_cs_noalloc live here instead of in
// the library's growable workspace: 32 MiB per GPU, held until the process
// ends.  In host code `scratch` is a stand-in for the symbol, not a device
// address; only noalloc_scratch_resolve's result may reach a kernel.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

size_t noalloc_scratch_bytes() { return kNoAllocScratchBytes; }

hipError_t noalloc_scratch_resolve(void **device_address) {
    *device_address = nullptr;
    return hipGetSymbolAddress(device_address, HIP_SYMBOL(scratch));
}


hipError_t launch_copy_words(void *dst, const void *src, int64_t bytes, hipStream_t s) {
    if (bytes <= 0) return hipSuccess;
    if (bytes % 4 || !aligned(dst, 4) || !aligned(src, 4)) return hipErrorInvalidValue;
    const int64_t words = bytes / 4;
    const bool v4 = aligned(dst, 16) && aligned(src, 16);
    const unsigned groups = (unsigned)std::min<int64_t>(64, std::max<int64_t>(1, (words / (v4 ? 4 : 1) + 255) / 256));
    hipLaunchKernelGGL(copy_words_kernel, dim3(groups), dim3(256), 0, s, static_cast<uint32_t *>(dst),
                       static_cast<const uint32_t *>(src), words, v4);
    return hipGetLastError();
}

hipError_t launch_fill_counter_bf16(uint16_t *dst, int64_t count, int64_t offset, uint64_t key,
                                    const uint16_t *table, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    const uint64_t groups = std::min<uint64_t>(65536, ((uint64_t)count + kThreads - 1) / kThreads);
    hipLaunchKernelGGL(fill_counter_bf16_kernel, dim3((unsigned)groups), dim3(kThreads), 0, s, dst,
                       (uint64_t)count, (uint64_t)offset, key, table);
    return hipGetLastError();
}

// Workgroups for a grid-stride elementwise or tile pass: enough to fill the
// device several times over, no more than the work.
unsigned stride_grid(int64_t work_items) {
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(2048, work_items));
}

hipError_t launch_transpose_bf16(const uint16_t *src, uint16_t *dst, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (rows % 8 == 0 && cols % 8 == 0 && aligned(src, 16) && aligned(dst, 16)) {
        const int64_t tiles_c = (cols + kTile - 1) / kTile;
        const int64_t ntiles = tiles_c * ((rows + kTile - 1) / kTile);
        hipLaunchKernelGGL(transpose_bf16_v8_kernel, dim3(stride_grid(ntiles)), dim3(256), 0, s, src, dst, rows, cols,
                           tiles_c, ntiles);
        return hipGetLastError();
    }
    const unsigned gx = (unsigned)std::min<int64_t>(65535, (cols + kTile - 1) / kTile);
    const unsigned gy = (unsigned)std::min<int64_t>(65535, (rows + kTile - 1) / kTile);
    hipLaunchKernelGGL(transpose_bf16_kernel, dim3(gx, gy), dim3(kThreads), 0, s, src, dst, rows, cols);
    return hipGetLastError();
}

template <bool F16>
hipError_t launch_widen16(const uint16_t *src, float *dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (aligned(src, 16) && aligned(dst, 16))
        hipLaunchKernelGGL((bf16_upconvert_kernel<8, F16>), dim3(stride_grid((n / 8 + 255) / 256)), dim3(256), 0, s,
                           src, dst, n);
    else
        hipLaunchKernelGGL((bf16_upconvert_kernel<1, F16>), dim3(stride_grid((n + 255) / 256)), dim3(256), 0, s, src,
                           dst, n);
    return hipGetLastError();
}

hipError_t launch_bf16_upconvert(const uint16_t *src, float *dst, int64_t n, hipStream_t s) {
    return launch_widen16<false>(src, dst, n, s);
}

hipError_t launch_f16_upconvert(const uint16_t *src, float *dst, int64_t n, hipStream_t s) {
    return launch_widen16<true>(src, dst, n, s);
}

hipError_t launch_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (aligned(src, 16) && aligned(dst, 16))
        hipLaunchKernelGGL(f32_to_bf16_kernel<8>, dim3(stride_grid((n / 8 + 255) / 256)), dim3(256), 0, s, src, dst,
                           n);
    else
        hipLaunchKernelGGL(f32_to_bf16_kernel<1>, dim3(stride_grid((n + 255) / 256)), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}

hipError_t launch_probe_read(const void *src, int64_t bytes, void *sink, hipStream_t s) {
    const uint64_t n16 = (uint64_t)(bytes > 0 ? bytes : 0) / 16;
    // n16 / groups must stay below 2^28 so a workgroup's byte range fits the
    // 32-bit buffer offset.
    if (n16 > ((uint64_t)kProbeGroups << 27)) return hipErrorInvalidValue;
    unsigned groups = (unsigned)std::min<uint64_t>(kProbeGroups, std::max<uint64_t>(1, n16 / 512));
    if (n16 == 0) groups = 256;  // empty launch: the dispatch floor
    hipLaunchKernelGGL(probe_read_kernel, dim3(groups), dim3(kThreads), 0, s,
                       static_cast<const uint8_t *>(src), n16, static_cast<uint32_t *>(sink));
    return hipGetLastError();
}

}  // namespace dmc
