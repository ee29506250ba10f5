// gemv_launch.h -- host-side launch interface of the gfx950 bf16 GEMV kernels.
//
// Two weight layouts, one numeric contract:
//   RD (row-dot)        W stored [N,K] row-major: y[m,n] = sum_k x[m,k] * w[n,k]
//                       (demoniC `x @ W'` and `W @ x` on an HF/PyTorch-layout weight)
//   CS (column-stream)  W stored [K,N] row-major: y[m,n] = sum_k x[m,k] * w[k,n]
//                       (demoniC `x @ W`, the layout of the reference kernel
//                       compiler/src/jit.rs:29481-29487 and gpu.rs:140-143)
// w is bf16 widened exactly (bits << 16, jit.rs:29225-29227); x, y are f32;
// every product is one fused multiply-add into an f32 accumulator that starts
// at +0.0f.  The k reduction is split across lanes, waves and (CS) workgroups,
// so the result is tolerance-equal to the reference's ascending-k chain, not
// bit-equal; the split is fixed, so repeated calls are bit-identical.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dmc {

struct RdProblem {
    const uint16_t *w;  // [n, ldw] bf16 bits
    int64_t ldw;        // elements between weight rows (>= k)
    const float *x;     // [m, ldx]
    int64_t ldx;        // elements between activation rows (>= k)
    float *y;           // [m, ldy]
    int64_t ldy;        // elements between output rows (>= n)
    int64_t m, k, n;
};

// Padding the library allocates after every resident weight and weight
// region: the any-alignment kernel reads whole dwords, so it may read up to 2
// bytes past a matrix whose last element ends at 2 mod 4 (within the same
// dword, and here within the allocation too).
constexpr int64_t kWeightSlack = 16;

struct CsProblem {
    const uint16_t *w;  // slice z: w + z*rs, [k, n] row-major
    const float *x;     // slice z: x + z*ls, [m, k] row-major
    float *y;           // slice z: y + z*m*n, [m, n] row-major (contiguous)
    int64_t m, k, n;
    int64_t batch, ls, rs;
};

// Launch shape chosen for a problem; exposed so the host library can report
// and test its planning without a device.
//
// Two row-dot kernels:
//   streaming (vec == 8, k <= 32768): the workgroup's `waves` waves split k,
//     each lane keeps its slice of x in registers for the whole workgroup, and
//     the workgroup walks `rpw` consecutive weight rows, `rows` at a time,
//     with the next rows' weights in flight while the current ones are summed;
//   general (any alignment or k): 4 waves split k of `rows` rows, x re-read
//     per chunk.
//   mfma (mfma == true; M >= a threshold, K % 64 == 0, 16-byte rows): bf16
//     MFMA on 16-row weight tiles against x split into three bf16 terms,
//     `rpw` weight rows and 16 activation rows per workgroup.
struct RdPlan {
    bool mfma;  // skinny-M MFMA kernel
    int mkind;  // MFMA layout: 6 = 256 rows per workgroup, weights and x staged through LDS;
                // 7 = 16 rows per workgroup read whole, waves own lines of each window
    int vec;    // bf16 elements per lane per weight load (8 = 128-bit loads)
    int rows;   // weight rows per step (streaming) / per workgroup (general)
    int mt;     // activation rows per workgroup (skinny-M tile)
    int waves;  // waves per workgroup
    int kvec;   // 8-element vectors of k per lane (streaming), 0 = general kernel
    int rpw;    // weight rows per workgroup
    int64_t grid_x, grid_y;
    // gemm layout (mkind 8): k split over `kslices` workgroups of `kchunks`
    // 64-element chunks each; workspace for x's bf16 planes and the partials
    int kslices = 1, kchunks = 0;
    bool xfuse = false;  // gemm layout, 16-row activation tiles: x split inside the kernel (no planes)
    // streaming over misaligned rows: windows cover k < kmain, and the 1..8
    // elements [kmain, k) are each row's short tail (0: kmain = k)
    int64_t kmain = 0;
    // streaming over rows at any 2-byte alignment (any_align): a workgroup's
    // rows are rstep apart (2 when ldw is odd, so that they share one
    // alignment), rstep consecutive workgroups sharing a block of rstep * rpw
    // rows
    bool any_align = false;
    int rstep = 1;
    bool xreg8 = false;  // the 14-wave kernel's layout on `waves` = 8 (K <= 4096) or 4 (K <= 2048)
    size_t workspace_bytes = 0;
};

// Two column-stream kernels:
//   streaming (rw == 0): lanes own 8 columns, a workgroup owns 512 columns
//     and a k slice, `waves` waves split the slice; with `unaligned` (vec < 8:
//     rows at any 2-byte alignment, N >= 8, K >= 2) the slice pass also
//     applies the last k row;
//   general (any N): 4 waves, RW k rows per wave-wide load.
// Either way, when k is split over several workgroups a second launch sums
// the slice partials in slice order.
struct CsPlan {
    int vec;        // bf16 columns per lane per load
    int rw;         // k-rows covered by one wave-wide load (streaming kernel: its row groups, 0 for one)
    int mt;         // activation rows per workgroup
    int cb;         // output columns per workgroup
    int waves;      // waves per workgroup
    bool stream;    // streaming kernel
    bool unaligned; // streaming over rows at any 2-byte alignment (the last k row in the slice pass)
    int64_t kslice; // k rows per workgroup (split-K)
    int64_t slices; // number of k slices (1 = no reduction across workgroups)
    int64_t grid_x;
    size_t workspace_bytes;  // partial sums when slices > 1
};

// Up to kMaxGroup independent row-dot problems that share m and k (and x's
// alignment class), run by one launch of the streaming kernel -- e.g. the
// q/k/v or gate/up projections of one decode step.  All are packed:
// w_g [n_g, k], x_g [m, k], y_g [m, n_g].
constexpr int kMaxGroup = 8;
struct RdGroup {
    const uint16_t *w[kMaxGroup];
    const float *x[kMaxGroup];
    float *y[kMaxGroup];
    int64_t n[kMaxGroup];
    int count;
    int64_t m, k;
};

RdPlan plan_rd(const RdProblem &p, int num_cus);
// Streaming plan for a group; kvec == 0 when the streaming kernel cannot take
// it (the caller then launches the problems one by one).
RdPlan plan_rd_group(const RdGroup &g, int num_cus);
CsPlan plan_cs(const CsProblem &p, int num_cus);

// Enqueue on `stream`.  `workspace` must hold plan.workspace_bytes (row-dot:
// the gemm layout's x planes and partial sums; column-stream: the partial sums
// when plan.slices > 1).  Returns hipSuccess or the launch error.
hipError_t launch_rd(const RdProblem &p, const RdPlan &plan, void *workspace, hipStream_t stream);
hipError_t launch_rd_group(const RdGroup &g, const RdPlan &plan, hipStream_t stream);

hipError_t launch_cs(const CsProblem &p, const CsPlan &plan, void *workspace, hipStream_t stream);

// f32 weights, row-dot (the f32 path of `W @ x`, jit.rs:20806-20831): output
// (activation row a, weight row i) = sum_k x[a, k] * w[i, k], an f32 fma per
// product from +0 as for bf16, stored at y[a * ys_act + i * ys_row] (the
// drop-in writes either orientation of its [m, n] result).
struct F32Problem {
    const float *w;  // [n, ldw]
    int64_t ldw;
    const float *x;  // [m, ldx]
    int64_t ldx;
    float *y;
    int64_t ys_act, ys_row;
    int64_t m, k, n;
};
// Streaming (kvec > 0: 16-byte rows, k <= 16384; the bf16 streaming layout with
// 4 weights per load) or general (kvec == 0: any k and 4-byte alignment, one
// row per wave).
struct F32Plan {
    int waves, kvec, rows, mt, rpw;
    int64_t grid_x, grid_y;
};
F32Plan plan_f32(const F32Problem &p, int num_cus);
hipError_t launch_f32(const F32Problem &p, const F32Plan &plan, hipStream_t stream);
// dst [cols, rows] = src [rows, cols]^T for 4-byte elements.
hipError_t launch_transpose_f32(const float *src, float *dst, int64_t rows, int64_t cols, hipStream_t stream);

// Measurement probe: a read-only nontemporal pass over [src, src+bytes) in
// 16-byte granules (bytes == 0: an empty launch, the dispatch floor).  `sink`
// holds probe_sink_bytes().
size_t probe_sink_bytes();
hipError_t launch_probe_read(const void *src, int64_t bytes, void *sink, hipStream_t stream);

// Copy `bytes` (a multiple of 4, both ends 4-byte aligned) between two
// device-visible ranges with a kernel: the drop-in path's activation upload
// from pinned host memory, and the deferred outputs back to pinned staging;
// a copy-engine transfer delays either by its own scheduling.
hipError_t launch_copy_words(void *dst, const void *src, int64_t bytes, hipStream_t stream);

// The fixed scratch of the no-allocation column-stream entry: a file-scope
// device array of noalloc_scratch_bytes() bytes in gemv_kernels.hip.  Its
// device address differs per GPU; resolve it once per device, with that
// device current, and pass only the resolved address to kernels and copies.
size_t noalloc_scratch_bytes();
hipError_t noalloc_scratch_resolve(void **device_address);

// dst [cols, rows] = src [rows, cols]^T for bf16 bit patterns (weight
// residency in the row-dot layout, dmc_hip_bf16_transpose_2d).
hipError_t launch_transpose_bf16(const uint16_t *src, uint16_t *dst, int64_t rows, int64_t cols, hipStream_t stream);

// dst[i] = widen(src[i]) (bits << 16), and dst[i] = bits(src[i]) >> 16.
hipError_t launch_bf16_upconvert(const uint16_t *src, float *dst, int64_t n, hipStream_t stream);
// dst[i] = the f32 value of the IEEE binary16 pattern src[i], exactly (NaN payloads kept).
hipError_t launch_f16_upconvert(const uint16_t *src, float *dst, int64_t n, hipStream_t stream);
hipError_t launch_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, hipStream_t stream);

// Synthetic weights for measurements: dst[i] = table[h(offset + i) >> 48],
// h(j) = splitmix64(j ^ key), table = 65,536 bf16 bit patterns.
hipError_t launch_fill_counter_bf16(uint16_t *dst, int64_t count, int64_t offset, uint64_t key,
                                    const uint16_t *table, hipStream_t stream);

}  // namespace dmc
