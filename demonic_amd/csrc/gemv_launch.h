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

struct CsProblem {
    const uint16_t *w;  // slice z: w + z*rs, [k, n] row-major
    const float *x;     // slice z: x + z*ls, [m, k] row-major
    float *y;           // slice z: y + z*m*n, [m, n] row-major (contiguous)
    int64_t m, k, n;
    int64_t batch, ls, rs;
};

// Launch shape chosen for a problem; exposed so the host library can report
// and test its planning without a device.
struct RdPlan {
    int vec;    // bf16 elements per lane per weight load (8 = 128-bit loads)
    int rows;   // output rows per workgroup
    int mt;     // activation rows per workgroup (skinny-M tile)
    int64_t grid_x, grid_y;
};

struct CsPlan {
    int vec;        // bf16 columns per lane per load
    int rw;         // k-rows covered by one wave-wide load
    int mt;         // activation rows per workgroup
    int cb;         // output columns per workgroup
    int64_t kslice; // k rows per workgroup (split-K)
    int64_t slices; // number of k slices (1 = no second pass)
    int64_t grid_x;
    size_t workspace_bytes;  // partial sums when slices > 1
};

RdPlan plan_rd(const RdProblem &p, int num_cus);
CsPlan plan_cs(const CsProblem &p, int num_cus);

// Enqueue on `stream`.  `workspace` must hold plan.workspace_bytes when
// plan.slices > 1.  Returns hipSuccess or the launch error.
hipError_t launch_rd(const RdProblem &p, const RdPlan &plan, hipStream_t stream);
hipError_t launch_cs(const CsProblem &p, const CsPlan &plan, void *workspace, hipStream_t stream);

}  // namespace dmc
