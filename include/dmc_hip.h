/*
 * dmc_hip.h -- C ABI of libdmc_hip, the MI355X (gfx950) bf16 GEMV backend for
 * demoniC's `@` operator.
 *
 * The first block is the drop-in boundary: the exact operator surface of the
 * reference's Metal backend (compiler/src/gpu.rs:400-474), bound by the JIT as
 * `__dmc_matmul_bf16_gpu*` symbols (compiler/src/jit.rs:3064-3072) with SysV
 * i64 signatures (jit.rs:5389-5445).  Pointers are host addresses passed as
 * int64; the weight `r` is bf16 bit patterns (u16), `l` and `out` are f32;
 * all row-major.  Each output is computed on the GPU as the reference's
 * ascending-k fma chain (docs/SPEC.md:1149-1163) up to summation order: the
 * result is tolerance-equal (normwise <= 1e-5), with NaN/+-inf classes and the
 * sign of exact zeros preserved.  This route is a non-deterministic fast path
 * in the sense of docs/SPEC.md:1165-1181: a JIT must never select it inside
 * `@deterministic` (see dmc_hip_gemv_selected).
 *
 * Error behaviour.  The reference entries have no error channel and degrade
 * to a CPU kernel when Metal is absent (gpu.rs:327-332, gpu.rs:483-486).  This
 * library has no CPU arithmetic: a caller asks dmc_hip_available() first (as
 * the reference asks blas_gemm_available(), jit.rs:29359) and keeps its own CPU
 * kernel otherwise.  If a void entry point still meets a device error it
 * prints "dmc_hip: fatal: ..." to stderr and aborts rather than return wrong
 * data.  The int32-returning entries report errors instead (0 = success,
 * negative = DMC_HIP_E*) with a message in dmc_hip_last_error().
 *
 * Threading.  One process-wide context (one device, one HIP stream) guarded by
 * a mutex; calls from several threads serialize.  The reference keeps one
 * context per thread for the same single-threaded decode loop (gpu.rs:186-189).
 */
#ifndef DMC_HIP_H
#define DMC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DMC_HIP_OK 0
#define DMC_HIP_ENODEV (-1)  /* no usable gfx950 device, or disabled       */
#define DMC_HIP_EINVAL (-2)  /* bad argument (negative size, null pointer) */
#define DMC_HIP_ENOMEM (-3)  /* device or pinned allocation failed          */
#define DMC_HIP_EDEVICE (-4) /* a HIP runtime call failed                   */
#define DMC_HIP_EIO (-5)     /* file missing or unreadable, not a valid .npz */

/* ---- drop-in operator surface (compiler/src/gpu.rs) --------------------- */

/* Replaces dmc_matmul_bf16_gpu (gpu.rs:400-409), same ABI as the CPU kernel
 * dmc_matmul_bf16 (jit.rs:29488): out[m,n] = l[m,k] @ bf16(r[k,n]).
 * m == 0 or n == 0 returns without touching out (gpu.rs:402); k == 0 writes
 * +0.0 (jit.rs:29655).  Any m runs on the GPU (the reference sends m != 1 to
 * its CPU kernel, gpu.rs:404-407).  Synchronous: out is written on return,
 * after every deferred call has been materialized. */
void dmc_matmul_bf16_gpu(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n);

/* Replaces dmc_matmul_bf16_gpu_batched (gpu.rs:410-437): `batch` slices; slice
 * z reads l + z*ls f32 ([m,k]), r + z*rs u16 ([k,n]) and writes out + z*m*n
 * f32.  Negative ls/rs, or m, k, n, batch < 0, abort. */
void dmc_matmul_bf16_gpu_batched(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k,
                                 int64_t n, int64_t batch, int64_t ls, int64_t rs);

/* Replaces dmc_matmul_bf16_gpu_batched_deferred (gpu.rs:439-466): same ABI and
 * result as the batched entry, but returns once the work is queued; `out` is
 * written by the next synchronous call or by dmc_matmul_bf16_gpu_flush.  A
 * later call whose l, r or out range overlaps a pending out range flushes
 * first (gpu.rs:491-499).  Inputs are copied before return, so the caller may
 * reuse l at once. */
void dmc_matmul_bf16_gpu_batched_deferred(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k,
                                          int64_t n, int64_t batch, int64_t ls, int64_t rs);

/* Replaces dmc_matmul_bf16_gpu_flush (gpu.rs:468-474): materialize every
 * deferred call.  No-op when nothing is pending or before first use. */
void dmc_matmul_bf16_gpu_flush(void);

/* ---- error-returning forms of the drop-in entries ------------------------ */

/* The five entries above abort the process on a device failure, because the
 * reference's signatures return nothing.  The reference itself degrades to its
 * CPU kernel instead: when device init fails (gpu.rs:327-332, 483-486) and for
 * shapes it does not offload (gpu.rs:404-407, 500-507).  These forms let a
 * caller do the same: identical arguments and results, but a failure returns
 * DMC_HIP_E* (the message in dmc_hip_last_error) and leaves `out` untouched
 * -- the kernel writes pinned staging, which is copied to `out` only once the
 * stream has completed -- so the caller computes that call on its own CPU
 * kernel (dmc_matmul_bf16, jit.rs:29488).  No CPU arithmetic happens in the
 * library.  DMC_HIP_ENOMEM: no device memory for the weight even after the
 * cached resident weights were released (DMC_HIP_RESIDENT_CAP, in bytes, caps
 * resident weights, so this can be forced); DMC_HIP_ENODEV: no device, or
 * DMC_HIP_DISABLE set.  The deferred form queues nothing when it fails.  The
 * flush form returns the failure of materializing pending deferred calls;
 * their outputs are then not written. */
int32_t dmc_matmul_bf16_gpu_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n);
int32_t dmc_matmul_bf16_gpu_t_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n);
int32_t dmc_matmul_bf16_gpu_batched_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n,
                                        int64_t batch, int64_t ls, int64_t rs);
int32_t dmc_matmul_bf16_gpu_batched_deferred_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k,
                                                 int64_t n, int64_t batch, int64_t ls, int64_t rs);
int32_t dmc_matmul_bf16_gpu_flush_try(void);

/* ---- additions for MI355X (no Metal counterpart) ------------------------ */

/* Transposed-RHS form of dmc_matmul_bf16_gpu: r holds W[n,k] row-major (the
 * HF/PyTorch Linear layout), out[m,n] = sum_k l[m,k] * bf16(r[n,k]).  This is
 * demoniC's `x @ W'` without materializing W' (the reference transposes at
 * native width first, jit.rs:19420-19454 and jit.rs:29794-29834) and
 * `W @ x` with x:[k,1] (m = 1).  Same error behaviour and synchronicity. */
void dmc_matmul_bf16_gpu_t(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n);

/* ---- f32 weights: the f32 path of `@` ------------------------------------ */

/* Device route for the reference's f32 matmul on GEMV shapes, same ABI as
 * dmc_matmul_par (jit.rs:29415): out[m,n] = l[m,k] @ r[k,n], all f32
 * row-major, each output the ascending-k fma chain from +0 of scalar_matmul /
 * simd_matmul / matmul_tile (jit.rs:20715-20802, jit.rs:29448-29466), up to
 * summation order as for bf16 (normwise <= 1e-5, NaN/+-inf classes and zero
 * signs kept).  It replaces the single-threaded scalar_matmul that an f32
 * `W @ x` takes (emit_2d_matmul_at, jit.rs:20806-20831: W [m,k] @ x [k,1],
 * n = 1).  Served shapes: n <= 16 (W @ x: l is the weight) and m <= 16
 * (x @ W: r is the weight, run as its transpose); any other shape is
 * DMC_HIP_EINVAL (the void form aborts) -- ask dmc_hip_f32_selected first.
 * The weight side is uploaded on every call, as the reference keeps nothing
 * between f32 calls and either operand may be updated in place; only bytes
 * registered at that address (dmc_hip_register_weight, the caller's promise
 * that they stay unchanged) stay resident, x @ W's as a transpose built once.
 * m == 0 or n == 0 returns without touching
 * out (jit.rs:29419); k == 0 writes +0.0.  Synchronous; pending deferred bf16
 * calls are materialized first.  The _try form returns DMC_HIP_E* with out
 * untouched instead of aborting. */
void dmc_matmul_f32_gpu(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n);
int32_t dmc_matmul_f32_gpu_try(int64_t l, int64_t r, int64_t out, int64_t m, int64_t k, int64_t n);

/* The route predicate for dmc_matmul_f32_gpu, shaped like
 * dmc_hip_gemv_selected: opt-in flag on, outside `@deterministic`, a served
 * shape (m <= 16 or n <= 16) and at least DMC_HIP_MIN_MACS multiply-adds.
 * Pure function; touches no device. */
int32_t dmc_hip_f32_selected(int32_t hip_on, int32_t deterministic_depth, int64_t m, int64_t k, int64_t n);

/* Device-pointer f32 row-dot GEMV: y[m,n] = x[m,k] @ w[n,k]' (w f32, rows
 * the output columns), enqueued on the library stream without waiting. */
int32_t dmc_hip_gemv_f32_rd(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k, int64_t n);

/* Launch plan of the f32 row-dot GEMV (w [n,k], x [m,k]) for tests and
 * reports: out8 = {kvec (0: the general kernel; > 0: the streaming kernel's
 * 4-element vectors per lane), rows per register buffer, activation rows per
 * workgroup, grid_x, grid_y, waves, weight rows per workgroup, 0}. */
int32_t dmc_hip_plan_f32(int64_t x_addr, int64_t w_addr, int64_t m, int64_t k, int64_t n, int64_t *out8);

/* 1 when a gfx950 device is usable (initializing the context on first call),
 * 0 otherwise; DMC_HIP_DISABLE=1 in the environment forces 0.  The analogue
 * of blas_gemm_available() (jit.rs:29359). */
int32_t dmc_hip_available(void);

/* The host-independent half of the route decision, shaped like
 * blas_gemm_selected (jit.rs:29346-29351): opt-in flag on, no enclosing
 * `@deterministic` block, and at least DMC_HIP_MIN_MACS multiply-adds.
 * Pure function; touches no device.  The threshold is measured (bench.py
 * --crossover, m = 1 on an MI355X host): a synchronous drop-in call costs
 * 19-20 us up to k*n = 2^20, the reference's CPU kernel (dmc_matmul_bf16,
 * restated) 20.6 us at k*n = 2^14 and 12.3 us at 2^13, so from 2^14 the
 * device wins at every size.  (The reference's Metal route starts at
 * 4,000,000 k*n, jit.rs:20933, because a Metal dispatch costs ~165 us.) */
#define DMC_HIP_MIN_MACS (1LL << 14)
int32_t dmc_hip_gemv_selected(int32_t hip_on, int32_t deterministic_depth, int64_t m, int64_t k,
                              int64_t n);

/* Message of the last error on this thread ("" if none). */
const char *dmc_hip_last_error(void);

/* Device regions: hipMalloc-backed HBM for Forge/Vault tensors (the reserved
 * device.vault / device.forge of docs/MEMORY.md:631-636).  Addresses are
 * device addresses as int64, 256-byte aligned; 0 means failure. */
int64_t dmc_hip_region_alloc(int64_t bytes);
int32_t dmc_hip_region_free(int64_t dptr);
int32_t dmc_hip_upload(int64_t dst_dev, int64_t src_host, int64_t bytes);   /* synchronous */
int32_t dmc_hip_download(int64_t dst_host, int64_t src_dev, int64_t bytes); /* synchronous */
int32_t dmc_hip_copy_device(int64_t dst_dev, int64_t src_dev, int64_t bytes); /* stream-ordered */

/* Make a host weight resident ahead of its first GEMV (the content-keyed memo
 * of gpu.rs:261-280, filled at load time instead of on first use).  Returns
 * the device address of the resident copy (0 on failure).  The entry is
 * pinned: the residency cap (2048 cached weights, gpu.rs:266), an
 * out-of-memory retry and DMC_HIP_RESIDENT_CAP never free it, so the address
 * stays valid until dmc_hip_release_weights. */
int64_t dmc_hip_register_weight(int64_t host_ptr, int64_t bytes);
/* Drop every resident weight, registered ones included (after materializing
 * deferred work); addresses from dmc_hip_register_weight become invalid. */
int32_t dmc_hip_release_weights(void);
/* Number and total bytes of resident weights. */
int64_t dmc_hip_resident_count(void);
int64_t dmc_hip_resident_bytes(void);

/* Device-pointer GEMVs, enqueued on the library stream without waiting.
 * Column-stream: w [k,n] per slice (slice z at w + z*rs u16, x + z*ls f32,
 * y + z*m*n f32).  Row-dot: w [n,k], x [m,k], y [m,n].  Partial sums of the
 * column-stream split use a library-owned workspace grown on demand. */
int32_t dmc_hip_gemv_cs(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k,
                        int64_t n, int64_t batch, int64_t ls, int64_t rs);
int32_t dmc_hip_gemv_rd(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k,
                        int64_t n);
int32_t dmc_hip_synchronize(void);

/* dmc_hip_gemv_cs for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * No counterpart in the reference.  Same arguments, kernels and results as
 * dmc_hip_gemv_cs, but the split-k partial sums go to a fixed 32 MiB device
 * array owned by the library (one per GPU, held until the process ends), and
 * the call allocates nothing (no hipMalloc, hipFree or allocating library
 * routine).  The library must be set up first (dmc_hip_available()): the
 * call returns DMC_HIP_ENODEV otherwise.  A shape whose partial sums exceed
 * 32 MiB returns DMC_HIP_EINVAL with the sizes in dmc_hip_last_error.  Calls
 * share the array: they are ordered on the library stream, but work that
 * overlaps on one GPU outside that order (a captured graph replayed on
 * another stream while a call runs) races on it.  Nothing in the array needs
 * to start at zero; it keeps the last call's partials. */
int32_t dmc_hip_gemv_cs_noalloc(int64_t x_dev, int64_t w_dev, int64_t y_dev, int64_t m, int64_t k,
                                int64_t n, int64_t batch, int64_t ls, int64_t rs);

/* Grouped row-dot GEMV on device pointers: `count` independent problems
 * y_i[m, n_i] = x_i[m, k] @ bf16(w_i[n_i, k])', all packed and sharing m and
 * k, enqueued as one launch per 8 problems when rows are 16-byte aligned and
 * k <= 32768 (else one launch per problem).  For the projections of one
 * decode step that read the same activation (q/k/v, gate/up).  The MI355X
 * counterpart of the reference's one-dispatch batched projection
 * (gpu.rs:410-437, jit.rs:19897-19956) for weights that are separate tensors
 * rather than one affine-strided array. */
int32_t dmc_hip_gemv_rd_grouped(int64_t count, const int64_t *x_devs, const int64_t *w_devs,
                                const int64_t *y_devs, const int64_t *ns, int64_t m, int64_t k);

/* Launch plan a GEMV would use on this device (or on a 256-CU gfx950 when no
 * device is present), for tests and reports.  out8 receives
 * {vec, rows_or_rw, mt, grid_x, slices, workspace_bytes, waves, rows_per_group}.
 * Row-dot layout: `vec` is the weight rows' alignment in bf16 elements (8 =
 * 16 bytes); `slices` > 0 is a streaming plan with that many 8-element k
 * windows per lane (with vec < 8, the variant that reads misaligned rows with
 * unaligned 128-bit loads), 0 the general kernel, -6 / -7 / -8 the MFMA layouts
 * (wide: 256 rows per workgroup; rows16: 16 rows per block; gemm: 256 rows
 * against 16, 32 or 64 activation rows, k possibly split; mt activation rows);
 * waves and rows_per_group (weight rows per workgroup) describe the workgroup.
 * Column-stream layout: `vec` is the row alignment as above; rows_or_rw <= 0 is
 * the streaming kernel (512 columns per workgroup, or with -G row groups per
 * wave 512/G, rows_per_group k rows per slice; with vec < 8 it reads
 * misaligned rows and the slice pass applies the last k row), > 0 the
 * general kernel's k rows per wave-wide load
 * (rows_per_group columns per workgroup); `slices` k slices, summed by a
 * second launch into `workspace_bytes` of partials. */
int32_t dmc_hip_plan(int32_t layout_rd, int64_t x_addr, int64_t w_addr, int64_t m, int64_t k,
                     int64_t n, int64_t batch, int64_t rs, int64_t *out8);

/* Measurement probe for reports: enqueue a read-only pass over the device
 * range [src_dev, src_dev + bytes) with the same nontemporal 128-bit loads
 * the GEMV kernels use (the stream-read ceiling of the GEMV's weight
 * traffic); bytes == 0 enqueues an empty launch (the dispatch floor).  No
 * reference counterpart: it reproduces nothing in demoniC and exists so a
 * report can state a GEMV's bandwidth as a fraction of what a pure read
 * reaches on the same device. */
int32_t dmc_hip_probe_read(int64_t src_dev, int64_t bytes);

/* Synthetic weights for measurements, generated in HBM: dst[i] (u16, i <
 * count) = table[splitmix64((offset + i) ^ key) >> 48], `table` being 65,536
 * bf16 bit patterns on the device.  Integer-only, so a host regenerates any
 * element bit for bit (the 14 GB decode sweep cannot be generated on the
 * host in reasonable time).  No reference counterpart. */
int32_t dmc_hip_fill_counter_bf16(int64_t dst_dev, int64_t count, int64_t offset, uint64_t key,
                                  int64_t table_dev);

/* Device forms of the reference's bf16 helpers, on device pointers, ordered
 * on the library stream.  Results are bit-exact:
 *   dmc_hip_bf16_upconvert: dst f32[n] = widen(src bf16[n]), bits << 16
 *     (replaces dmc_bf16_upconvert, jit.rs:29760);
 *   dmc_hip_f32_to_bf16: dst bf16[n] = src f32 bits >> 16, truncation
 *     (replaces dmc_f32_to_bf16, jit.rs:29783);
 *   dmc_hip_bf16_transpose_2d: dst [n, m] = src [m, n]^T, bit patterns moved
 *     unchanged (replaces dmc_bf16_transpose_2d, jit.rs:29801).
 * The reference allocates and returns the result; here the caller passes it
 * (for instance a region from dmc_hip_region_alloc), and the ranges must not
 * overlap.  n == 0 (or m == 0) does nothing. */
int32_t dmc_hip_bf16_upconvert(int64_t src_dev, int64_t dst_dev, int64_t n);
int32_t dmc_hip_f32_to_bf16(int64_t src_dev, int64_t dst_dev, int64_t n);
int32_t dmc_hip_bf16_transpose_2d(int64_t src_dev, int64_t dst_dev, int64_t m, int64_t n);

/* HIP graphs of the library stream.  Between capture_begin and capture_end,
 * device-pointer GEMVs (dmc_hip_gemv_rd, _gemv_rd_grouped, _gemv_cs) are
 * recorded instead of run, provided that any plan whose dmc_hip_plan
 * workspace_bytes > 0 (column-stream split-K partials; row-dot k-slice
 * partials on the rows16 and gemm layouts, or x's bf16 planes) already fits
 * the library workspace, i.e. after one uncaptured call of the same shape;
 * capture_end returns an
 * executable graph (0 on error: an entry that allocates or waits was called
 * while capturing) that graph_launch replays on the library stream.  While
 * any graph is alive, a workspace outgrown by a later call stays allocated
 * (graph_destroy of the last graph frees it), so replays stay valid.  The
 * MI355X form of the reference's pipelined command buffers (gpu.rs:206-219,
 * gpu.rs:539-624): one host call issues a whole decode step. */
int32_t dmc_hip_capture_begin(void);
int64_t dmc_hip_capture_end(void);
int32_t dmc_hip_graph_launch(int64_t exec);
int32_t dmc_hip_graph_destroy(int64_t exec);

/* ---- weight ingress (the loader behind vault.load_npz) ------------------ */

/* Device form of dmc_vault_load_npz (jit.rs:29836-29944), the loader the JIT
 * emits for `vault.load_npz[T, shape](path, key=...)` (jit.rs:12639-12728):
 * array `key` of the NumPy .npz archive at `path` goes straight into a new
 * device region (free it with dmc_hip_region_free) instead of a host Vault
 * buffer.  The reference's rules: the entry is "{key}.npy", else "{key}";
 * the .npy header is skipped (major version 1: 2-byte length at byte 8,
 * otherwise 4-byte) and not checked against the request; numel * elem_bytes
 * bytes of data follow; convert 0 copies them raw (bf16 weights stay 2-byte,
 * the Bf16Tensor route of jit.rs:12673-12676), 1 widens bf16 and 2 widens
 * f16 to f32 (npz_fill, jit.rs:29928-29941; region of numel * 4 bytes,
 * elem_bytes must be 2).  An entry shorter than the request loads what it
 * holds, reports the short count on stderr as the reference does, and the
 * rest of the region is zero.  Stored and deflated entries, ZIP64 archives;
 * the entry's CRC-32 is checked.  16 zero bytes follow the data (the padding
 * of resident weights).  Returns the region's device address, or 0 with the
 * reason in dmc_hip_last_error() (the reference prints it and returns 0). */
int64_t dmc_hip_vault_load_npz(const char *path, const char *key, int64_t numel, int64_t elem_bytes,
                               int64_t convert);

/* Where dmc_hip_vault_load_npz finds `key` in `path`, touching no device:
 * info[0] 1 if the entry is "{key}" rather than "{key}.npy"; [1] compression
 * method (0 stored, 8 deflate); [2] compressed and [3] uncompressed bytes;
 * [4] file offset of the entry's data; [5] .npy major version (-1: not a
 * .npy); [6] offset of the array data in the entry (-1 not a .npy, -2 a
 * header cut short); [7] CRC-32 from the central directory.  Returns
 * DMC_HIP_OK or DMC_HIP_EIO / DMC_HIP_EINVAL. */
int32_t dmc_hip_npz_locate(const char *path, const char *key, int64_t *info);

/* Enqueue dst f32[n] = the IEEE binary16 patterns src[n] widened exactly:
 * f16_bits_to_f32 (jit.rs:29231-29257), the conversion npz_fill applies for
 * convert == 2 (jit.rs:29937), by integer steps so NaN payloads and the
 * signalling bit survive. */
int32_t dmc_hip_f16_upconvert(int64_t src_dev, int64_t dst_dev, int64_t n);

/* HIP events on the library stream, for timing device work. */
int64_t dmc_hip_event_create(void);
int32_t dmc_hip_event_record(int64_t ev);
int32_t dmc_hip_event_synchronize(int64_t ev);
float dmc_hip_event_elapsed_ms(int64_t start, int64_t stop); /* < 0 on error */
int32_t dmc_hip_event_destroy(int64_t ev);

/* Device facts for reports: compute units, and the name (e.g. "gfx950"). */
int32_t dmc_hip_device_cus(void);
const char *dmc_hip_device_arch(void);

#ifdef __cplusplus
}
#endif

#endif /* DMC_HIP_H */
