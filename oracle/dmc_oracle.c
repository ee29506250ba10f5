/*
 * dmc_oracle.c -- CPU restatement of demoniC's bf16 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP product
 * path and the CPU baseline that bench.py times beside it.  Nothing in the
 * product library (demonic_amd/) links, loads or calls it; only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg do.
 *
 * What it restates (all citations are into the reference checkout):
 *   oracle_bf16_to_f32      compiler/src/jit.rs:29223-29227  bf16_bits_to_f32
 *   oracle_f32_to_bf16      compiler/src/jit.rs:29781-29792  dmc_f32_to_bf16 (truncation)
 *   oracle_bf16_transpose   compiler/src/jit.rs:29794-29834  dmc_bf16_transpose_2d
 *   oracle_bf16_upconvert   compiler/src/jit.rs:29754-29776  dmc_bf16_upconvert
 *   oracle_matmul_bf16      compiler/src/jit.rs:29481-29566  dmc_matmul_bf16
 *       + matmul_tile_bf16_cols / matmul_tile_bf16  jit.rs:29647-29681
 *       + bf16_fma_row (scalar x86 arm)             jit.rs:29568-29601
 *       + matmul_threads                            jit.rs:29467-29479
 *   oracle_matmul_bf16_t    the reference's `x @ W'` route: transpose at
 *                           native width (jit.rs:19420-19454) then the kernel
 *                           above (jit.rs:20916-20946)
 *   oracle_gemv_points      the same closed form evaluated for a subset of
 *                           outputs (sampled-row parity at full sizes)
 *   oracle_matmul_f32       compiler/src/jit.rs:29415-29466  dmc_matmul_par / matmul_tile,
 *                           = scalar_matmul / simd_matmul    jit.rs:20525-20802
 *                           (the f32 `@`, jit.rs:20806-20831)
 *   oracle_gemv_points_f32  that closed form for a subset of outputs, W [N,K]
 *
 * The numeric contract (docs/SPEC.md:1149-1163, docs/NUMERICS.md:28-33): each
 * output is acc = +0.0f; for k ascending: acc = fmaf(x[k], w(k), acc).  fmaf
 * is IEEE-754 fusedMultiplyAdd (correctly rounded), so every value below is
 * reproducible bit for bit on any conforming host.  Build without -ffast-math
 * and with -ffp-contract=off so no other expression is contracted.
 *
 * Parity pins (tests/test_oracle.py): widen/truncate/transpose known-answer
 * tests from jit.rs:30171-30178 and jit.rs:30249-30263; the m=3,k=5,n=4 case
 * of jit.rs:30204-30243 and C5-style edge cases against an independent
 * exact-rational fma chain (tests/golden/); the ones KATs of
 * jit.rs:42643-42655 and tools/jit_probes.py:932; the thread-count
 * invariance the reference states at jit.rs:29501-29503; a rigorous forward
 * error bound at the large shape of jit.rs:30016-30030; and planted
 * mutations (oracle_set_mutation) that every pin set must catch.
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define ORACLE_API __attribute__((visibility("default")))

/* ---- planted mistakes, for the tests that show the pins have teeth ------ */
/* 0 = faithful.  Any other value plants one plausible bug in the chain.     */
enum {
    MUT_NONE = 0,
    MUT_DROP_LAST_K = 1,   /* loop stops one k early                         */
    MUT_NEG_ZERO_INIT = 2, /* accumulator seeded with -0.0 instead of +0.0   */
    MUT_UNFUSED = 3,       /* a*b rounded, then added (two roundings)        */
    MUT_TRANSPOSED_W = 4,  /* weight indexed as [N,K] instead of [K,N]       */
    MUT_WIDEN_SHIFT = 5,   /* widen with << 15 instead of << 16              */
    MUT_DESCENDING_K = 6,  /* accumulate k descending                        */
};
#ifdef ORACLE_NO_MUTATION
/* Baseline build: the knob is compiled out so the loops vectorize freely. */
#define g_mutation MUT_NONE
ORACLE_API void oracle_set_mutation(int code) { (void)code; }
ORACLE_API int oracle_get_mutation(void) { return -1; }
#else
static int g_mutation = MUT_NONE;
ORACLE_API void oracle_set_mutation(int code) { g_mutation = code; }
ORACLE_API int oracle_get_mutation(void) { return g_mutation; }
#endif

/* ---- scalar helpers ------------------------------------------------------ */

/* jit.rs:29223-29227: f32::from_bits((h as u32) << 16) -- exact, keeps NaN
 * payloads, signed zeros and subnormals. */
ORACLE_API float oracle_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << (g_mutation == MUT_WIDEN_SHIFT ? 15 : 16);
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* jit.rs:29781-29792: (f32_bits >> 16) -- truncation, the inverse of the
 * widen for bf16-representable values. */
ORACLE_API uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return (uint16_t)(u >> 16);
}

ORACLE_API void oracle_bf16_upconvert(const uint16_t *src, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_bf16_to_f32(src[i]);
}

ORACLE_API void oracle_f32_to_bf16_n(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_bf16(src[i]);
}

/* jit.rs:29801-29834: [m,n] -> [n,m] at native 2-byte width.  The reference
 * blocks by 64 for cache reuse; blocking does not change the result (each
 * element is a plain move), so the same blocking is kept only for speed. */
ORACLE_API void oracle_bf16_transpose(const uint16_t *src, uint16_t *dst, int64_t m, int64_t n) {
    const int64_t B = 64;
    for (int64_t i0 = 0; i0 < m; i0 += B) {
        int64_t i1 = i0 + B < m ? i0 + B : m;
        for (int64_t j0 = 0; j0 < n; j0 += B) {
            int64_t j1 = j0 + B < n ? j0 + B : n;
            for (int64_t i = i0; i < i1; ++i)
                for (int64_t j = j0; j < j1; ++j) dst[j * m + i] = src[i * n + j];
        }
    }
}

static inline float step(float a, float w, float acc) {
    if (g_mutation == MUT_UNFUSED) {
        volatile float p = a * w; /* volatile: force the separate rounding */
        return p + acc;
    }
    return fmaf(a, w, acc);
}

/* jit.rs:29647-29672 (matmul_tile_bf16_cols) with the scalar bf16_fma_row of
 * jit.rs:29594-29599: zero the column range, then one fma row pass per k in
 * ascending order.  k outer / j inner, exactly the reference's loop nest. */
static void tile_bf16_cols(const float *a, const uint16_t *b, float *c, int64_t k, int64_t n,
                           int64_t j0, int64_t j1) {
    if (g_mutation == MUT_NONE) {
        for (int64_t j = j0; j < j1; ++j) c[j] = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) {
            const float av = a[kk];
            const uint16_t *brow = b + kk * n;
            for (int64_t j = j0; j < j1; ++j) {
                uint32_t u = (uint32_t)brow[j] << 16;
                float w;
                memcpy(&w, &u, sizeof w);
                c[j] = fmaf(av, w, c[j]);
            }
        }
        return;
    }
    const float init = g_mutation == MUT_NEG_ZERO_INIT ? -0.0f : 0.0f;
    for (int64_t j = j0; j < j1; ++j) c[j] = init;
    int64_t kend = g_mutation == MUT_DROP_LAST_K && k > 0 ? k - 1 : k;
    for (int64_t t = 0; t < kend; ++t) {
        int64_t kk = g_mutation == MUT_DESCENDING_K ? kend - 1 - t : t;
        const float av = a[kk];
        if (g_mutation == MUT_TRANSPOSED_W) {
            for (int64_t j = j0; j < j1; ++j)
                c[j] = step(av, oracle_bf16_to_f32(b[j * k + kk]), c[j]);
        } else {
            const uint16_t *brow = b + kk * n;
            for (int64_t j = j0; j < j1; ++j) c[j] = step(av, oracle_bf16_to_f32(brow[j]), c[j]);
        }
    }
}

/* jit.rs:29674-29681 */
static void tile_bf16_rows(const float *a, const uint16_t *b, float *c, int64_t k, int64_t n,
                           int64_t i0, int64_t i1) {
    for (int64_t i = i0; i < i1; ++i) tile_bf16_cols(a + i * k, b, c + i * n, k, n, 0, n);
}

/* ---- threading policy ---------------------------------------------------- */

typedef struct {
    const float *a;
    const uint16_t *b;
    float *c;
    int64_t k, n, lo, hi;
    int by_cols;
} job_t;

static void *job_run(void *p) {
    job_t *j = (job_t *)p;
    if (j->by_cols)
        tile_bf16_cols(j->a, j->b, j->c, j->k, j->n, j->lo, j->hi);
    else
        tile_bf16_rows(j->a, j->b, j->c, j->k, j->n, j->lo, j->hi);
    return NULL;
}

/* Run jobs[0..cnt) on cnt threads (the reference's std::thread::scope). */
static void run_jobs(job_t *jobs, int cnt) {
    if (cnt == 1) {
        job_run(&jobs[0]);
        return;
    }
    pthread_t th[64];
    int started[64] = {0};
    for (int i = 0; i < cnt; ++i) started[i] = pthread_create(&th[i], NULL, job_run, &jobs[i]) == 0;
    for (int i = 0; i < cnt; ++i) {
        if (started[i])
            pthread_join(th[i], NULL);
        else
            job_run(&jobs[i]); /* could not spawn: do the band inline */
    }
}

static int env_int(const char *name, int dflt) {
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    return atoi(v);
}

/* jit.rs:29467-29479 (matmul_threads): serial below 2^20 MACs or m < 2; cap
 * from DMC_MATMUL_THREADS else available_parallelism clamped to [1,16]; never
 * more than m. */
ORACLE_API int oracle_matmul_threads(int64_t m, int64_t k, int64_t n) {
    __int128 macs = (__int128)m * k * n;
    if (macs < ((__int128)1 << 20) || m < 2) return 1;
    int cap = env_int("DMC_MATMUL_THREADS", 0);
    if (cap <= 0) {
        long p = sysconf(_SC_NPROCESSORS_ONLN);
        cap = p < 1 ? 1 : (p > 16 ? 16 : (int)p);
    }
    return (int64_t)cap < m ? cap : (int)m;
}

/* jit.rs:29527-29529: m == 1 column split ways by weight bytes (>= 16 MiB ->
 * 4, >= 2 MiB -> 2, else 1); DMC_BF16_COLSPLIT=0 forces serial
 * (jit.rs:29506-29510). */
ORACLE_API int oracle_gemv_ways(int64_t k, int64_t n) {
    const char *v = getenv("DMC_BF16_COLSPLIT");
    if (v && strcmp(v, "0") == 0) return 1;
    int64_t bytes = k * n * 2;
    if (bytes >= (16LL << 20)) return 4;
    if (bytes >= (2LL << 20)) return 2;
    return 1;
}

/* Core of dmc_matmul_bf16 with an explicit worker count (0 = the reference's
 * policy).  A forced count exercises the invariance the reference relies on
 * (jit.rs:29501-29503): outputs are partitioned, never the k reduction. */
ORACLE_API void oracle_matmul_bf16_ex(const float *l, const uint16_t *r, float *out, int64_t m,
                                      int64_t k, int64_t n, int force_workers) {
    if (m <= 0 || n <= 0) return; /* jit.rs:29490 */
    job_t jobs[64];
    if (m == 1) {
        int ways = force_workers > 0 ? force_workers : oracle_gemv_ways(k, n);
        if (ways > 64) ways = 64;
        if (ways <= 1) {
            tile_bf16_rows(l, r, out, k, n, 0, 1);
            return;
        }
        /* jit.rs:29535: 32-column-aligned disjoint chunks */
        int64_t chunk = ((n + ways - 1) / ways + 31) & ~(int64_t)31;
        int cnt = 0;
        for (int64_t j0 = 0; j0 < n; j0 += chunk) {
            int64_t j1 = j0 + chunk < n ? j0 + chunk : n;
            jobs[cnt++] = (job_t){l, r, out, k, n, j0, j1, 1};
        }
        run_jobs(jobs, cnt);
        return;
    }
    int workers = force_workers > 0 ? force_workers : oracle_matmul_threads(m, k, n);
    if (workers > m) workers = (int)m;
    if (workers > 64) workers = 64;
    if (workers <= 1) {
        tile_bf16_rows(l, r, out, k, n, 0, m);
        return;
    }
    int64_t chunk = (m + workers - 1) / workers;
    int cnt = 0;
    for (int64_t i0 = 0; i0 < m; i0 += chunk) {
        int64_t i1 = i0 + chunk < m ? i0 + chunk : m;
        jobs[cnt++] = (job_t){l, r, out, k, n, i0, i1, 0};
    }
    run_jobs(jobs, cnt);
}

/* dmc_matmul_bf16 (jit.rs:29488): C[m,n] = A[m,k] @ bf16(B[k,n]); l f32
 * [m,k], r u16 [k,n], out f32 [m,n], all row-major. */
ORACLE_API void oracle_matmul_bf16(const float *l, const uint16_t *r, float *out, int64_t m,
                                   int64_t k, int64_t n) {
    oracle_matmul_bf16_ex(l, r, out, m, k, n, 0);
}

/* The reference's `x @ W'` with W stored [n,k]: materialize the transpose at
 * native width (dmc_bf16_transpose_2d), then the bf16 kernel.  The transpose
 * buffer is allocated here (the reference takes it from the Forge or its
 * MAT_CACHE; either way the values are the transposed bits). */
ORACLE_API int oracle_matmul_bf16_t(const float *l, const uint16_t *w_nk, float *out, int64_t m,
                                    int64_t k, int64_t n) {
    if (m <= 0 || n <= 0) return 0;
    uint16_t *wt = (uint16_t *)malloc((size_t)(k * n > 0 ? k * n : 1) * sizeof(uint16_t));
    if (!wt) return -1;
    oracle_bf16_transpose(w_nk, wt, n, k); /* [n,k] -> [k,n] */
    oracle_matmul_bf16_ex(l, wt, out, m, k, n, 0);
    free(wt);
    return 0;
}

/* The closed form for a subset of outputs, used to check full-size device
 * results on sampled rows/columns without a full CPU GEMV.
 *   layout 0 (column-stream): w(n,k) = W[k*ldw + n]   (W stored [K,N])
 *   layout 1 (row-dot):       w(n,k) = W[n*ldw + k]   (W stored [N,K])
 * For each requested (mi, ni): acc = +0; for k ascending: fmaf.  Identical
 * per element to oracle_matmul_bf16 (the reference kernel's chain). */
ORACLE_API void oracle_gemv_points(const float *x, int64_t ldx, const uint16_t *w, int64_t ldw,
                                   int layout, int64_t k, const int64_t *mi, const int64_t *ni,
                                   int64_t npts, float *out) {
    const float init = g_mutation == MUT_NEG_ZERO_INIT ? -0.0f : 0.0f;
    for (int64_t p = 0; p < npts; ++p) {
        const float *xr = x + mi[p] * ldx;
        const int64_t n = ni[p];
        float acc = init;
        int64_t kend = g_mutation == MUT_DROP_LAST_K && k > 0 ? k - 1 : k;
        for (int64_t t = 0; t < kend; ++t) {
            int64_t kk = g_mutation == MUT_DESCENDING_K ? kend - 1 - t : t;
            uint16_t h = layout == 0 ? w[kk * ldw + n] : w[n * ldw + kk];
            acc = step(xr[kk], oracle_bf16_to_f32(h), acc);
        }
        out[p] = acc;
    }
}

/* The reference's f32 matmul (dmc_matmul_par's matmul_tile, jit.rs:29448-
 * 29466; bit-identical to the inline scalar_matmul and simd_matmul kernels,
 * jit.rs:29404-29408 and jit.rs:20769-20775): out[m,n] = l[m,k] @ r[k,n], all
 * f32 row-major; per output acc = +0.0f, then acc = fmaf(l[i][kk], r[kk][j],
 * acc) for kk ascending -- matmul_tile's loop nest (row zeroed, kk outer, j
 * inner).  m == 0 or n == 0 returns (jit.rs:29419); k == 0 leaves the zeros.
 * Serial: the reference partitions output rows over threads
 * (jit.rs:29421-29445), which changes no value. */
ORACLE_API void oracle_matmul_f32(const float *l, const float *r, float *out, int64_t m, int64_t k, int64_t n) {
    if (m <= 0 || n <= 0) return;
    const float init = g_mutation == MUT_NEG_ZERO_INIT ? -0.0f : 0.0f;
    const int64_t kend = g_mutation == MUT_DROP_LAST_K && k > 0 ? k - 1 : k;
    for (int64_t i = 0; i < m; ++i) {
        float *c = out + i * n;
        for (int64_t j = 0; j < n; ++j) c[j] = init;
        for (int64_t t = 0; t < kend; ++t) {
            const int64_t kk = g_mutation == MUT_DESCENDING_K ? kend - 1 - t : t;
            const float a = l[i * k + kk];
            for (int64_t j = 0; j < n; ++j) {
                const float b = g_mutation == MUT_TRANSPOSED_W ? r[j * k + kk] : r[kk * n + j];
                c[j] = step(a, b, c[j]);
            }
        }
    }
}

/* The f32 closed form at selected outputs, weight stored [N,K] (row-dot):
 * out[p] = chain over k of x[mi[p]][k] * w[ni[p]][k], from +0, ascending. */
ORACLE_API void oracle_gemv_points_f32(const float *x, int64_t ldx, const float *w, int64_t ldw, int64_t k,
                                       const int64_t *mi, const int64_t *ni, int64_t npts, float *out) {
    const float init = g_mutation == MUT_NEG_ZERO_INIT ? -0.0f : 0.0f;
    const int64_t kend = g_mutation == MUT_DROP_LAST_K && k > 0 ? k - 1 : k;
    for (int64_t p = 0; p < npts; ++p) {
        const float *xr = x + mi[p] * ldx;
        const float *wr = w + ni[p] * ldw;
        float acc = init;
        for (int64_t t = 0; t < kend; ++t) {
            const int64_t kk = g_mutation == MUT_DESCENDING_K ? kend - 1 - t : t;
            acc = step(xr[kk], wr[kk], acc);
        }
        out[p] = acc;
    }
}

/* Batched affine form of the Metal backend's CPU fallback
 * (gpu.rs:366-391, cpu_bf16_gemm_batched): slice z reads x at z*ls f32 and
 * W at z*rs u16, writes n f32 at z*n. */
ORACLE_API void oracle_matmul_bf16_batched(const float *l, const uint16_t *r, float *out,
                                           int64_t k, int64_t n, int64_t batch, int64_t ls,
                                           int64_t rs) {
    for (int64_t z = 0; z < batch; ++z)
        tile_bf16_rows(l + z * ls, r + z * rs, out + z * n, k, n, 0, 1);
}
