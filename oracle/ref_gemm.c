/*
 * oracle/ref_gemm.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the T0-GPU reference's CPU GEMM, its bf16 helpers and its
 * deterministic data generators.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product path (libt0g.so) never links it.
 *
 * The reference is Rust and cannot be built here (no cargo/rustc), so there is
 * no oracle/_ref build: this file restates the algorithm.  Every function names
 * the reference lines it follows (paths relative to the reference repo root).
 *
 * Build flags (see oracle/Makefile): -O2 -ffp-contract=off -fno-fast-math.
 * With contraction off, `acc = acc + a * b` is a rounded fp32 multiply followed
 * by a rounded fp32 add, exactly what the reference's `acc += a * b` does in
 * Rust (which never fuses into FMA).
 *
 * Parity pins (tests/test_oracle.py):
 *   - torch goldens held by the reference (benchmarks/torch_ref/ binaries, copied
 *     as data to tests/golden/torch_ref/) pin the NT orientation and the fp32
 *     result of oracle_gemm_nt_naive;
 *   - the fast variant is checked bit-for-bit against the naive one;
 *   - all-ones inputs give C = K exactly (examples/hello_gemm_gen.rs:72-133);
 *   - small cases are checked against an exact fp64 sum (bf16 products are
 *     exact in fp64) within the fp32 sequential-sum error bound;
 *   - the PRNGs are checked against hand-derived first outputs and their
 *     documented ranges; the bf16 rounding helpers against IEEE tie cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* bf16 helpers                                                             */
/* ------------------------------------------------------------------------ */

/* bf16 -> f32: `f32::from_bits((x as u32) << 16)`
 * (examples/test_gemm_correctness.rs:22-24, src/t0/tile_ir.rs:3210-3212). */
static inline float bf16_to_f32(uint16_t x) {
    uint32_t b = ((uint32_t)x) << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* f32 -> bf16 round-to-nearest-even, no NaN special case:
 * `((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16)` in wrapping u32 arithmetic
 * (examples/test_gemm_correctness.rs:15-20, src/ignis/ops/bf16_matmul.rs:369-371). */
uint16_t oracle_f32_to_bf16_rne(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    uint32_t r = ((b >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((b + r) >> 16);
}

/* f32 -> bf16 truncation: `(val.to_bits() >> 16) as u16`
 * (src/t0/tile_ir.rs:3205-3207, src/t0/tile_boundary_tests.rs:22-24). */
uint16_t oracle_f32_to_bf16_trunc(float x) {
    uint32_t b;
    memcpy(&b, &x, 4);
    return (uint16_t)(b >> 16);
}

float oracle_bf16_to_f32(uint16_t x) { return bf16_to_f32(x); }

void oracle_f32_to_bf16_rne_array(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = oracle_f32_to_bf16_rne(src[i]);
}

void oracle_bf16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = bf16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* Data generators                                                          */
/* ------------------------------------------------------------------------ */

/* xorshift64 uniform [-1,1] -> bf16 RNE
 * (examples/test_gemm_correctness.rs:45-58; same at examples/test_gemm_backward.rs:29-41).
 * f = ((state >> 32) as f32 / u32::MAX as f32) * 2.0 - 1.0, all in f32. */
void oracle_rand_bf16_xorshift(uint16_t *out, size_t n, uint64_t seed) {
    uint64_t s = seed ^ 0xDEADBEEFCAFEBABEull;
    const float denom = (float)UINT32_MAX;
    for (size_t i = 0; i < n; i++) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        float f = ((float)(s >> 32) / denom) * 2.0f - 1.0f;
        out[i] = oracle_f32_to_bf16_rne(f);
    }
}

/* LCG uniform [-0.5,0.5) -> bf16 truncation
 * (src/t0/tile_boundary_tests.rs:42-49):
 * rng = rng*6364136223846793005 + 1442695040888963407 (wrapping);
 * f = ((rng >> 33) as f32 / (1u64 << 31) as f32) - 1.0; bf16_trunc(f * 0.5). */
void oracle_rand_bf16_lcg(uint16_t *out, size_t n, uint64_t seed) {
    uint64_t rng = seed;
    const float denom = (float)(1ull << 31);
    for (size_t i = 0; i < n; i++) {
        rng = rng * 6364136223846793005ull + 1442695040888963407ull;
        float f = ((float)(rng >> 33) / denom) - 1.0f;
        out[i] = oracle_f32_to_bf16_trunc(f * 0.5f);
    }
}

/* LCG pattern generator of the tile GEMM suite (src/t0/test_tile_gemm_suite.rs:17-24):
 * s = s*6364136223846793005 + 1; f = ((((s >> 33) as u32) % 200) as f32 - 100.0) * 0.01;
 * bf16 by truncation. */
void oracle_make_bf16_suite(uint16_t *out, size_t n, uint64_t seed) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) {
        s = s * 6364136223846793005ull + 1ull;
        uint32_t v = (uint32_t)(s >> 33) % 200u;
        float f = ((float)v - 100.0f) * 0.01f;
        out[i] = oracle_f32_to_bf16_trunc(f);
    }
}

/* He-uniform init of Linear (src/ignis/nn/linear.rs:36-43):
 * scale = sqrt(2 / in_features) computed in f64 then cast to f32;
 * rng = 42 (seedable here), LCG as above; u = (rng >> 33) as f32 / 2^31 - 1.0; w = u * scale.
 * Returns f32 weights laid out [in_features, out_features]; the reference's
 * matmul converts them to bf16 with RNE (src/ignis/ops/bf16_matmul.rs:357-384). */
void oracle_linear_init_f32(float *out, size_t in_features, size_t out_features, uint64_t seed) {
    float scale = (float)sqrt(2.0 / (double)in_features);
    uint64_t rng = seed;
    const float denom = (float)(1ull << 31);
    size_t n = in_features * out_features;
    for (size_t i = 0; i < n; i++) {
        rng = rng * 6364136223846793005ull + 1442695040888963407ull;
        float u = (float)(rng >> 33) / denom - 1.0f;
        out[i] = u * scale;
    }
}

/* N(0,1)*sigma -> bf16 RNE.  The reference has no normal generator; this one is
 * this build's own, documented so the bench inputs are reproducible:
 * splitmix64 stream; for each pair, u1 = (x1 >> 11 + 1) * 2^-53 in (0,1],
 * u2 = (x2 >> 11) * 2^-53 in [0,1); Box-Muller in double:
 * r = sqrt(-2 ln u1); z0 = r cos(2 pi u2), z1 = r sin(2 pi u2);
 * value = (float)(z * sigma) then RNE to bf16. */
static inline uint64_t splitmix64_next(uint64_t *st) {
    uint64_t z = (*st += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_randn_bf16(uint16_t *out, size_t n, uint64_t seed, double sigma) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        uint64_t x1 = splitmix64_next(&st), x2 = splitmix64_next(&st);
        double u1 = ((double)(x1 >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(x2 >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = oracle_f32_to_bf16_rne((float)(r * cos(two_pi * u2) * sigma));
        if (i + 1 < n) out[i + 1] = oracle_f32_to_bf16_rne((float)(r * sin(two_pi * u2) * sigma));
    }
}

/* ------------------------------------------------------------------------ */
/* CPU reference GEMM                                                       */
/* ------------------------------------------------------------------------ */

/* Faithful NT GEMM, single thread:
 * Y[M,N] = X[M,K] * WT[N,K]^T; acc = 0.0f; for kk ascending: acc += a * b
 * (examples/test_gemm_correctness.rs:28-42; src/t0/tile_ir.rs:3511-3528;
 *  src/t0/test_tile_gemm_suite.rs:26-35; src/t0/tile_boundary_tests.rs:27-39).
 * Only rows [row_begin, row_end) are computed, so a bounded sample of a large
 * problem can be timed; pass 0, m for the full product. */
void oracle_gemm_nt_naive_rows(const uint16_t *x, const uint16_t *wt, float *y,
                               size_t m, size_t k, size_t n,
                               size_t row_begin, size_t row_end) {
    (void)m;
    for (size_t i = row_begin; i < row_end; i++) {
        for (size_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (size_t kk = 0; kk < k; kk++) {
                float a = bf16_to_f32(x[i * k + kk]);
                float b = bf16_to_f32(wt[j * k + kk]);
                acc = acc + a * b;
            }
            y[i * n + j] = acc;
        }
    }
}

void oracle_gemm_nt_naive(const uint16_t *x, const uint16_t *wt, float *y,
                          size_t m, size_t k, size_t n) {
    oracle_gemm_nt_naive_rows(x, wt, y, m, k, n, 0, m);
}

/* General-layout GEMM with the reference's per-element operation order.
 *   C[i,j] = sum_{p=0..K-1, ascending} A(i,p) * B(p,j), fp32, starting at 0.0f.
 * Layouts (letters give op(A), op(B) as stored):
 *   0 NT: A stored [M][lda>=K],  B stored [N][ldb>=K]   (the reference's native form,
 *         examples/test_gemm_correctness.rs:28-42)
 *   1 NN: A stored [M][lda>=K],  B stored [K][ldb>=N]   (cpu_backward_data,
 *         examples/test_gemm_backward.rs:44-60: dX = dY * W)
 *   2 TN: A stored [K][lda>=M],  B stored [K][ldb>=N]   (cpu_backward_weight,
 *         examples/test_gemm_backward.rs:62-77: dW = dY^T * X)
 *   3 TT: A stored [K][lda>=M],  B stored [N][ldb>=K]
 * Fast and bit-identical to the naive loop: for each output row the fp32
 * accumulators of all columns advance together through p in ascending order,
 * each step one rounded multiply and one rounded add (no FMA), so every C[i,j]
 * sees exactly the same operation sequence as the triple loop.  Rows are split
 * over OpenMP threads (nthreads <= 0: library default).
 * C is written densely [M][ldc]. */
void oracle_gemm(int layout, const uint16_t *a, const uint16_t *b, float *c,
                 size_t m, size_t n, size_t k, size_t lda, size_t ldb, size_t ldc,
                 int nthreads) {
    /* Stage op(B) as fp32 [K][N] and op(A) as fp32 rows on the fly. */
    float *bt = (float *)malloc(sizeof(float) * (k ? k : 1) * (n ? n : 1));
    if (!bt) return;
    int b_kn = (layout == 1 || layout == 2); /* B stored [K][N] */
    for (size_t p = 0; p < k; p++)
        for (size_t j = 0; j < n; j++)
            bt[p * n + j] = bf16_to_f32(b_kn ? b[p * ldb + j] : b[j * ldb + p]);
    int a_mk = (layout == 0 || layout == 1); /* A stored [M][K] */
#ifdef _OPENMP
    int nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#else
    (void)nthreads;
#endif
    for (long long ii = 0; ii < (long long)m; ii++) {
        size_t i = (size_t)ii;
        float *crow = c + i * ldc;
        for (size_t j = 0; j < n; j++) crow[j] = 0.0f;
        for (size_t p = 0; p < k; p++) {
            float av = bf16_to_f32(a_mk ? a[i * lda + p] : a[p * lda + i]);
            const float *brow = bt + p * n;
            for (size_t j = 0; j < n; j++) {
                float prod = av * brow[j];
                crow[j] = crow[j] + prod;
            }
        }
    }
    free(bt);
}

/* Split-K partial product: the same as oracle_gemm restricted to p in
 * [k_begin, k_end), i.e. what one K-slice of the reference's split-K kernel
 * writes into its fp32 plane (src/t0/gemm_gen.rs:728-752). */
void oracle_gemm_krange(int layout, const uint16_t *a, const uint16_t *b, float *c,
                        size_t m, size_t n, size_t lda, size_t ldb, size_t ldc,
                        size_t k_begin, size_t k_end, int nthreads) {
    int a_mk = (layout == 0 || layout == 1);
    int b_kn = (layout == 1 || layout == 2);
    const uint16_t *a_off = a_mk ? a + k_begin : a + k_begin * lda;
    const uint16_t *b_off = b_kn ? b + k_begin * ldb : b + k_begin;
    oracle_gemm(layout, a_off, b_off, c, m, n, k_end - k_begin, lda, ldb, ldc, nthreads);
}

/* Split-K reduction on the host, plane order s = 0..sk-1 starting from 0.0f
 * (examples/test_gemm_correctness.rs:190-207; examples/hello_gemm_gen.rs:109-124). */
void oracle_splitk_reduce(const float *planes, float *y, size_t elems, size_t sk) {
    for (size_t i = 0; i < elems; i++) y[i] = 0.0f;
    for (size_t s = 0; s < sk; s++)
        for (size_t i = 0; i < elems; i++) y[i] = y[i] + planes[s * elems + i];
}

/* Host bf16 transpose A[rows][cols] -> A^T[cols][rows]
 * (examples/test_gemm_backward.rs:79-88). */
void oracle_transpose_bf16(const uint16_t *a, uint16_t *out, size_t rows, size_t cols) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[c * rows + r] = a[r * cols + c];
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
