/*
 * tg_oracle.c -- CPU restatement of the reference CPU tropical GEMM.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path links, loads or
 * calls this file: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU baseline.
 *
 * What it restates (reference paths are relative to the reference root):
 *
 *  - Semiring identities and scalar ops:
 *      crates/tropical-gemm/src/types/scalar.rs:32-126
 *      (floats: tropical zero -inf/+inf/0, ⊗ = one IEEE add or mul;
 *       integers: tropical zero MIN/MAX/0, ⊗ = two's-complement add/mul,
 *       which wraps in a release build).
 *  - The argmax-carrying ⊕:
 *      types/max_plus.rs:66-73 (keep acc iff acc >= p),
 *      types/min_plus.rs:66-73 (keep acc iff acc <= p),
 *      types/max_mul.rs:65-72  (keep acc iff acc >= p).
 *    Argmax starts at 0 (core/argmax.rs:28) and k is visited in ascending
 *    global order (core/gemm.rs:167-244 with k_offset, core/kernel.rs:145-158).
 *  - The backward scatter loops: api.rs:563-582 (grad_a), api.rs:627-646
 *    (grad_b); MaxMul multiplicative rule: tropical-gemm-python/src/lib.rs:877-950.
 *
 * Two families of functions live here:
 *
 *  1. tgo_gemm_* : the ORACLE.  Row-major C = A (x) B (+ argmax), computed
 *     with the CPU select rule per output in ascending k.  The loop order is
 *     i-k-j (so the j loop vectorises) which visits each output's k in the
 *     same ascending order as the reference's BLIS loops; rows are split over
 *     pthreads.  Results are therefore identical to the reference CPU path
 *     for every non-NaN input (NaN handling also follows the select rule).
 *
 *  2. tgo_portable_argmax_{f32,f64,i32,i64}, tgo_portable_gemm_{i32,i64}, tgo_avx2_gemm_f32 and
 *     tgo_avx2_gemm_maxplus_f64 : the CPU BASELINES used for timing.  Faithful single-thread restatements of the
 *     reference's two CPU paths:
 *       argmax (every dtype): BLIS 5-loop with TilingParams::PORTABLE
 *       (MC=NC=64, KC=256, MR=NR=4; core/tiling.rs:39-45), pack_a/pack_b
 *       (core/packing.rs:46-161) and the 4x4 scalar microkernel with
 *       k_offset (core/kernel.rs:119-167);
 *       value-only f32: the same 5-loop with TilingParams::F32_AVX2 (MC=NC=
 *       256, KC=512, MR=NR=8) and the AVX2 8x8 microkernel
 *       (simd/kernels/avx2.rs), which the reference dispatches to on AVX2 and
 *       AVX-512 hosts alike (simd/dispatch.rs);
 *       value-only MaxPlus f64: the 5-loop with TilingParams::F64_AVX2 (MC=NC=
 *       128, KC=256, MR=NR=4; core/tiling.rs:29-35) and the AVX2 4x4 f64
 *       microkernel (simd/kernels/avx2.rs:77-143; simd/dispatch.rs:86-108).
 *       MinPlus and MaxMul f64 take the portable path there
 *       (simd/dispatch.rs:233-243), so they have no restatement here.
 *     Their results equal the oracle's on ordinary data; they exist so the
 *     timed numbers reflect the reference's algorithms, not the oracle's
 *     vectorised loop.
 *
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -ffp-contract=off, no
 * fast-math, so every float op is the single IEEE op the reference performs).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { TGO_MAXPLUS = 0, TGO_MINPLUS = 1, TGO_MAXMUL = 2 };

/* ------------------------------------------------------------------------ */
/* Scalar semantics per dtype (types/scalar.rs:32-126)                       */
/* ------------------------------------------------------------------------ */

static inline float zero_f32(int sr) {
    return sr == TGO_MAXPLUS ? -INFINITY : (sr == TGO_MINPLUS ? INFINITY : 0.0f);
}
static inline double zero_f64(int sr) {
    return sr == TGO_MAXPLUS ? -INFINITY : (sr == TGO_MINPLUS ? INFINITY : 0.0);
}
static inline int32_t zero_i32(int sr) {
    return sr == TGO_MAXPLUS ? INT32_MIN : (sr == TGO_MINPLUS ? INT32_MAX : 0);
}
static inline int64_t zero_i64(int sr) {
    return sr == TGO_MAXPLUS ? INT64_MIN : (sr == TGO_MINPLUS ? INT64_MAX : 0);
}

/* ⊗: floats use one IEEE op; integers wrap (scalar.rs:94-102, release build). */
static inline float mul_f32(int sr, float a, float b) { return sr == TGO_MAXMUL ? a * b : a + b; }
static inline double mul_f64(int sr, double a, double b) { return sr == TGO_MAXMUL ? a * b : a + b; }
static inline int32_t mul_i32(int sr, int32_t a, int32_t b) {
    uint32_t r = sr == TGO_MAXMUL ? (uint32_t)a * (uint32_t)b : (uint32_t)a + (uint32_t)b;
    return (int32_t)r;
}
static inline int64_t mul_i64(int sr, int64_t a, int64_t b) {
    uint64_t r = sr == TGO_MAXMUL ? (uint64_t)a * (uint64_t)b : (uint64_t)a + (uint64_t)b;
    return (int64_t)r;
}

/* ------------------------------------------------------------------------ */
/* Oracle: threaded i-k-j loop with the CPU select rule                      */
/* ------------------------------------------------------------------------ */

typedef struct {
    int sr;
    const void* A;
    const void* B;
    void* C;
    uint32_t* argmax;
    int64_t M, N, K;
    int64_t row_begin, row_end;
} tgo_job;

/*
 * One macro body per dtype.  For row i: acc[j] = zero, idx[j] = 0; then for
 * k ascending and every j: p = A[i,k] (x) B[k,j]; replace (acc,idx) by (p,k)
 * iff the reference would NOT keep acc, i.e. iff !(acc >= p) for
 * MaxPlus/MaxMul and !(acc <= p) for MinPlus (max_plus.rs:66-73,
 * min_plus.rs:66-73, max_mul.rs:65-72).
 */
#define TGO_ROWS_BODY(T, ZERO, MUL)                                              \
    const T* A = (const T*)job->A;                                               \
    const T* B = (const T*)job->B;                                               \
    T* C = (T*)job->C;                                                           \
    uint32_t* AM = job->argmax;                                                  \
    const int64_t N = job->N, K = job->K;                                        \
    const int sr = job->sr;                                                      \
    T* acc = (T*)malloc(sizeof(T) * (size_t)(N > 0 ? N : 1));                    \
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(N > 0 ? N : 1)); \
    for (int64_t i = job->row_begin; i < job->row_end; ++i) {                    \
        const T z = ZERO(sr);                                                    \
        for (int64_t j = 0; j < N; ++j) { acc[j] = z; idx[j] = 0; }              \
        for (int64_t k = 0; k < K; ++k) {                                        \
            const T a = A[i * K + k];                                            \
            const T* brow = B + k * N;                                           \
            const uint32_t kk = (uint32_t)k;                                     \
            if (sr == TGO_MINPLUS) {                                             \
                for (int64_t j = 0; j < N; ++j) {                                \
                    const T p = MUL(sr, a, brow[j]);                             \
                    const int take = !(acc[j] <= p);                             \
                    acc[j] = take ? p : acc[j];                                  \
                    idx[j] = take ? kk : idx[j];                                 \
                }                                                                \
            } else {                                                             \
                for (int64_t j = 0; j < N; ++j) {                                \
                    const T p = MUL(sr, a, brow[j]);                             \
                    const int take = !(acc[j] >= p);                             \
                    acc[j] = take ? p : acc[j];                                  \
                    idx[j] = take ? kk : idx[j];                                 \
                }                                                                \
            }                                                                    \
        }                                                                        \
        memcpy(C + i * N, acc, sizeof(T) * (size_t)N);                           \
        if (AM) memcpy(AM + i * N, idx, sizeof(uint32_t) * (size_t)N);          \
    }                                                                            \
    free(acc);                                                                   \
    free(idx);                                                                   \
    return NULL;

static void* rows_f32(void* p) { tgo_job* job = (tgo_job*)p; TGO_ROWS_BODY(float, zero_f32, mul_f32) }
static void* rows_f64(void* p) { tgo_job* job = (tgo_job*)p; TGO_ROWS_BODY(double, zero_f64, mul_f64) }
static void* rows_i32(void* p) { tgo_job* job = (tgo_job*)p; TGO_ROWS_BODY(int32_t, zero_i32, mul_i32) }
static void* rows_i64(void* p) { tgo_job* job = (tgo_job*)p; TGO_ROWS_BODY(int64_t, zero_i64, mul_i64) }

static int run_rows(void* (*fn)(void*), int sr, const void* A, const void* B, void* C,
                    uint32_t* argmax, int64_t M, int64_t N, int64_t K, int nthreads) {
    if (sr < 0 || sr > 2 || M < 0 || N < 0 || K < 0) return -1;
    if (M == 0 || N == 0) return 0;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t)nthreads > M) nthreads = (int)M;
    tgo_job jobs[256];
    pthread_t th[256];
    const int64_t per = (M + nthreads - 1) / nthreads;
    int launched = 0;
    for (int t = 0; t < nthreads; ++t) {
        const int64_t b = (int64_t)t * per;
        const int64_t e = b + per < M ? b + per : M;
        if (b >= e) break;
        jobs[t] = (tgo_job){sr, A, B, C, argmax, M, N, K, b, e};
        launched++;
    }
    if (launched == 1) {
        fn(&jobs[0]);
        return 0;
    }
    for (int t = 0; t < launched; ++t) pthread_create(&th[t], NULL, fn, &jobs[t]);
    for (int t = 0; t < launched; ++t) pthread_join(th[t], NULL);
    return 0;
}

/* argmax may be NULL (value-only).  Returns 0 on success, -1 on bad args. */
int tgo_gemm_f32(int sr, const float* A, const float* B, float* C, uint32_t* argmax,
                 int64_t M, int64_t N, int64_t K, int nthreads) {
    return run_rows(rows_f32, sr, A, B, C, argmax, M, N, K, nthreads);
}
int tgo_gemm_f64(int sr, const double* A, const double* B, double* C, uint32_t* argmax,
                 int64_t M, int64_t N, int64_t K, int nthreads) {
    return run_rows(rows_f64, sr, A, B, C, argmax, M, N, K, nthreads);
}
int tgo_gemm_i32(int sr, const int32_t* A, const int32_t* B, int32_t* C, uint32_t* argmax,
                 int64_t M, int64_t N, int64_t K, int nthreads) {
    return run_rows(rows_i32, sr, A, B, C, argmax, M, N, K, nthreads);
}
int tgo_gemm_i64(int sr, const int64_t* A, const int64_t* B, int64_t* C, uint32_t* argmax,
                 int64_t M, int64_t N, int64_t K, int nthreads) {
    return run_rows(rows_i64, sr, A, B, C, argmax, M, N, K, nthreads);
}

/* ------------------------------------------------------------------------ */
/* Backward (api.rs:563-582, api.rs:627-646; python/src/lib.rs:877-950)      */
/* Row-major, loops i then j ascending, skip idx >= K.  Output overwritten.  */
/* b_or_a == NULL gives the additive (MaxPlus/MinPlus) rule; otherwise the   */
/* MaxMul rule multiplies grad_c by the winning B (for grad_a) or A (grad_b) */
/* value before accumulating.                                                */
/* ------------------------------------------------------------------------ */

#define TGO_BACKWARD_A(NAME, T)                                                       \
    void NAME(const T* grad_c, const uint32_t* argmax, const T* b, T* grad_a,         \
              int64_t M, int64_t N, int64_t K) {                                      \
        memset(grad_a, 0, sizeof(T) * (size_t)(M * K));                               \
        for (int64_t i = 0; i < M; ++i)                                               \
            for (int64_t j = 0; j < N; ++j) {                                         \
                const uint32_t kk = argmax[i * N + j];                                \
                if ((int64_t)kk < K) {                                                \
                    T g = grad_c[i * N + j];                                          \
                    if (b) g = g * b[(int64_t)kk * N + j];                            \
                    grad_a[i * K + kk] += g;                                          \
                }                                                                     \
            }                                                                         \
    }

#define TGO_BACKWARD_B(NAME, T)                                                       \
    void NAME(const T* grad_c, const uint32_t* argmax, const T* a, T* grad_b,         \
              int64_t M, int64_t N, int64_t K) {                                      \
        memset(grad_b, 0, sizeof(T) * (size_t)(K * N));                               \
        for (int64_t i = 0; i < M; ++i)                                               \
            for (int64_t j = 0; j < N; ++j) {                                         \
                const uint32_t kk = argmax[i * N + j];                                \
                if ((int64_t)kk < K) {                                                \
                    T g = grad_c[i * N + j];                                          \
                    if (a) g = g * a[i * K + kk];                                     \
                    grad_b[(int64_t)kk * N + j] += g;                                 \
                }                                                                     \
            }                                                                         \
    }

TGO_BACKWARD_A(tgo_backward_a_f32, float)
TGO_BACKWARD_A(tgo_backward_a_f64, double)
TGO_BACKWARD_B(tgo_backward_b_f32, float)
TGO_BACKWARD_B(tgo_backward_b_f64, double)

/* ------------------------------------------------------------------------ */
/* CPU baseline: single-thread restatement of the reference argmax path     */
/* (core/gemm.rs:167-244, packing.rs:46-161, kernel.rs:119-167,              */
/*  tiling.rs PORTABLE = MC 64, NC 64, KC 256, MR 4, NR 4).                  */
/* ------------------------------------------------------------------------ */

#define P_MC 64
#define P_NC 64
#define P_KC 256
#define P_MR 4
#define P_NR 4

/* The portable path for one scalar type T (suffix S): pack_a (mr-row
 * panels, k-major inside a panel, rows padded with scalar 0), pack_b
 * (nr-column panels, k-major, columns padded with 0), the 4x4 microkernel
 * with argmax (load (acc, idx) from C/argmax, visit k = k_offset + p
 * ascending with the CPU select rule, store back) and the 5-loop driver.
 * Row-major A (M x K), B (K x N); C/argmax are initialised to tropical zero
 * / 0 exactly as GemmWithArgmax::new does (core/argmax.rs:24-33). */
#define TGO_PORTABLE(T, S, ZERO, MUL)                                                           \
    static void pack_a_##S(int64_t mc, int64_t kc, const T* a, int64_t lda, T* packed) {        \
        int64_t p = 0;                                                                          \
        for (int64_t r0 = 0; r0 < mc; r0 += P_MR)                                               \
            for (int64_t col = 0; col < kc; ++col)                                              \
                for (int64_t ro = 0; ro < P_MR; ++ro) {                                         \
                    const int64_t row = r0 + ro;                                                \
                    packed[p++] = row < mc ? a[row * lda + col] : (T)0;                         \
                }                                                                               \
    }                                                                                           \
    static void pack_b_##S(int64_t kc, int64_t nc, const T* b, int64_t ldb, T* packed) {        \
        int64_t p = 0;                                                                          \
        for (int64_t c0 = 0; c0 < nc; c0 += P_NR)                                               \
            for (int64_t row = 0; row < kc; ++row)                                              \
                for (int64_t co = 0; co < P_NR; ++co) {                                         \
                    const int64_t col = c0 + co;                                                \
                    packed[p++] = col < nc ? b[row * ldb + col] : (T)0;                         \
                }                                                                               \
    }                                                                                           \
    static void micro_argmax_##S(int sr, int64_t mr, int64_t nr, int64_t kc, int64_t k_offset,  \
                                 const T* pa, const T* pb, T* c, uint32_t* am, int64_t ldc) {   \
        T acc[P_MR][P_NR];                                                                      \
        uint32_t idx[P_MR][P_NR];                                                               \
        for (int64_t i = 0; i < P_MR; ++i)                                                      \
            for (int64_t j = 0; j < P_NR; ++j) {                                                \
                acc[i][j] = ZERO(sr);                                                           \
                idx[i][j] = 0;                                                                  \
            }                                                                                   \
        for (int64_t i = 0; i < mr; ++i)                                                        \
            for (int64_t j = 0; j < nr; ++j) {                                                  \
                acc[i][j] = c[i * ldc + j];                                                     \
                idx[i][j] = am[i * ldc + j];                                                    \
            }                                                                                   \
        for (int64_t p = 0; p < kc; ++p) {                                                      \
            const uint32_t cur = (uint32_t)(k_offset + p);                                      \
            for (int64_t i = 0; i < mr; ++i) {                                                  \
                const T av = pa[p * P_MR + i];                                                  \
                for (int64_t j = 0; j < nr; ++j) {                                              \
                    const T prod = MUL(sr, av, pb[p * P_NR + j]);                               \
                    const int keep =                                                            \
                        sr == TGO_MINPLUS ? (acc[i][j] <= prod) : (acc[i][j] >= prod);          \
                    if (!keep) {                                                                \
                        acc[i][j] = prod;                                                       \
                        idx[i][j] = cur;                                                        \
                    }                                                                           \
                }                                                                               \
            }                                                                                   \
        }                                                                                       \
        for (int64_t i = 0; i < mr; ++i)                                                        \
            for (int64_t j = 0; j < nr; ++j) {                                                  \
                c[i * ldc + j] = acc[i][j];                                                     \
                am[i * ldc + j] = idx[i][j];                                                    \
            }                                                                                   \
    }                                                                                           \
    int tgo_portable_argmax_##S(int sr, const T* A, const T* B, T* C, uint32_t* argmax,         \
                                int64_t M, int64_t N, int64_t K) {                              \
        if (sr < 0 || sr > 2 || M < 0 || N < 0 || K < 0) return -1;                             \
        for (int64_t t = 0; t < M * N; ++t) {                                                   \
            C[t] = ZERO(sr);                                                                    \
            argmax[t] = 0;                                                                      \
        }                                                                                       \
        if (M == 0 || N == 0 || K == 0) return 0;                                               \
        T* pa = (T*)malloc(sizeof(T) * P_MC * P_KC);                                            \
        T* pb = (T*)malloc(sizeof(T) * P_KC * P_NC);                                            \
        if (!pa || !pb) {                                                                       \
            free(pa);                                                                           \
            free(pb);                                                                           \
            return -2;                                                                          \
        }                                                                                       \
        const int64_t ldc = N;                                                                  \
        for (int64_t jc = 0; jc < N; jc += P_NC) {                                              \
            const int64_t nc = N - jc < P_NC ? N - jc : P_NC;                                   \
            for (int64_t pc = 0; pc < K; pc += P_KC) {                                          \
                const int64_t kc = K - pc < P_KC ? K - pc : P_KC;                               \
                pack_b_##S(kc, nc, B + pc * N + jc, N, pb);                                     \
                for (int64_t ic = 0; ic < M; ic += P_MC) {                                      \
                    const int64_t mc = M - ic < P_MC ? M - ic : P_MC;                           \
                    pack_a_##S(mc, kc, A + ic * K + pc, K, pa);                                 \
                    for (int64_t jr = 0; jr * P_NR < nc; ++jr) {                                \
                        const int64_t j0 = jr * P_NR;                                           \
                        const int64_t nr = nc - j0 < P_NR ? nc - j0 : P_NR;                     \
                        for (int64_t ir = 0; ir * P_MR < mc; ++ir) {                            \
                            const int64_t i0 = ir * P_MR;                                       \
                            const int64_t mr = mc - i0 < P_MR ? mc - i0 : P_MR;                 \
                            micro_argmax_##S(sr, mr, nr, kc, pc, pa + ir * P_MR * kc,           \
                                             pb + jr * P_NR * kc,                               \
                                             C + (ic + i0) * ldc + (jc + j0),                   \
                                             argmax + (ic + i0) * ldc + (jc + j0), ldc);        \
                        }                                                                       \
                    }                                                                           \
                }                                                                               \
            }                                                                                   \
        }                                                                                       \
        free(pa);                                                                               \
        free(pb);                                                                               \
        return 0;                                                                               \
    }

TGO_PORTABLE(float, f32, zero_f32, mul_f32)
TGO_PORTABLE(double, f64, zero_f64, mul_f64)
TGO_PORTABLE(int32_t, i32, zero_i32, mul_i32)
TGO_PORTABLE(int64_t, i64, zero_i64, mul_i64)

/* ------------------------------------------------------------------------ */
/* CPU BASELINE for value-only integer products: the reference's portable   */
/* value path (simd/dispatch.rs:233-242 sends every i32 / i64 semiring to    */
/* PortableKernel with TilingParams::PORTABLE): the same 5-loop driver and   */
/* packing as above, and the 4x4 value microkernel of core/kernel.rs:72-117  */
/* (load the accumulators from C, acc = acc (+) a (x) b for k ascending,     */
/* store back).  (+) is max (MaxPlus, MaxMul) or min (MinPlus); on integers  */
/* the reference's tropical_add returns the same value whichever way ties   */
/* go (types/max_plus.rs, min_plus.rs, max_mul.rs).                          */
/* ------------------------------------------------------------------------ */
#define TGO_PORTABLE_VALUE(T, S, ZERO, MUL)                                                     \
    static void micro_value_##S(int sr, int64_t mr, int64_t nr, int64_t kc, const T* pa,       \
                                const T* pb, T* c, int64_t ldc) {                               \
        T acc[P_MR][P_NR];                                                                      \
        for (int64_t i = 0; i < P_MR; ++i)                                                      \
            for (int64_t j = 0; j < P_NR; ++j) acc[i][j] = ZERO(sr);                            \
        for (int64_t i = 0; i < mr; ++i)                                                        \
            for (int64_t j = 0; j < nr; ++j) acc[i][j] = c[i * ldc + j];                        \
        for (int64_t p = 0; p < kc; ++p)                                                        \
            for (int64_t i = 0; i < mr; ++i) {                                                  \
                const T av = pa[p * P_MR + i];                                                  \
                for (int64_t j = 0; j < nr; ++j) {                                              \
                    const T prod = MUL(sr, av, pb[p * P_NR + j]);                               \
                    if (sr == TGO_MINPLUS ? prod < acc[i][j] : prod > acc[i][j]) acc[i][j] = prod; \
                }                                                                               \
            }                                                                                   \
        for (int64_t i = 0; i < mr; ++i)                                                        \
            for (int64_t j = 0; j < nr; ++j) c[i * ldc + j] = acc[i][j];                        \
    }                                                                                           \
    int tgo_portable_gemm_##S(int sr, const T* A, const T* B, T* C, int64_t M, int64_t N,     \
                              int64_t K) {                                                      \
        if (sr < 0 || sr > 2 || M < 0 || N < 0 || K < 0) return -1;                             \
        for (int64_t t = 0; t < M * N; ++t) C[t] = ZERO(sr);                                    \
        if (M == 0 || N == 0 || K == 0) return 0;                                               \
        T* pa = (T*)malloc(sizeof(T) * P_MC * P_KC);                                            \
        T* pb = (T*)malloc(sizeof(T) * P_KC * P_NC);                                            \
        if (!pa || !pb) {                                                                       \
            free(pa);                                                                           \
            free(pb);                                                                           \
            return -2;                                                                          \
        }                                                                                       \
        for (int64_t jc = 0; jc < N; jc += P_NC) {                                              \
            const int64_t nc = N - jc < P_NC ? N - jc : P_NC;                                   \
            for (int64_t pc = 0; pc < K; pc += P_KC) {                                          \
                const int64_t kc = K - pc < P_KC ? K - pc : P_KC;                               \
                pack_b_##S(kc, nc, B + pc * N + jc, N, pb);                                     \
                for (int64_t ic = 0; ic < M; ic += P_MC) {                                      \
                    const int64_t mc = M - ic < P_MC ? M - ic : P_MC;                           \
                    pack_a_##S(mc, kc, A + ic * K + pc, K, pa);                                 \
                    for (int64_t jr = 0; jr * P_NR < nc; ++jr) {                                \
                        const int64_t j0 = jr * P_NR;                                           \
                        const int64_t nr = nc - j0 < P_NR ? nc - j0 : P_NR;                     \
                        for (int64_t ir = 0; ir * P_MR < mc; ++ir) {                            \
                            const int64_t i0 = ir * P_MR;                                       \
                            const int64_t mr = mc - i0 < P_MR ? mc - i0 : P_MR;                 \
                            micro_value_##S(sr, mr, nr, kc, pa + ir * P_MR * kc,                \
                                            pb + jr * P_NR * kc, C + (ic + i0) * N + (jc + j0), \
                                            N);                                                 \
                        }                                                                       \
                    }                                                                           \
                }                                                                               \
            }                                                                                   \
        }                                                                                       \
        free(pa);                                                                               \
        free(pb);                                                                               \
        return 0;                                                                               \
    }

TGO_PORTABLE_VALUE(int32_t, i32, zero_i32, mul_i32)
TGO_PORTABLE_VALUE(int64_t, i64, zero_i64, mul_i64)

/* ------------------------------------------------------------------------ */
/* CPU BASELINE for value-only f32: the reference's AVX2 path                */
/* (simd/kernels/avx2.rs: 8x8 f32 microkernels for MaxPlus, MinPlus and      */
/*  MaxMul; core/gemm.rs:81-134 5-loop driver; tiling.rs F32_AVX2 = MC 256,  */
/*  NC 256, KC 512, MR 8, NR 8; packing.rs:46-161 with MR = NR = 8).         */
/* The microkernel keeps one 8-wide row of C per register, and per k         */
/* broadcasts A[i,k] and combines it with the packed 8-wide row of B.        */
/* ------------------------------------------------------------------------ */
#include <immintrin.h>

#define V_MC 256
#define V_NC 256
#define V_KC 512
#define V_MR 8
#define V_NR 8

static void vpack_a_f32(int64_t mc, int64_t kc, const float* a, int64_t lda, float* packed) {
    int64_t p = 0;
    for (int64_t r0 = 0; r0 < mc; r0 += V_MR)
        for (int64_t col = 0; col < kc; ++col)
            for (int64_t ro = 0; ro < V_MR; ++ro) {
                const int64_t row = r0 + ro;
                packed[p++] = row < mc ? a[row * lda + col] : 0.0f;
            }
}

static void vpack_b_f32(int64_t kc, int64_t nc, const float* b, int64_t ldb, float* packed) {
    int64_t p = 0;
    for (int64_t c0 = 0; c0 < nc; c0 += V_NR)
        for (int64_t row = 0; row < kc; ++row)
            for (int64_t co = 0; co < V_NR; ++co) {
                const int64_t col = c0 + co;
                packed[p++] = col < nc ? b[row * ldb + col] : 0.0f;
            }
}

/* One 8x8 block: acc rows start as tropical zero, the valid mr x nr part is
 * loaded from C; per k, acc[i] = acc[i] (+) (A[i,k] (x) B[k, 0..7]). */
static void vmicro_f32(int sr, int64_t mr, int64_t nr, int64_t kc, const float* pa,
                       const float* pb, float* c, int64_t ldc) {
    __m256 acc[V_MR];
    for (int64_t i = 0; i < V_MR; ++i) {
        float row[V_NR];
        for (int64_t j = 0; j < V_NR; ++j) row[j] = (i < mr && j < nr) ? c[i * ldc + j] : zero_f32(sr);
        acc[i] = _mm256_loadu_ps(row);
    }
    if (sr == TGO_MAXPLUS) {
        for (int64_t p = 0; p < kc; ++p) {
            const __m256 bv = _mm256_loadu_ps(pb + p * V_NR);
            for (int64_t i = 0; i < V_MR; ++i)
                acc[i] = _mm256_max_ps(acc[i], _mm256_add_ps(_mm256_set1_ps(pa[p * V_MR + i]), bv));
        }
    } else if (sr == TGO_MINPLUS) {
        for (int64_t p = 0; p < kc; ++p) {
            const __m256 bv = _mm256_loadu_ps(pb + p * V_NR);
            for (int64_t i = 0; i < V_MR; ++i)
                acc[i] = _mm256_min_ps(acc[i], _mm256_add_ps(_mm256_set1_ps(pa[p * V_MR + i]), bv));
        }
    } else {
        for (int64_t p = 0; p < kc; ++p) {
            const __m256 bv = _mm256_loadu_ps(pb + p * V_NR);
            for (int64_t i = 0; i < V_MR; ++i)
                acc[i] = _mm256_max_ps(acc[i], _mm256_mul_ps(_mm256_set1_ps(pa[p * V_MR + i]), bv));
        }
    }
    for (int64_t i = 0; i < mr; ++i) {
        float row[V_NR];
        _mm256_storeu_ps(row, acc[i]);
        for (int64_t j = 0; j < nr; ++j) c[i * ldc + j] = row[j];
    }
}

/* Row-major value-only C = A (x) B; C is initialised to tropical zero. */
int tgo_avx2_gemm_f32(int sr, const float* A, const float* B, float* C, int64_t M, int64_t N,
                      int64_t K) {
    if (sr < 0 || sr > 2 || M < 0 || N < 0 || K < 0) return -1;
    for (int64_t t = 0; t < M * N; ++t) C[t] = zero_f32(sr);
    if (M == 0 || N == 0 || K == 0) return 0;
    float* pa = (float*)malloc(sizeof(float) * V_MC * V_KC);
    float* pb = (float*)malloc(sizeof(float) * V_KC * V_NC);
    if (!pa || !pb) {
        free(pa);
        free(pb);
        return -2;
    }
    for (int64_t jc = 0; jc < N; jc += V_NC) {
        const int64_t nc = N - jc < V_NC ? N - jc : V_NC;
        for (int64_t pc = 0; pc < K; pc += V_KC) {
            const int64_t kc = K - pc < V_KC ? K - pc : V_KC;
            vpack_b_f32(kc, nc, B + pc * N + jc, N, pb);
            for (int64_t ic = 0; ic < M; ic += V_MC) {
                const int64_t mc = M - ic < V_MC ? M - ic : V_MC;
                vpack_a_f32(mc, kc, A + ic * K + pc, K, pa);
                for (int64_t jr = 0; jr * V_NR < nc; ++jr) {
                    const int64_t j0 = jr * V_NR;
                    const int64_t nr = nc - j0 < V_NR ? nc - j0 : V_NR;
                    for (int64_t ir = 0; ir * V_MR < mc; ++ir) {
                        const int64_t i0 = ir * V_MR;
                        const int64_t mr = mc - i0 < V_MR ? mc - i0 : V_MR;
                        vmicro_f32(sr, mr, nr, kc, pa + ir * V_MR * kc, pb + jr * V_NR * kc,
                                   C + (ic + i0) * N + (jc + j0), N);
                    }
                }
            }
        }
    }
    free(pa);
    free(pb);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* CPU BASELINE for value-only MaxPlus f64: the reference's AVX2 path        */
/* (simd/kernels/avx2.rs:77-143: a 4x4 microkernel on f64x4 rows, per k     */
/*  acc[i] = max(acc[i], A[i,k] + B[k,0..3]); core/gemm.rs:81-134 driver;    */
/*  tiling.rs:29-35 F64_AVX2 = MC 128, NC 128, KC 256, MR 4, NR 4).          */
/* ------------------------------------------------------------------------ */
#define D_MC 128
#define D_NC 128
#define D_KC 256
#define D_MR 4
#define D_NR 4

static void dpack_a_f64(int64_t mc, int64_t kc, const double* a, int64_t lda, double* packed) {
    int64_t p = 0;
    for (int64_t r0 = 0; r0 < mc; r0 += D_MR)
        for (int64_t col = 0; col < kc; ++col)
            for (int64_t ro = 0; ro < D_MR; ++ro) {
                const int64_t row = r0 + ro;
                packed[p++] = row < mc ? a[row * lda + col] : 0.0;
            }
}

static void dpack_b_f64(int64_t kc, int64_t nc, const double* b, int64_t ldb, double* packed) {
    int64_t p = 0;
    for (int64_t c0 = 0; c0 < nc; c0 += D_NR)
        for (int64_t row = 0; row < kc; ++row)
            for (int64_t co = 0; co < D_NR; ++co) {
                const int64_t col = c0 + co;
                packed[p++] = col < nc ? b[row * ldb + col] : 0.0;
            }
}

static void dmicro_maxplus_f64(int64_t mr, int64_t nr, int64_t kc, const double* pa,
                               const double* pb, double* c, int64_t ldc) {
    __m256d acc[D_MR];
    for (int64_t i = 0; i < D_MR; ++i) {
        double row[D_NR];
        for (int64_t j = 0; j < D_NR; ++j) row[j] = (i < mr && j < nr) ? c[i * ldc + j] : -INFINITY;
        acc[i] = _mm256_loadu_pd(row);
    }
    for (int64_t p = 0; p < kc; ++p) {
        const __m256d bv = _mm256_loadu_pd(pb + p * D_NR);
        for (int64_t i = 0; i < D_MR; ++i)
            acc[i] = _mm256_max_pd(acc[i], _mm256_add_pd(_mm256_set1_pd(pa[p * D_MR + i]), bv));
    }
    for (int64_t i = 0; i < mr; ++i) {
        double row[D_NR];
        _mm256_storeu_pd(row, acc[i]);
        for (int64_t j = 0; j < nr; ++j) c[i * ldc + j] = row[j];
    }
}

/* Row-major value-only MaxPlus C = A (x) B; C is initialised to -inf. */
int tgo_avx2_gemm_maxplus_f64(const double* A, const double* B, double* C, int64_t M, int64_t N,
                              int64_t K) {
    if (M < 0 || N < 0 || K < 0) return -1;
    for (int64_t t = 0; t < M * N; ++t) C[t] = -INFINITY;
    if (M == 0 || N == 0 || K == 0) return 0;
    double* pa = (double*)malloc(sizeof(double) * D_MC * D_KC);
    double* pb = (double*)malloc(sizeof(double) * D_KC * D_NC);
    if (!pa || !pb) {
        free(pa);
        free(pb);
        return -2;
    }
    for (int64_t jc = 0; jc < N; jc += D_NC) {
        const int64_t nc = N - jc < D_NC ? N - jc : D_NC;
        for (int64_t pc = 0; pc < K; pc += D_KC) {
            const int64_t kc = K - pc < D_KC ? K - pc : D_KC;
            dpack_b_f64(kc, nc, B + pc * N + jc, N, pb);
            for (int64_t ic = 0; ic < M; ic += D_MC) {
                const int64_t mc = M - ic < D_MC ? M - ic : D_MC;
                dpack_a_f64(mc, kc, A + ic * K + pc, K, pa);
                for (int64_t jr = 0; jr * D_NR < nc; ++jr) {
                    const int64_t j0 = jr * D_NR;
                    const int64_t nr = nc - j0 < D_NR ? nc - j0 : D_NR;
                    for (int64_t ir = 0; ir * D_MR < mc; ++ir) {
                        const int64_t i0 = ir * D_MR;
                        const int64_t mr = mc - i0 < D_MR ? mc - i0 : D_MR;
                        dmicro_maxplus_f64(mr, nr, kc, pa + ir * D_MR * kc, pb + jr * D_NR * kc,
                                           C + (ic + i0) * N + (jc + j0), N);
                    }
                }
            }
        }
    }
    free(pa);
    free(pb);
    return 0;
}

int tgo_version(void) { return 2; }
