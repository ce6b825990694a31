/*
 * tropical_gemm_hip.h -- C ABI of the MI355X (gfx950) tropical GEMM library.
 *
 * This is the drop-in boundary that replaces the GPU layer of the reference's
 * `tropical-gemm-cuda` crate (kernels + cudarc launch code).  Every entry
 * point takes plain pointers and sizes; buffers are caller-owned device
 * memory (as with the reference's ExternalGpuMatrix / DLPack path,
 * crates/tropical-gemm-cuda/src/memory.rs:263-454).  All compute calls are
 * asynchronous on the given HIP stream (NULL = the device's null stream);
 * callers that need the reference's blocking behaviour call
 * tg_stream_synchronize() afterwards (the reference synchronises after every
 * launch, crates/tropical-gemm-cuda/src/kernels.rs:65).
 *
 * Semantics (bit-exact with the reference CPU path; a NaN product replaces
 * the running value and the next product replaces a NaN, as the CPU's
 * "keep acc iff acc >= p" rule does, types/max_plus.rs:66-73):
 *   C[i,j]      = (+)_k A[i,k] (x) B[k,j], k visited in ascending order;
 *   argmax[i,j] = the first k attaining C[i,j] (0 when no product beats the
 *                 tropical zero), written as int32 (the reference GPU's
 *                 ArgmaxIndex = i32, memory.rs:10; same bits as the CPU's u32).
 *   MaxPlus: (+)=max, (x)=+, zero=-inf | INT_MIN
 *   MinPlus: (+)=min, (x)=+, zero=+inf | INT_MAX
 *   MaxMul : (+)=max, (x)=*, zero=0
 *   Integer (x) wraps (two's complement), as the reference CPU release build
 *   (crates/tropical-gemm/src/types/scalar.rs:94-112).
 *
 * Layouts: TG_ROW_MAJOR (PyTorch/DLPack, the CPU API) or TG_COL_MAJOR (the
 * reference GPU API, crates/tropical-gemm-cuda/src/lib.rs:1-4).  Matrices are
 * dense (leading dimension = rows for col-major, cols for row-major).
 */
#ifndef TROPICAL_GEMM_HIP_H
#define TROPICAL_GEMM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  One per CudaError variant of the reference
 * (crates/tropical-gemm-cuda/src/error.rs:8-29), plus argument errors that the
 * reference reports through panics/asserts or PyO3 ValueErrors. */
enum {
    TG_OK = 0,
    TG_ERR_DRIVER = 1,             /* CudaError::Driver -> a HIP runtime error      */
    TG_ERR_COMPILE = 2,            /* CudaError::Compile: unreachable (AOT kernels)  */
    TG_ERR_NO_DEVICE = 3,          /* CudaError::NoDevice                           */
    TG_ERR_DIMENSION_MISMATCH = 4, /* CudaError::DimensionMismatch(String)          */
    TG_ERR_KERNEL_NOT_FOUND = 5,   /* CudaError::KernelNotFound(String)             */
    TG_ERR_INVALID_ARGUMENT = 6,   /* null pointer, bad enum, negative size         */
    TG_ERR_UNSUPPORTED = 7         /* e.g. integer gradients (none in the reference) */
};

typedef enum { TG_MAXPLUS = 0, TG_MINPLUS = 1, TG_MAXMUL = 2 } tg_semiring;
typedef enum { TG_F32 = 0, TG_F64 = 1, TG_I32 = 2, TG_I64 = 3 } tg_dtype;
typedef enum { TG_ROW_MAJOR = 0, TG_COL_MAJOR = 1 } tg_layout;

/* ---- diagnostics ------------------------------------------------------- */

/* Library ABI version (bumped on any signature change). */
int tg_version(void);
/* Static description of a status code. */
const char* tg_status_string(int status);
/* Thread-local detail of the last failing call on this thread (the String
 * payload of CudaError::DimensionMismatch etc.).  Never NULL. */
const char* tg_last_error(void);

/* ---- devices and contexts ---------------------------------------------- */

/* Replaces cuda_device_count (crates/tropical-gemm-cuda/src/lib.rs:60-63). */
int tg_device_count(int* count);
/* Replaces get_context_for_device (lib.rs:79-122): validates the ordinal and
 * initialises the device once per process (thread-safe).  Code objects are
 * compiled ahead of time, so there is no NVRTC step (context.rs:87-104). */
int tg_context_init(int device);
/* Device name, like CudaContext::device_name (context.rs:121-123). */
int tg_device_name(int device, char* buf, size_t len);

/* ---- memory (backs GpuMatrix / GpuTensor3, memory.rs:31-573) ----------- */

int tg_malloc(int device, void** ptr, size_t bytes);
int tg_free(int device, void* ptr);
int tg_memcpy_htod(int device, void* dst, const void* src, size_t bytes); /* blocking */
int tg_memcpy_dtoh(int device, void* dst, const void* src, size_t bytes); /* blocking */
int tg_memcpy_dtod(int device, void* dst, const void* src, size_t bytes, void* stream);
/* Fills with zero bytes using a kernel (safe under graph capture). */
int tg_memset_zero(int device, void* ptr, size_t bytes, void* stream);
int tg_synchronize(int device);
int tg_stream_synchronize(int device, void* stream);

/* ---- kernel timing (diagnostics) ----------------------------------------
 * No counterpart in the reference; used by benchmarks to time the main GEMM
 * kernel apart from the B^T staging kernel that some argmax calls also launch. */

/* on != 0: every forward call records a HIP event pair on its stream around
 * its main GEMM kernel(s).  Off by default (no events, no overhead). */
int tg_kernel_timing_enable(int on);
/* Waits for the recorded events, returns the summed main-kernel time in
 * milliseconds and the number of launches since the last read, and clears
 * the record. */
int tg_kernel_timing_read(double* total_ms, int64_t* launches);

/* ---- forward ----------------------------------------------------------- */

/*
 * C = A (x) B with optional argmax.
 * Replaces CudaKernel::launch_gemm / CudaKernelWithArgmax::launch_gemm_with_argmax
 * (kernels.rs:12-360) and the row-major external launchers
 * launch_gemm_external_f32 / launch_gemm_external_with_argmax_f32
 * (kernels.rs:388-473), for all four dtypes and three semirings.
 *   A: m x k, B: k x n, C: m x n, argmax: m x n int32 or NULL (value-only).
 * m, n, k >= 0; k == 0 yields C = tropical zero and argmax = 0
 * (core/gemm.rs:70-72 leaves the zero-initialised result untouched).
 * Uses a stream-ordered workspace allocation when the kernel it picks needs
 * one (argmax with B^T staging, split K); see tg_gemm_workspace_size /
 * tg_gemm_ws to pass one instead.
 */
int tg_gemm(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
            const void* A, const void* B, void* C, int32_t* argmax,
            int64_t m, int64_t n, int64_t k, void* stream);

/* Bytes of device workspace tg_gemm_ws needs for this problem, each part
 * 256-byte aligned: with argmax, B^T staging of batch x k x max(m, n)
 * elements (column-major calls swap the operands, so the bound covers both
 * layouts); for f64, 4 bytes per row of A and column of B (operand classes
 * of the f64 direct-to-LDS kernel); for 32-bit problems the library splits
 * in k, the per-slice partials (values, and indices with argmax).  0 for
 * 32-bit value-only problems that are not split.  batch = 1 for single
 * products. */
size_t tg_gemm_workspace_size(tg_dtype dtype, int64_t batch, int64_t m, int64_t n, int64_t k,
                              int with_argmax);

/* Name of the kernel path tg_gemm_ws would run for this problem with a
 * workspace of workspace_bytes (tg_gemm passes tg_gemm_workspace_size), e.g.
 * "dl_4x8_cl16", "shortk", "tiles_exact", "dl_4x4_cl32 split 4" (K in four
 * launches merged afterwards) or "dl_4x4_cl8 slices 4" (four K slices in one
 * workgroup per tile); "invalid" for arguments the call would reject, "none"
 * for an empty product.  Strides
 * 0 mean dense single products.  Pure host logic: pointers are only checked
 * for alignment, never dereferenced, and no device is needed.  Diagnostic,
 * with no counterpart in the reference (which has one kernel per dtype). */
const char* tg_gemm_plan(tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                         const void* A, const void* B, const void* C, const int32_t* argmax,
                         int64_t batch, int64_t m, int64_t n, int64_t k,
                         int64_t stride_a, int64_t stride_b, int64_t stride_c,
                         size_t workspace_bytes);

/* Launch geometry the backward entry points would use for a gradient
 * (want_a: 1 for grad A, 0 for grad B), e.g. "rows lds waves=2 lds=32768
 * grid=2048": the kernel family (rows / cols), where the bins live (LDS, or
 * the gradient itself for very large k), waves per workgroup, dynamic LDS
 * bytes and workgroups; grad B plans end in " passes=P" when long columns
 * take their keys in P passes.  Grids are capped (the kernels loop with a
 * grid stride), so no launch dimension grows with m, n or batch.  Host logic
 * only; diagnostic, with no counterpart in the reference. */
const char* tg_backward_plan(tg_dtype dtype, tg_layout layout, int want_a, int64_t batch,
                             int64_t m, int64_t n, int64_t k);

/* tg_gemm with a caller-provided workspace of at least
 * tg_gemm_workspace_size(...) bytes, 256-byte aligned (no allocation). */
int tg_gemm_ws(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
               const void* A, const void* B, void* C, int32_t* argmax,
               int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
               void* stream);

/* tg_gemm that allocates nothing (no hipMalloc / hipFree, no allocating
 * library call): its workspace is a fixed 64 MiB device array of the library
 * (TG_NOALLOC_SCRATCH_BYTES), one per device, held until the process ends.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, serving loops, harnesses that forbid it).  A
 * problem whose kernel needs more workspace than that (argmax with
 * k x max(m, n) elements above it on the chunked-argmax paths) is rejected
 * with TG_ERR_INVALID_ARGUMENT before any device work.  Every call on one
 * device shares that device's array, so calls that overlap on one device
 * (other streams, other host threads) race; serialise them.  The kernels
 * write every scratch byte they read, so nothing needs clearing between
 * calls.  Same arguments, results and errors as tg_gemm otherwise. */
#define TG_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int tg_gemm_noalloc(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                    const void* A, const void* B, void* C, int32_t* argmax,
                    int64_t m, int64_t n, int64_t k, void* stream);

/* Bytes of the fixed scratch array tg_gemm_noalloc would use for this
 * problem (0 when its kernel reads no workspace); a call whose need is above
 * TG_NOALLOC_SCRATCH_BYTES is rejected.  (size_t)-1 for arguments the call
 * would reject.  Pure host logic, as tg_gemm_plan (pointers are checked for
 * alignment only).  Diagnostic, with no counterpart in the reference. */
size_t tg_gemm_noalloc_bytes(tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                             const void* A, const void* B, const void* C, const int32_t* argmax,
                             int64_t m, int64_t n, int64_t k);

/*
 * Strided batched product: C[t] = A[t] (x) B[t] for t < batch, element
 * strides between consecutive matrices.  Replaces
 * launch_gemm_external_batched_with_argmax_f32 (kernels.rs:498-550, f32 only
 * in the reference) and the per-item loops of tropical_matmul_gpu_batched /
 * tropical_matmul_gpu_strided_batched (lib.rs:486-616).
 * argmax (batch x m x n, stride stride_c) may be NULL.
 */
int tg_gemm_strided_batched(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                            const void* A, const void* B, void* C, int32_t* argmax,
                            int64_t batch, int64_t m, int64_t n, int64_t k,
                            int64_t stride_a, int64_t stride_b, int64_t stride_c, void* stream);

int tg_gemm_strided_batched_ws(int device, tg_semiring semiring, tg_dtype dtype,
                               tg_layout layout, const void* A, const void* B, void* C,
                               int32_t* argmax, int64_t batch, int64_t m, int64_t n, int64_t k,
                               int64_t stride_a, int64_t stride_b, int64_t stride_c,
                               void* workspace, size_t workspace_bytes, void* stream);

/* ---- backward (argmax scatter) ---------------------------------------- */

/*
 * grad_a[i, argmax[i,j]] += grad_c[i,j]   (entries with argmax outside
 * [0,k) are skipped).  grad_a (m x k) is fully overwritten.
 * Replaces tropical_backward_a_gpu_kernel + kernel tropical_backward_a_{f32,f64}
 * (crates/tropical-gemm-cuda/src/lib.rs:841-882, tropical_gemm.cu:1002-1018) and
 * the torch scatter_add_ backward (pytorch.py:386-403).  Float dtypes only.
 * Deterministic: every element is summed from +0 in ascending j, the order of
 * the reference CPU loop (crates/tropical-gemm/src/api.rs:563-582), so the
 * result is bit-identical to it and to every other run.  m == 0 or n == 0
 * (grad_c and argmax may then be NULL) gives an all-(+0) gradient.
 */
int tg_backward_a(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                  const int32_t* argmax, void* grad_a, int64_t m, int64_t n, int64_t k,
                  void* stream);

/* grad_b[argmax[i,j], j] += grad_c[i,j]; grad_b (k x n) fully overwritten.
 * Replaces tropical_backward_b_gpu_kernel (lib.rs:901-942, .cu:1020-1036).
 * Summed from +0 in ascending i (api.rs:627-646): bit-identical, deterministic. */
int tg_backward_b(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                  const int32_t* argmax, void* grad_b, int64_t m, int64_t n, int64_t k,
                  void* stream);

/* MaxMul multiplicative rule (pytorch.py:521-548, python/src/lib.rs:877-950):
 *   grad_a[i, kk] += grad_c[i,j] * B[kk, j],  kk = argmax[i,j]. */
int tg_maxmul_backward_a(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                         const int32_t* argmax, const void* B, void* grad_a, int64_t m,
                         int64_t n, int64_t k, void* stream);

/*   grad_b[kk, j] += grad_c[i,j] * A[i, kk]. */
int tg_maxmul_backward_b(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                         const int32_t* argmax, const void* A, void* grad_b, int64_t m,
                         int64_t n, int64_t k, void* stream);

/* Batched forms of the four backward entry points (the batched autograd
 * classes, pytorch.py:624-640, 714-730, 811-832; lib.rs:758-818).  Element
 * strides: grad_c/argmax use stride_c, grad_a uses stride_a (m*k when dense),
 * grad_b uses stride_b (k*n when dense); `other` (B for _a, A for _b) is NULL
 * for the additive rule and uses stride_other. */
int tg_backward_a_strided_batched(int device, tg_dtype dtype, tg_layout layout,
                                  const void* grad_c, const int32_t* argmax, const void* other,
                                  void* grad_a, int64_t batch, int64_t m, int64_t n, int64_t k,
                                  int64_t stride_c, int64_t stride_other, int64_t stride_a,
                                  void* stream);
int tg_backward_b_strided_batched(int device, tg_dtype dtype, tg_layout layout,
                                  const void* grad_c, const int32_t* argmax, const void* other,
                                  void* grad_b, int64_t batch, int64_t m, int64_t n, int64_t k,
                                  int64_t stride_c, int64_t stride_other, int64_t stride_b,
                                  void* stream);

/* Dense batched transpose: dst[z][c][r] = src[z][r][c] for batch matrices
 * of rows x cols (each dst matrix cols x rows), any dtype.  No counterpart in
 * the reference: it is the data movement of the tropical einsum (the
 * permutations its contraction plan leaves to a tensor library,
 * docs/plans/2026-01-26-tropical-einsum-design.md:245-300), which moves one
 * group of adjacent axes past another.  rows < 2^21 (the grid); src and dst
 * must not overlap. */
int tg_transpose(int device, tg_dtype dtype, const void* src, void* dst, int64_t batch,
                 int64_t rows, int64_t cols, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TROPICAL_GEMM_HIP_H */
