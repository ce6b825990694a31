// tropical_gemm_hip.hpp -- C++ host API of the MI355X tropical GEMM backend.
//
// Mirrors the public surface of the reference's GPU crate
// (crates/tropical-gemm-cuda/src/lib.rs:135-145 re-exports): the same names,
// argument meaning, column-major data convention, blocking behaviour and
// error kinds, over the C ABI of include/tropical_gemm_hip.h.  Header-only;
// link with -ltropical_gemm_hip.
//
//   reference (Rust)                         here (C++)
//   CudaError / Result<T>                    HipError (exception), ErrorKind
//   CudaContext                              HipContext
//   cuda_device_count / get_context_for_device / get_global_context
//                                            hip_device_count / same names
//   GpuMatrix, GpuMatrixWithArgmax,          same names
//   GpuTensor3(+WithArgmax), ExternalGpu*    same names
//   tropical_matmul_gpu* / tropical_gemm_gpu* / backward fns   same names
//   GpuMat<S>, GpuMatWithArgmax<S>           same names
//   TropicalMaxPlus<T> etc. (tropical-gemm)  semiring tags of the same names
//
// All matrices are column-major, as in the reference GPU API
// (crates/tropical-gemm-cuda/src/lib.rs:1-4); the library maps them onto its
// row-major kernels with the operand swap C^T = B^T (x) A^T.
#pragma once

#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "../../include/tropical_gemm_hip.h"

namespace tropical_gemm_hip {

// ---------------------------------------------------------------------------
// Errors (crates/tropical-gemm-cuda/src/error.rs:8-29)
// ---------------------------------------------------------------------------

enum class ErrorKind {
    Driver,             // CudaError::Driver
    Compile,            // CudaError::Compile (unreachable: kernels are compiled ahead of time)
    NoDevice,           // CudaError::NoDevice
    DimensionMismatch,  // CudaError::DimensionMismatch(String)
    KernelNotFound,     // CudaError::KernelNotFound(String)
    InvalidArgument,    // argument errors the reference reports by panicking
    Unsupported,        // e.g. integer gradients
};

class HipError : public std::runtime_error {
  public:
    HipError(ErrorKind kind, const std::string& msg) : std::runtime_error(format(kind, msg)), kind_(kind) {}
    ErrorKind kind() const noexcept { return kind_; }

  private:
    // Display strings follow the reference's #[error(...)] attributes.
    static std::string format(ErrorKind k, const std::string& msg) {
        switch (k) {
            case ErrorKind::Driver: return "HIP driver error: " + msg;
            case ErrorKind::Compile: return "HIP compilation error: " + msg;
            case ErrorKind::NoDevice: return "No HIP device available";
            case ErrorKind::DimensionMismatch: return "Dimension mismatch: " + msg;
            case ErrorKind::KernelNotFound: return "Kernel not found: " + msg;
            case ErrorKind::InvalidArgument: return "Invalid argument: " + msg;
            case ErrorKind::Unsupported: return "Unsupported: " + msg;
        }
        return msg;
    }
    ErrorKind kind_;
};

namespace detail {

inline ErrorKind kind_of(int rc) {
    switch (rc) {
        case TG_ERR_COMPILE: return ErrorKind::Compile;
        case TG_ERR_NO_DEVICE: return ErrorKind::NoDevice;
        case TG_ERR_DIMENSION_MISMATCH: return ErrorKind::DimensionMismatch;
        case TG_ERR_KERNEL_NOT_FOUND: return ErrorKind::KernelNotFound;
        case TG_ERR_INVALID_ARGUMENT: return ErrorKind::InvalidArgument;
        case TG_ERR_UNSUPPORTED: return ErrorKind::Unsupported;
        default: return ErrorKind::Driver;
    }
}

inline void check(int rc) {
    if (rc != TG_OK) throw HipError(kind_of(rc), tg_last_error());
}

[[noreturn]] inline void mismatch(const std::string& msg) {
    throw HipError(ErrorKind::DimensionMismatch, msg);
}

template <typename T>
struct DType;
template <>
struct DType<float> {
    static constexpr tg_dtype value = TG_F32;
};
template <>
struct DType<double> {
    static constexpr tg_dtype value = TG_F64;
};
template <>
struct DType<int32_t> {
    static constexpr tg_dtype value = TG_I32;
};
template <>
struct DType<int64_t> {
    static constexpr tg_dtype value = TG_I64;
};

}  // namespace detail

// ---------------------------------------------------------------------------
// Semiring tags (crates/tropical-gemm/src/types/max_plus.rs, min_plus.rs,
// max_mul.rs): Scalar is f32, f64, i32 or i64.
// ---------------------------------------------------------------------------

template <typename T>
struct TropicalMaxPlus {
    using Scalar = T;
    static constexpr tg_semiring semiring = TG_MAXPLUS;
};
template <typename T>
struct TropicalMinPlus {
    using Scalar = T;
    static constexpr tg_semiring semiring = TG_MINPLUS;
};
template <typename T>
struct TropicalMaxMul {
    using Scalar = T;
    static constexpr tg_semiring semiring = TG_MAXMUL;
};

// Argmax index type of the GPU path (memory.rs:10).
using ArgmaxIndex = int32_t;

// ---------------------------------------------------------------------------
// Devices and contexts (context.rs:66-151, lib.rs:57-133)
// ---------------------------------------------------------------------------

// Replaces cuda_device_count (lib.rs:60-63).
inline size_t hip_device_count() {
    int n = 0;
    detail::check(tg_device_count(&n));
    return size_t(n);
}

class HipContext {
  public:
    // CudaContext::new_on_device: validates the ordinal and initialises the
    // device.  There is no runtime kernel compilation step.
    static HipContext new_on_device(size_t device_id) {
        detail::check(tg_context_init(int(device_id)));
        return HipContext(int(device_id));
    }
    // CudaContext::new (device 0).
    static HipContext create() { return new_on_device(0); }

    int device_id() const noexcept { return device_; }
    std::string device_name() const {
        char buf[256];
        detail::check(tg_device_name(device_, buf, sizeof buf));
        return buf;
    }
    void synchronize() const { detail::check(tg_synchronize(device_)); }

  private:
    explicit HipContext(int d) : device_(d) {}
    int device_;
};

// lib.rs:79-122: one context per device, created once under a lock and kept
// for the life of the process.
inline const HipContext& get_context_for_device(size_t device_id) {
    static std::mutex mu;
    static std::map<size_t, std::unique_ptr<HipContext>> contexts;
    const size_t n = hip_device_count();
    if (device_id >= n)
        detail::mismatch("Device " + std::to_string(device_id) + " not available (only " +
                         std::to_string(n) + " HIP device(s) found)");
    std::lock_guard<std::mutex> lk(mu);
    auto it = contexts.find(device_id);
    if (it == contexts.end())
        it = contexts
                 .emplace(device_id, std::make_unique<HipContext>(HipContext::new_on_device(device_id)))
                 .first;
    return *it->second;
}

// lib.rs:131-133.
inline const HipContext& get_global_context() { return get_context_for_device(0); }

// ---------------------------------------------------------------------------
// Owning device buffer and the device-matrix types (memory.rs:31-573)
// ---------------------------------------------------------------------------

namespace detail {

template <typename T>
class DeviceBuffer {
  public:
    DeviceBuffer() = default;
    DeviceBuffer(int device, size_t n) : device_(device), n_(n) {
        check(tg_malloc(device, &ptr_, n * sizeof(T)));
    }
    ~DeviceBuffer() {
        if (ptr_) (void)tg_free(device_, ptr_);
    }
    DeviceBuffer(DeviceBuffer&& o) noexcept : device_(o.device_), ptr_(o.ptr_), n_(o.n_) {
        o.ptr_ = nullptr;
        o.n_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            if (ptr_) (void)tg_free(device_, ptr_);
            device_ = o.device_;
            ptr_ = o.ptr_;
            n_ = o.n_;
            o.ptr_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    T* get() const noexcept { return static_cast<T*>(ptr_); }
    size_t size() const noexcept { return n_; }
    int device() const noexcept { return device_; }

    void upload(const T* src, size_t n) { check(tg_memcpy_htod(device_, ptr_, src, n * sizeof(T))); }
    void zero() { check(tg_memset_zero(device_, ptr_, n_ * sizeof(T), nullptr)); }
    std::vector<T> download() const {
        std::vector<T> out(n_);
        if (n_) check(tg_memcpy_dtoh(device_, out.data(), ptr_, n_ * sizeof(T)));
        return out;
    }

  private:
    int device_ = 0;
    void* ptr_ = nullptr;
    size_t n_ = 0;
};

template <typename T>
void validate_dims(size_t len, size_t rows, size_t cols) {  // memory.rs:16-25
    if (len != rows * cols)
        mismatch("Expected " + std::to_string(rows * cols) + " elements, got " + std::to_string(len));
}

template <typename T>
std::vector<T> row_to_col(const T* data, size_t rows, size_t cols) {
    std::vector<T> out(rows * cols);
    for (size_t i = 0; i < rows; ++i)
        for (size_t j = 0; j < cols; ++j) out[i + j * rows] = data[i * cols + j];
    return out;
}

template <typename T>
std::vector<T> col_to_row(const std::vector<T>& data, size_t rows, size_t cols) {
    std::vector<T> out(rows * cols);
    for (size_t i = 0; i < rows; ++i)
        for (size_t j = 0; j < cols; ++j) out[i * cols + j] = data[i + j * rows];
    return out;
}

}  // namespace detail

// A column-major matrix in device memory (leading dimension = rows).
template <typename T>
class GpuMatrix {
  public:
    static GpuMatrix from_host(const HipContext& ctx, const T* data, size_t len, size_t rows, size_t cols) {
        detail::validate_dims<T>(len, rows, cols);
        GpuMatrix m(ctx, rows, cols);
        m.buf_.upload(data, len);
        return m;
    }
    static GpuMatrix from_host(const HipContext& ctx, const std::vector<T>& data, size_t rows, size_t cols) {
        return from_host(ctx, data.data(), data.size(), rows, cols);
    }
    // memory.rs:63-86 (deprecated in the reference: transposes on the host).
    static GpuMatrix from_host_row_major(const HipContext& ctx, const std::vector<T>& data, size_t rows,
                                         size_t cols) {
        detail::validate_dims<T>(data.size(), rows, cols);
        auto cm = detail::row_to_col(data.data(), rows, cols);
        return from_host(ctx, cm, rows, cols);
    }
    static GpuMatrix from_host_col_major(const HipContext& ctx, const std::vector<T>& data, size_t rows,
                                         size_t cols) {
        return from_host(ctx, data, rows, cols);
    }
    // Zero-initialised, like alloc_zeros (memory.rs:100-110).
    static GpuMatrix alloc(const HipContext& ctx, size_t rows, size_t cols) {
        GpuMatrix m(ctx, rows, cols);
        m.buf_.zero();
        return m;
    }

    std::vector<T> to_host(const HipContext&) const { return buf_.download(); }
    std::vector<T> to_host_row_major(const HipContext& ctx) const {
        return detail::col_to_row(to_host(ctx), rows_, cols_);
    }
    std::vector<T> to_host_col_major(const HipContext& ctx) const { return to_host(ctx); }

    size_t rows() const noexcept { return rows_; }
    size_t cols() const noexcept { return cols_; }
    size_t ld() const noexcept { return rows_; }
    T* device_ptr() const noexcept { return buf_.get(); }
    int device() const noexcept { return buf_.device(); }

  private:
    GpuMatrix(const HipContext& ctx, size_t rows, size_t cols)
        : buf_(ctx.device_id(), rows * cols), rows_(rows), cols_(cols) {}
    detail::DeviceBuffer<T> buf_;
    size_t rows_, cols_;
};

// Result matrix plus argmax indices (memory.rs:188-257).
template <typename T>
class GpuMatrixWithArgmax {
  public:
    static GpuMatrixWithArgmax alloc(const HipContext& ctx, size_t rows, size_t cols) {
        return GpuMatrixWithArgmax(GpuMatrix<T>::alloc(ctx, rows, cols),
                                   GpuMatrix<ArgmaxIndex>::alloc(ctx, rows, cols));
    }
    size_t rows() const noexcept { return matrix.rows(); }
    size_t cols() const noexcept { return matrix.cols(); }
    std::vector<T> matrix_to_host(const HipContext& ctx) const { return matrix.to_host(ctx); }
    std::vector<ArgmaxIndex> argmax_to_host(const HipContext& ctx) const { return argmax.to_host(ctx); }
    std::vector<T> matrix_to_host_row_major(const HipContext& ctx) const { return matrix.to_host_row_major(ctx); }
    std::vector<ArgmaxIndex> argmax_to_host_row_major(const HipContext& ctx) const {
        return argmax.to_host_row_major(ctx);
    }
    std::vector<T> matrix_to_host_col_major(const HipContext& ctx) const { return matrix.to_host(ctx); }
    std::vector<ArgmaxIndex> argmax_to_host_col_major(const HipContext& ctx) const { return argmax.to_host(ctx); }
    std::pair<GpuMatrix<T>, GpuMatrix<ArgmaxIndex>> into_parts() && {
        return {std::move(matrix), std::move(argmax)};
    }

    GpuMatrix<T> matrix;
    GpuMatrix<ArgmaxIndex> argmax;

  private:
    GpuMatrixWithArgmax(GpuMatrix<T>&& m, GpuMatrix<ArgmaxIndex>&& a) : matrix(std::move(m)), argmax(std::move(a)) {}
};

// Non-owning views of caller memory (memory.rs:274-454), e.g. DLPack tensors.
template <typename T>
class ExternalGpuMemory {
  public:
    ExternalGpuMemory(T* ptr, size_t len) : ptr_(ptr), len_(len) {}
    T* device_ptr() const noexcept { return ptr_; }
    size_t len() const noexcept { return len_; }
    bool is_empty() const noexcept { return len_ == 0; }

  private:
    T* ptr_;
    size_t len_;
};

template <typename T>
class ExternalGpuMatrix {
  public:
    ExternalGpuMatrix(const T* ptr, size_t rows, size_t cols) : ptr_(ptr), rows_(rows), cols_(cols) {}
    const T* device_ptr() const noexcept { return ptr_; }
    size_t rows() const noexcept { return rows_; }
    size_t cols() const noexcept { return cols_; }
    size_t len() const noexcept { return rows_ * cols_; }
    bool is_empty() const noexcept { return len() == 0; }

  private:
    const T* ptr_;
    size_t rows_, cols_;
};

template <typename T>
class ExternalGpuTensor3 {
  public:
    ExternalGpuTensor3(const T* ptr, size_t batch, size_t rows, size_t cols, size_t stride)
        : ptr_(ptr), batch_(batch), rows_(rows), cols_(cols), stride_(stride) {}
    static ExternalGpuTensor3 from_raw_contiguous(const T* ptr, size_t batch, size_t rows, size_t cols) {
        return ExternalGpuTensor3(ptr, batch, rows, cols, rows * cols);
    }
    const T* device_ptr() const noexcept { return ptr_; }
    size_t batch() const noexcept { return batch_; }
    size_t rows() const noexcept { return rows_; }
    size_t cols() const noexcept { return cols_; }
    size_t stride() const noexcept { return stride_; }
    size_t len() const noexcept { return batch_ * stride_; }
    bool is_empty() const noexcept { return len() == 0; }
    bool is_contiguous() const noexcept { return stride_ == rows_ * cols_; }

  private:
    const T* ptr_;
    size_t batch_, rows_, cols_, stride_;
};

// Batched device tensor, row-major per batch item (memory.rs:459-573).
template <typename T>
class GpuTensor3 {
  public:
    static GpuTensor3 alloc(const HipContext& ctx, size_t batch, size_t rows, size_t cols) {
        GpuTensor3 t(ctx, batch, rows, cols);
        t.buf_.zero();
        return t;
    }
    std::vector<T> to_host(const HipContext&) const { return buf_.download(); }
    size_t batch() const noexcept { return batch_; }
    size_t rows() const noexcept { return rows_; }
    size_t cols() const noexcept { return cols_; }
    size_t stride() const noexcept { return rows_ * cols_; }
    T* device_ptr() const noexcept { return buf_.get(); }

  private:
    GpuTensor3(const HipContext& ctx, size_t batch, size_t rows, size_t cols)
        : buf_(ctx.device_id(), batch * rows * cols), batch_(batch), rows_(rows), cols_(cols) {}
    detail::DeviceBuffer<T> buf_;
    size_t batch_, rows_, cols_;
};

template <typename T>
class GpuTensor3WithArgmax {
  public:
    static GpuTensor3WithArgmax alloc(const HipContext& ctx, size_t batch, size_t rows, size_t cols) {
        return GpuTensor3WithArgmax(GpuTensor3<T>::alloc(ctx, batch, rows, cols),
                                    GpuTensor3<ArgmaxIndex>::alloc(ctx, batch, rows, cols));
    }
    size_t batch() const noexcept { return tensor.batch(); }
    size_t rows() const noexcept { return tensor.rows(); }
    size_t cols() const noexcept { return tensor.cols(); }
    std::vector<T> tensor_to_host(const HipContext& ctx) const { return tensor.to_host(ctx); }
    std::vector<ArgmaxIndex> argmax_to_host(const HipContext& ctx) const { return argmax.to_host(ctx); }
    std::pair<GpuTensor3<T>, GpuTensor3<ArgmaxIndex>> into_parts() && {
        return {std::move(tensor), std::move(argmax)};
    }

    GpuTensor3<T> tensor;
    GpuTensor3<ArgmaxIndex> argmax;

  private:
    GpuTensor3WithArgmax(GpuTensor3<T>&& t, GpuTensor3<ArgmaxIndex>&& a)
        : tensor(std::move(t)), argmax(std::move(a)) {}
};

// ---------------------------------------------------------------------------
// Kernel launch traits (CudaKernel / CudaKernelWithArgmax, kernels.rs:12-360)
// ---------------------------------------------------------------------------

// launch_gemm: C = A (x) B on column-major device matrices; blocks until done
// (the reference synchronises after every launch, kernels.rs:65).
template <class S>
void launch_gemm(const HipContext& ctx, const GpuMatrix<typename S::Scalar>& a,
                 const GpuMatrix<typename S::Scalar>& b, GpuMatrix<typename S::Scalar>& c) {
    using T = typename S::Scalar;
    detail::check(tg_gemm(ctx.device_id(), S::semiring, detail::DType<T>::value, TG_COL_MAJOR,
                          a.device_ptr(), b.device_ptr(), c.device_ptr(), nullptr, int64_t(a.rows()),
                          int64_t(b.cols()), int64_t(a.cols()), nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
}

template <class S>
void launch_gemm_with_argmax(const HipContext& ctx, const GpuMatrix<typename S::Scalar>& a,
                             const GpuMatrix<typename S::Scalar>& b,
                             GpuMatrixWithArgmax<typename S::Scalar>& c) {
    using T = typename S::Scalar;
    detail::check(tg_gemm(ctx.device_id(), S::semiring, detail::DType<T>::value, TG_COL_MAJOR,
                          a.device_ptr(), b.device_ptr(), c.matrix.device_ptr(), c.argmax.device_ptr(),
                          int64_t(a.rows()), int64_t(b.cols()), int64_t(a.cols()), nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
}

// ---------------------------------------------------------------------------
// Public entry points (lib.rs:153-1067)
// ---------------------------------------------------------------------------

namespace detail {
template <typename T>
void validate_gemm_input(size_t a_len, size_t b_len, size_t m, size_t k, size_t n) {  // lib.rs:153-169
    if (a_len != m * k)
        mismatch("A: expected " + std::to_string(m * k) + " elements, got " + std::to_string(a_len));
    if (b_len != k * n)
        mismatch("B: expected " + std::to_string(k * n) + " elements, got " + std::to_string(b_len));
}
}  // namespace detail

// One-shot C = A (x) B; A is m x k, B is k x n, all column-major (lib.rs:221-243).
template <class S>
std::vector<typename S::Scalar> tropical_matmul_gpu(const std::vector<typename S::Scalar>& a, size_t m,
                                                    size_t k, const std::vector<typename S::Scalar>& b,
                                                    size_t n) {
    using T = typename S::Scalar;
    detail::validate_gemm_input<T>(a.size(), b.size(), m, k, n);
    const HipContext& ctx = get_global_context();
    auto a_gpu = GpuMatrix<T>::from_host(ctx, a, m, k);
    auto b_gpu = GpuMatrix<T>::from_host(ctx, b, k, n);
    auto c_gpu = GpuMatrix<T>::alloc(ctx, m, n);
    launch_gemm<S>(ctx, a_gpu, b_gpu, c_gpu);
    return c_gpu.to_host(ctx);
}

// Persistent-context product into an existing C (lib.rs:256-284).
template <class S>
void tropical_gemm_gpu(const HipContext& ctx, const GpuMatrix<typename S::Scalar>& a,
                       const GpuMatrix<typename S::Scalar>& b, GpuMatrix<typename S::Scalar>& c) {
    if (a.cols() != b.rows())
        detail::mismatch("A.cols (" + std::to_string(a.cols()) + ") != B.rows (" + std::to_string(b.rows()) + ")");
    if (c.rows() != a.rows() || c.cols() != b.cols())
        detail::mismatch("C dimensions (" + std::to_string(c.rows()) + ", " + std::to_string(c.cols()) +
                         ") don't match A×B (" + std::to_string(a.rows()) + ", " + std::to_string(b.cols()) + ")");
    launch_gemm<S>(ctx, a, b, c);
}

// lib.rs:289-309.
template <class S>
std::vector<typename S::Scalar> tropical_matmul_gpu_with_ctx(const HipContext& ctx,
                                                             const std::vector<typename S::Scalar>& a, size_t m,
                                                             size_t k, const std::vector<typename S::Scalar>& b,
                                                             size_t n) {
    using T = typename S::Scalar;
    detail::validate_gemm_input<T>(a.size(), b.size(), m, k, n);
    auto a_gpu = GpuMatrix<T>::from_host(ctx, a, m, k);
    auto b_gpu = GpuMatrix<T>::from_host(ctx, b, k, n);
    auto c_gpu = GpuMatrix<T>::alloc(ctx, m, n);
    launch_gemm<S>(ctx, a_gpu, b_gpu, c_gpu);
    return c_gpu.to_host(ctx);
}

// (values, argmax), both column-major (lib.rs:354-379).
template <class S>
std::pair<std::vector<typename S::Scalar>, std::vector<ArgmaxIndex>> tropical_matmul_gpu_with_ctx_and_argmax(
    const HipContext& ctx, const std::vector<typename S::Scalar>& a, size_t m, size_t k,
    const std::vector<typename S::Scalar>& b, size_t n) {
    using T = typename S::Scalar;
    detail::validate_gemm_input<T>(a.size(), b.size(), m, k, n);
    auto a_gpu = GpuMatrix<T>::from_host(ctx, a, m, k);
    auto b_gpu = GpuMatrix<T>::from_host(ctx, b, k, n);
    auto c = GpuMatrixWithArgmax<T>::alloc(ctx, m, n);
    launch_gemm_with_argmax<S>(ctx, a_gpu, b_gpu, c);
    return {c.matrix_to_host(ctx), c.argmax_to_host(ctx)};
}

template <class S>
std::pair<std::vector<typename S::Scalar>, std::vector<ArgmaxIndex>> tropical_matmul_gpu_with_argmax(
    const std::vector<typename S::Scalar>& a, size_t m, size_t k, const std::vector<typename S::Scalar>& b,
    size_t n) {
    detail::validate_gemm_input<typename S::Scalar>(a.size(), b.size(), m, k, n);  // before the device
    return tropical_matmul_gpu_with_ctx_and_argmax<S>(get_global_context(), a, m, k, b, n);
}

// lib.rs:392-420.
template <class S>
void tropical_gemm_gpu_with_argmax(const HipContext& ctx, const GpuMatrix<typename S::Scalar>& a,
                                   const GpuMatrix<typename S::Scalar>& b,
                                   GpuMatrixWithArgmax<typename S::Scalar>& c) {
    if (a.cols() != b.rows())
        detail::mismatch("A.cols (" + std::to_string(a.cols()) + ") != B.rows (" + std::to_string(b.rows()) + ")");
    if (c.rows() != a.rows() || c.cols() != b.cols())
        detail::mismatch("C dimensions (" + std::to_string(c.rows()) + ", " + std::to_string(c.cols()) +
                         ") don't match A×B (" + std::to_string(a.rows()) + ", " + std::to_string(b.cols()) + ")");
    launch_gemm_with_argmax<S>(ctx, a, b, c);
}

namespace detail {
template <typename T>
void validate_batch(const std::vector<std::vector<T>>& a, const std::vector<std::vector<T>>& b, size_t m,
                    size_t k, size_t n) {  // lib.rs:494-528
    if (a.size() != b.size())
        mismatch("Batch sizes must match: A has " + std::to_string(a.size()) + " matrices, B has " +
                 std::to_string(b.size()));
    for (size_t i = 0; i < a.size(); ++i) {
        if (a[i].size() != m * k)
            mismatch("A[" + std::to_string(i) + "] dimensions mismatch: expected " + std::to_string(m * k) +
                     ", got " + std::to_string(a[i].size()));
        if (b[i].size() != k * n)
            mismatch("B[" + std::to_string(i) + "] dimensions mismatch: expected " + std::to_string(k * n) +
                     ", got " + std::to_string(b[i].size()));
    }
}

// Runs the whole batch as one strided-batched launch (the reference loops
// over single products with per-item copies, lib.rs:533-541).
template <class S>
void batched_launch(const HipContext& ctx, const std::vector<typename S::Scalar>& a_flat,
                    const std::vector<typename S::Scalar>& b_flat, size_t batch, size_t m, size_t k, size_t n,
                    std::vector<typename S::Scalar>* c_out, std::vector<ArgmaxIndex>* am_out) {
    using T = typename S::Scalar;
    DeviceBuffer<T> a(ctx.device_id(), a_flat.size()), b(ctx.device_id(), b_flat.size());
    DeviceBuffer<T> c(ctx.device_id(), batch * m * n);
    DeviceBuffer<ArgmaxIndex> am;
    if (am_out) am = DeviceBuffer<ArgmaxIndex>(ctx.device_id(), batch * m * n);
    a.upload(a_flat.data(), a_flat.size());
    b.upload(b_flat.data(), b_flat.size());
    check(tg_gemm_strided_batched(ctx.device_id(), S::semiring, DType<T>::value, TG_COL_MAJOR, a.get(), b.get(),
                                  c.get(), am_out ? am.get() : nullptr, int64_t(batch), int64_t(m), int64_t(n),
                                  int64_t(k), int64_t(m * k), int64_t(k * n), int64_t(m * n), nullptr));
    check(tg_stream_synchronize(ctx.device_id(), nullptr));
    *c_out = c.download();
    if (am_out) *am_out = am.download();
}
}  // namespace detail

// lib.rs:486-544.
template <class S>
std::vector<std::vector<typename S::Scalar>> tropical_matmul_gpu_batched(
    const std::vector<std::vector<typename S::Scalar>>& a_batch,
    const std::vector<std::vector<typename S::Scalar>>& b_batch, size_t m, size_t k, size_t n) {
    using T = typename S::Scalar;
    detail::validate_batch(a_batch, b_batch, m, k, n);
    const size_t batch = a_batch.size();
    if (batch == 0) return {};
    std::vector<T> a, b, c;
    for (const auto& x : a_batch) a.insert(a.end(), x.begin(), x.end());
    for (const auto& x : b_batch) b.insert(b.end(), x.begin(), x.end());
    detail::batched_launch<S>(get_global_context(), a, b, batch, m, k, n, &c, nullptr);
    std::vector<std::vector<T>> out(batch);
    for (size_t t = 0; t < batch; ++t) out[t].assign(c.begin() + t * m * n, c.begin() + (t + 1) * m * n);
    return out;
}

// lib.rs:563-616: contiguous A (batch*m*k), B (batch*k*n) -> C (batch*m*n).
template <class S>
std::vector<typename S::Scalar> tropical_matmul_gpu_strided_batched(const std::vector<typename S::Scalar>& a,
                                                                    const std::vector<typename S::Scalar>& b,
                                                                    size_t batch_size, size_t m, size_t k, size_t n) {
    using T = typename S::Scalar;
    if (a.size() != batch_size * m * k)
        detail::mismatch("A size mismatch: expected " + std::to_string(batch_size * m * k) + ", got " +
                         std::to_string(a.size()));
    if (b.size() != batch_size * k * n)
        detail::mismatch("B size mismatch: expected " + std::to_string(batch_size * k * n) + ", got " +
                         std::to_string(b.size()));
    if (batch_size == 0) return {};
    std::vector<T> c;
    detail::batched_launch<S>(get_global_context(), a, b, batch_size, m, k, n, &c, nullptr);
    return c;
}

// lib.rs:1007-1067.
template <class S>
std::vector<std::pair<std::vector<typename S::Scalar>, std::vector<ArgmaxIndex>>>
tropical_matmul_gpu_batched_with_argmax(const std::vector<std::vector<typename S::Scalar>>& a_batch,
                                        const std::vector<std::vector<typename S::Scalar>>& b_batch, size_t m,
                                        size_t k, size_t n) {
    using T = typename S::Scalar;
    detail::validate_batch(a_batch, b_batch, m, k, n);
    const size_t batch = a_batch.size();
    if (batch == 0) return {};
    std::vector<T> a, b, c;
    std::vector<ArgmaxIndex> am;
    for (const auto& x : a_batch) a.insert(a.end(), x.begin(), x.end());
    for (const auto& x : b_batch) b.insert(b.end(), x.begin(), x.end());
    detail::batched_launch<S>(get_global_context(), a, b, batch, m, k, n, &c, &am);
    std::vector<std::pair<std::vector<T>, std::vector<ArgmaxIndex>>> out(batch);
    for (size_t t = 0; t < batch; ++t) {
        out[t].first.assign(c.begin() + t * m * n, c.begin() + (t + 1) * m * n);
        out[t].second.assign(am.begin() + t * m * n, am.begin() + (t + 1) * m * n);
    }
    return out;
}

// ---------------------------------------------------------------------------
// Row-major launchers on caller device memory (kernels.rs:388-550), as used
// by the DLPack path: C = A (x) B with A (m x k), B (k x n) row-major.
// ---------------------------------------------------------------------------

template <class S>
GpuMatrixWithArgmax<typename S::Scalar> launch_gemm_external_with_argmax(
    const HipContext& ctx, const ExternalGpuMatrix<typename S::Scalar>& a,
    const ExternalGpuMatrix<typename S::Scalar>& b, size_t m, size_t k, size_t n) {
    using T = typename S::Scalar;
    // The result buffers hold C and argmax row-major (m x n), like the
    // reference's swapped launch into an (m, n) allocation.
    auto c = GpuMatrixWithArgmax<T>::alloc(ctx, m, n);
    detail::check(tg_gemm(ctx.device_id(), S::semiring, detail::DType<T>::value, TG_ROW_MAJOR, a.device_ptr(),
                          b.device_ptr(), c.matrix.device_ptr(), c.argmax.device_ptr(), int64_t(m), int64_t(n),
                          int64_t(k), nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
    return c;
}

template <class S>
GpuMatrix<typename S::Scalar> launch_gemm_external(const HipContext& ctx,
                                                   const ExternalGpuMatrix<typename S::Scalar>& a,
                                                   const ExternalGpuMatrix<typename S::Scalar>& b, size_t m,
                                                   size_t k, size_t n) {
    using T = typename S::Scalar;
    auto c = GpuMatrix<T>::alloc(ctx, m, n);
    detail::check(tg_gemm(ctx.device_id(), S::semiring, detail::DType<T>::value, TG_ROW_MAJOR, a.device_ptr(),
                          b.device_ptr(), c.device_ptr(), nullptr, int64_t(m), int64_t(n), int64_t(k), nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
    return c;
}

template <class S>
GpuTensor3WithArgmax<typename S::Scalar> launch_gemm_external_batched_with_argmax(
    const HipContext& ctx, const ExternalGpuTensor3<typename S::Scalar>& a,
    const ExternalGpuTensor3<typename S::Scalar>& b, size_t batch, size_t m, size_t k, size_t n) {
    using T = typename S::Scalar;
    auto c = GpuTensor3WithArgmax<T>::alloc(ctx, batch, m, n);
    detail::check(tg_gemm_strided_batched(ctx.device_id(), S::semiring, detail::DType<T>::value, TG_ROW_MAJOR,
                                          a.device_ptr(), b.device_ptr(), c.tensor.device_ptr(),
                                          c.argmax.device_ptr(), int64_t(batch), int64_t(m), int64_t(n),
                                          int64_t(k), int64_t(a.stride()), int64_t(b.stride()), int64_t(m * n),
                                          nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
    return c;
}

// The reference's f32-only names (kernels.rs:388-550), semiring chosen at run
// time as it is by kernel name there.
inline GpuMatrixWithArgmax<float> launch_gemm_external_with_argmax_f32(const HipContext& ctx, tg_semiring sr,
                                                                       const ExternalGpuMatrix<float>& a,
                                                                       const ExternalGpuMatrix<float>& b,
                                                                       size_t m, size_t k, size_t n) {
    switch (sr) {
        case TG_MINPLUS: return launch_gemm_external_with_argmax<TropicalMinPlus<float>>(ctx, a, b, m, k, n);
        case TG_MAXMUL: return launch_gemm_external_with_argmax<TropicalMaxMul<float>>(ctx, a, b, m, k, n);
        default: return launch_gemm_external_with_argmax<TropicalMaxPlus<float>>(ctx, a, b, m, k, n);
    }
}
inline GpuMatrix<float> launch_gemm_external_f32(const HipContext& ctx, tg_semiring sr,
                                                 const ExternalGpuMatrix<float>& a, const ExternalGpuMatrix<float>& b,
                                                 size_t m, size_t k, size_t n) {
    switch (sr) {
        case TG_MINPLUS: return launch_gemm_external<TropicalMinPlus<float>>(ctx, a, b, m, k, n);
        case TG_MAXMUL: return launch_gemm_external<TropicalMaxMul<float>>(ctx, a, b, m, k, n);
        default: return launch_gemm_external<TropicalMaxPlus<float>>(ctx, a, b, m, k, n);
    }
}
inline GpuTensor3WithArgmax<float> launch_gemm_external_batched_with_argmax_f32(
    const HipContext& ctx, tg_semiring sr, const ExternalGpuTensor3<float>& a, const ExternalGpuTensor3<float>& b,
    size_t batch, size_t m, size_t k, size_t n) {
    switch (sr) {
        case TG_MINPLUS:
            return launch_gemm_external_batched_with_argmax<TropicalMinPlus<float>>(ctx, a, b, batch, m, k, n);
        case TG_MAXMUL:
            return launch_gemm_external_batched_with_argmax<TropicalMaxMul<float>>(ctx, a, b, batch, m, k, n);
        default:
            return launch_gemm_external_batched_with_argmax<TropicalMaxPlus<float>>(ctx, a, b, batch, m, k, n);
    }
}

// ---------------------------------------------------------------------------
// Backward (lib.rs:654-1002)
// ---------------------------------------------------------------------------

// Host scatter over column-major data, exactly the reference's loop order
// (lib.rs:654-740): j outer, i inner; indices outside [0, k) are skipped.
// Deterministic, so results equal the reference bit for bit.  Size mismatches
// throw InvalidArgument where the reference asserts.
template <typename T>
std::vector<T> tropical_backward_a_gpu(const std::vector<T>& grad_c, const std::vector<ArgmaxIndex>& argmax, size_t m,
                                       size_t k, size_t n) {
    if (grad_c.size() != m * n) throw HipError(ErrorKind::InvalidArgument, "grad_c size mismatch");
    if (argmax.size() != m * n) throw HipError(ErrorKind::InvalidArgument, "argmax size mismatch");
    std::vector<T> grad_a(m * k, T{});
    for (size_t j = 0; j < n; ++j)
        for (size_t i = 0; i < m; ++i) {
            const size_t idx = i + j * m;
            const int64_t kk = argmax[idx];
            if (kk >= 0 && size_t(kk) < k) grad_a[i + size_t(kk) * m] += grad_c[idx];
        }
    return grad_a;
}

template <typename T>
std::vector<T> tropical_backward_b_gpu(const std::vector<T>& grad_c, const std::vector<ArgmaxIndex>& argmax, size_t m,
                                       size_t k, size_t n) {
    if (grad_c.size() != m * n) throw HipError(ErrorKind::InvalidArgument, "grad_c size mismatch");
    if (argmax.size() != m * n) throw HipError(ErrorKind::InvalidArgument, "argmax size mismatch");
    std::vector<T> grad_b(k * n, T{});
    for (size_t j = 0; j < n; ++j)
        for (size_t i = 0; i < m; ++i) {
            const size_t idx = i + j * m;
            const int64_t kk = argmax[idx];
            if (kk >= 0 && size_t(kk) < k) grad_b[size_t(kk) + j * k] += grad_c[idx];
        }
    return grad_b;
}

template <typename T>
std::vector<std::vector<T>> tropical_backward_a_gpu_batched(const std::vector<std::vector<T>>& grad_c_batch,
                                                            const std::vector<std::vector<ArgmaxIndex>>& argmax_batch,
                                                            size_t m, size_t k, size_t n) {
    if (grad_c_batch.size() != argmax_batch.size())
        throw HipError(ErrorKind::InvalidArgument, "batch sizes must match");
    std::vector<std::vector<T>> out;
    out.reserve(grad_c_batch.size());
    for (size_t t = 0; t < grad_c_batch.size(); ++t)
        out.push_back(tropical_backward_a_gpu(grad_c_batch[t], argmax_batch[t], m, k, n));
    return out;
}

template <typename T>
std::vector<std::vector<T>> tropical_backward_b_gpu_batched(const std::vector<std::vector<T>>& grad_c_batch,
                                                            const std::vector<std::vector<ArgmaxIndex>>& argmax_batch,
                                                            size_t m, size_t k, size_t n) {
    if (grad_c_batch.size() != argmax_batch.size())
        throw HipError(ErrorKind::InvalidArgument, "batch sizes must match");
    std::vector<std::vector<T>> out;
    out.reserve(grad_c_batch.size());
    for (size_t t = 0; t < grad_c_batch.size(); ++t)
        out.push_back(tropical_backward_b_gpu(grad_c_batch[t], argmax_batch[t], m, k, n));
    return out;
}

// Device scatter with the HIP kernels (lib.rs:841-942): grad_c (m x n) and
// argmax column-major on the device; returns grad_A (m x k) / grad_B (k x n).
// f32 and f64; sums of several terms are accumulated in an unspecified order.
template <typename T>
GpuMatrix<T> tropical_backward_a_gpu_kernel(const HipContext& ctx, const GpuMatrix<T>& grad_c,
                                            const GpuMatrix<ArgmaxIndex>& argmax, size_t m, size_t k, size_t n) {
    static_assert(std::is_floating_point<T>::value, "gradients are f32 or f64");
    if (grad_c.rows() != m || grad_c.cols() != n || argmax.rows() != m || argmax.cols() != n)
        detail::mismatch("grad_c/argmax must be " + std::to_string(m) + "x" + std::to_string(n));
    auto grad_a = GpuMatrix<T>::alloc(ctx, m, k);
    detail::check(tg_backward_a(ctx.device_id(), detail::DType<T>::value, TG_COL_MAJOR, grad_c.device_ptr(),
                                argmax.device_ptr(), grad_a.device_ptr(), int64_t(m), int64_t(n), int64_t(k),
                                nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
    return grad_a;
}

template <typename T>
GpuMatrix<T> tropical_backward_b_gpu_kernel(const HipContext& ctx, const GpuMatrix<T>& grad_c,
                                            const GpuMatrix<ArgmaxIndex>& argmax, size_t m, size_t k, size_t n) {
    static_assert(std::is_floating_point<T>::value, "gradients are f32 or f64");
    if (grad_c.rows() != m || grad_c.cols() != n || argmax.rows() != m || argmax.cols() != n)
        detail::mismatch("grad_c/argmax must be " + std::to_string(m) + "x" + std::to_string(n));
    auto grad_b = GpuMatrix<T>::alloc(ctx, k, n);
    detail::check(tg_backward_b(ctx.device_id(), detail::DType<T>::value, TG_COL_MAJOR, grad_c.device_ptr(),
                                argmax.device_ptr(), grad_b.device_ptr(), int64_t(m), int64_t(n), int64_t(k),
                                nullptr));
    detail::check(tg_stream_synchronize(ctx.device_id(), nullptr));
    return grad_b;
}

// Upload, device scatter, download (lib.rs:950-1002, tropical_backward_*_gpu_cuda).
inline std::vector<float> tropical_backward_a_gpu_hip(const std::vector<float>& grad_c,
                                                      const std::vector<ArgmaxIndex>& argmax, size_t m, size_t k,
                                                      size_t n) {
    const HipContext& ctx = get_global_context();
    auto g = GpuMatrix<float>::from_host(ctx, grad_c, m, n);
    auto am = GpuMatrix<ArgmaxIndex>::from_host(ctx, argmax, m, n);
    return tropical_backward_a_gpu_kernel<float>(ctx, g, am, m, k, n).to_host(ctx);
}

inline std::vector<float> tropical_backward_b_gpu_hip(const std::vector<float>& grad_c,
                                                      const std::vector<ArgmaxIndex>& argmax, size_t m, size_t k,
                                                      size_t n) {
    const HipContext& ctx = get_global_context();
    auto g = GpuMatrix<float>::from_host(ctx, grad_c, m, n);
    auto am = GpuMatrix<ArgmaxIndex>::from_host(ctx, argmax, m, n);
    return tropical_backward_b_gpu_kernel<float>(ctx, g, am, m, k, n).to_host(ctx);
}

// ---------------------------------------------------------------------------
// Host matrices for GpuMat interop: the column-major Mat / MatRef /
// MatWithArgmax of the CPU crate (crates/tropical-gemm/src/mat/), reduced to
// what the GPU types exchange with them.
// ---------------------------------------------------------------------------

template <class S>
class Mat {
  public:
    using Scalar = typename S::Scalar;
    Mat() = default;
    static Mat from_col_major(const std::vector<Scalar>& data, size_t nrows, size_t ncols) {
        detail::validate_dims<Scalar>(data.size(), nrows, ncols);
        return Mat(data, nrows, ncols);
    }
    static Mat from_row_major(const std::vector<Scalar>& data, size_t nrows, size_t ncols) {
        detail::validate_dims<Scalar>(data.size(), nrows, ncols);
        return Mat(detail::row_to_col(data.data(), nrows, ncols), nrows, ncols);
    }
    template <class F>
    static Mat from_fn(size_t nrows, size_t ncols, F f) {
        std::vector<Scalar> d(nrows * ncols);
        for (size_t j = 0; j < ncols; ++j)
            for (size_t i = 0; i < nrows; ++i) d[i + j * nrows] = f(i, j);
        return Mat(std::move(d), nrows, ncols);
    }
    size_t nrows() const noexcept { return nrows_; }
    size_t ncols() const noexcept { return ncols_; }
    Scalar get(size_t i, size_t j) const { return data_[i + j * nrows_]; }
    const std::vector<Scalar>& as_slice() const noexcept { return data_; }

  private:
    Mat(std::vector<Scalar> d, size_t r, size_t c) : data_(std::move(d)), nrows_(r), ncols_(c) {}
    std::vector<Scalar> data_;
    size_t nrows_ = 0, ncols_ = 0;
};

template <class S>
struct MatWithArgmax {
    Mat<S> values;
    std::vector<uint32_t> argmax;  // the CPU crate's u32 indices (gpu_mat.rs:400-412)
};

template <class S>
class GpuMatWithArgmax;

// A semiring-typed device matrix (gpu_mat.rs:45-370).
template <class S>
class GpuMat {
  public:
    using Scalar = typename S::Scalar;

    static GpuMat from_matref(const HipContext& ctx, const Mat<S>& mat) {
        return GpuMat(GpuMatrix<Scalar>::from_host(ctx, mat.as_slice(), mat.nrows(), mat.ncols()));
    }
    static GpuMat from_slice(const HipContext& ctx, const std::vector<Scalar>& data, size_t nrows, size_t ncols) {
        return GpuMat(GpuMatrix<Scalar>::from_host(ctx, data, nrows, ncols));
    }
    static GpuMat zeros(const HipContext& ctx, size_t nrows, size_t ncols) {
        return GpuMat(GpuMatrix<Scalar>::alloc(ctx, nrows, ncols));
    }
    size_t nrows() const noexcept { return inner_.rows(); }
    size_t ncols() const noexcept { return inner_.cols(); }
    const GpuMatrix<Scalar>& as_gpu_matrix() const noexcept { return inner_; }
    GpuMatrix<Scalar>& as_gpu_matrix_mut() noexcept { return inner_; }
    Mat<S> to_mat(const HipContext& ctx) const {
        return Mat<S>::from_col_major(inner_.to_host(ctx), nrows(), ncols());
    }

    GpuMat matmul(const HipContext& ctx, const GpuMat& b) const {  // gpu_mat.rs:136-149
        check_inner(b);
        auto c = GpuMatrix<Scalar>::alloc(ctx, nrows(), b.ncols());
        launch_gemm<S>(ctx, inner_, b.inner_, c);
        return GpuMat(std::move(c));
    }
    GpuMatWithArgmax<S> matmul_argmax(const HipContext& ctx, const GpuMat& b) const;

    // gpu_mat.rs:321-370: pairwise products of equally shaped batches.
    static std::vector<GpuMat> matmul_batched(const HipContext& ctx, const std::vector<GpuMat>& a,
                                              const std::vector<GpuMat>& b) {
        check_batch(a, b);
        std::vector<GpuMat> out;
        out.reserve(a.size());
        for (size_t t = 0; t < a.size(); ++t) out.push_back(a[t].matmul(ctx, b[t]));
        return out;
    }
    static std::vector<GpuMatWithArgmax<S>> matmul_batched_with_argmax(const HipContext& ctx,
                                                                       const std::vector<GpuMat>& a,
                                                                       const std::vector<GpuMat>& b);
    static std::vector<GpuMat> from_mats(const HipContext& ctx, const std::vector<Mat<S>>& mats) {
        std::vector<GpuMat> out;
        out.reserve(mats.size());
        for (const auto& m : mats) out.push_back(from_matref(ctx, m));
        return out;
    }
    static std::vector<Mat<S>> to_mats(const HipContext& ctx, const std::vector<GpuMat>& mats) {
        std::vector<Mat<S>> out;
        out.reserve(mats.size());
        for (const auto& m : mats) out.push_back(m.to_mat(ctx));
        return out;
    }

  private:
    explicit GpuMat(GpuMatrix<Scalar>&& m) : inner_(std::move(m)) {}
    void check_inner(const GpuMat& b) const {
        if (ncols() != b.nrows())
            detail::mismatch("A.ncols (" + std::to_string(ncols()) + ") != B.nrows (" + std::to_string(b.nrows()) + ")");
    }
    static void check_batch(const std::vector<GpuMat>& a, const std::vector<GpuMat>& b) {
        if (a.size() != b.size())
            detail::mismatch("Batch sizes must match: A has " + std::to_string(a.size()) + " matrices, B has " +
                             std::to_string(b.size()));
        for (size_t t = 1; t < a.size(); ++t)
            if (a[t].nrows() != a[0].nrows() || a[t].ncols() != a[0].ncols() || b[t].nrows() != b[0].nrows() ||
                b[t].ncols() != b[0].ncols())
                detail::mismatch("All matrices in a batch must have the same dimensions");
    }
    GpuMatrix<Scalar> inner_;
};

// Result plus argmax (gpu_mat.rs:374-563).
template <class S>
class GpuMatWithArgmax {
  public:
    using Scalar = typename S::Scalar;
    size_t nrows() const noexcept { return inner_.rows(); }
    size_t ncols() const noexcept { return inner_.cols(); }
    MatWithArgmax<S> to_mat_with_argmax(const HipContext& ctx) const {
        auto am = inner_.argmax_to_host(ctx);
        MatWithArgmax<S> r{Mat<S>::from_col_major(inner_.matrix_to_host(ctx), nrows(), ncols()), {}};
        r.argmax.reserve(am.size());
        for (ArgmaxIndex x : am) r.argmax.push_back(uint32_t(x));
        return r;
    }
    Mat<S> to_mat(const HipContext& ctx) const {
        return Mat<S>::from_col_major(inner_.matrix_to_host(ctx), nrows(), ncols());
    }
    std::vector<ArgmaxIndex> to_argmax(const HipContext& ctx) const { return inner_.argmax_to_host(ctx); }
    const GpuMatrixWithArgmax<Scalar>& as_inner() const noexcept { return inner_; }

    // gpu_mat.rs:467-562: host scatter with the downloaded argmax, like the
    // reference; grad_c is m x n, the result m x k (backward_a) or k x n.
    template <class G>
    Mat<G> backward_a(const HipContext& ctx, const Mat<G>& grad_c, size_t k) const {
        check_grad(grad_c);
        auto g = tropical_backward_a_gpu(grad_c.as_slice(), to_argmax(ctx), nrows(), k, ncols());
        return Mat<G>::from_col_major(g, nrows(), k);
    }
    template <class G>
    Mat<G> backward_b(const HipContext& ctx, const Mat<G>& grad_c, size_t k) const {
        check_grad(grad_c);
        auto g = tropical_backward_b_gpu(grad_c.as_slice(), to_argmax(ctx), nrows(), k, ncols());
        return Mat<G>::from_col_major(g, k, ncols());
    }

  private:
    friend class GpuMat<S>;
    explicit GpuMatWithArgmax(GpuMatrixWithArgmax<Scalar>&& m) : inner_(std::move(m)) {}
    template <class G>
    void check_grad(const Mat<G>& g) const {
        if (g.nrows() != nrows() || g.ncols() != ncols())
            detail::mismatch("grad_c dimensions (" + std::to_string(g.nrows()) + ", " + std::to_string(g.ncols()) +
                             ") don't match C (" + std::to_string(nrows()) + ", " + std::to_string(ncols()) + ")");
    }
    GpuMatrixWithArgmax<Scalar> inner_;
};

template <class S>
GpuMatWithArgmax<S> GpuMat<S>::matmul_argmax(const HipContext& ctx, const GpuMat& b) const {  // gpu_mat.rs:159-176
    check_inner(b);
    auto c = GpuMatrixWithArgmax<Scalar>::alloc(ctx, nrows(), b.ncols());
    launch_gemm_with_argmax<S>(ctx, inner_, b.inner_, c);
    return GpuMatWithArgmax<S>(std::move(c));
}

template <class S>
std::vector<GpuMatWithArgmax<S>> GpuMat<S>::matmul_batched_with_argmax(const HipContext& ctx,
                                                                       const std::vector<GpuMat>& a,
                                                                       const std::vector<GpuMat>& b) {
    check_batch(a, b);
    std::vector<GpuMatWithArgmax<S>> out;
    out.reserve(a.size());
    for (size_t t = 0; t < a.size(); ++t) out.push_back(a[t].matmul_argmax(ctx, b[t]));
    return out;
}

}  // namespace tropical_gemm_hip
