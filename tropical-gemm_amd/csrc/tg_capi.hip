// tg_capi.hip -- the C ABI declared in include/tropical_gemm_hip.h.
//
// Host side of the drop-in boundary: argument validation (done before any HIP
// call, so it is testable without a GPU), device selection, layout mapping,
// workspace handling and kernel dispatch.  Reference counterparts are cited
// per entry point in the header.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/tropical_gemm_hip.h"
#include "tg_backward.hpp"
#include "tg_gemm_dl.hpp"
#include "tg_gemm_dl64.hpp"
#include "tg_gemm_kres.hpp"
#include "tg_gemm_kres8.hpp"
#include "tg_gemm_kresw.hpp"
#include "tg_gemm_shortk.hpp"
#include "tg_kernels.hpp"

namespace {

constexpr int kAbiVersion = 1;

thread_local std::string g_last_error = "";

int fail(int status, const std::string& msg) {
    g_last_error = msg;
    return status;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(TG_ERR_DRIVER, std::string(what) + ": " + hipGetErrorString(e));
}

#define TG_HIP(expr)                                   \
    do {                                               \
        hipError_t _e = (expr);                        \
        if (_e != hipSuccess) return hip_fail(_e, #expr); \
    } while (0)

int elem_size(tg_dtype dt) {
    switch (dt) {
        case TG_F32:
        case TG_I32:
            return 4;
        case TG_F64:
        case TG_I64:
            return 8;
    }
    return 0;
}

const char* dtype_name(int dt) {
    switch (dt) {
        case TG_F32: return "f32";
        case TG_F64: return "f64";
        case TG_I32: return "i32";
        case TG_I64: return "i64";
    }
    return "?";
}

bool valid_semiring(int s) { return s == TG_MAXPLUS || s == TG_MINPLUS || s == TG_MAXMUL; }
bool valid_dtype(int d) { return d == TG_F32 || d == TG_F64 || d == TG_I32 || d == TG_I64; }
bool valid_layout(int l) { return l == TG_ROW_MAJOR || l == TG_COL_MAJOR; }

// Device handling: the ordinal is validated against the device count (the
// reference answers an out-of-range ordinal with DimensionMismatch,
// crates/tropical-gemm-cuda/src/lib.rs:81-87) and made current.
std::once_flag g_count_once;
int g_device_count = -1;
hipError_t g_count_err = hipSuccess;

int device_count_cached(int* out) {
    std::call_once(g_count_once, [] {
        int n = 0;
        g_count_err = hipGetDeviceCount(&n);
        g_device_count = (g_count_err == hipSuccess) ? n : 0;
    });
    if (g_count_err != hipSuccess && g_count_err != hipErrorNoDevice)
        return hip_fail(g_count_err, "hipGetDeviceCount");
    *out = g_device_count;
    return TG_OK;
}

int select_device(int device) {
    int n = 0;
    int rc = device_count_cached(&n);
    if (rc != TG_OK) return rc;
    if (n <= 0) return fail(TG_ERR_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= n)
        return fail(TG_ERR_DIMENSION_MISMATCH, "Device " + std::to_string(device) +
                                                   " not available (only " + std::to_string(n) +
                                                   " HIP device(s) found)");
    int cur = -1;
    TG_HIP(hipGetDevice(&cur));
    if (cur != device) TG_HIP(hipSetDevice(device));
    return TG_OK;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Optional event timing of the main GEMM kernels (tg_kernel_timing_*).
std::atomic<bool> g_timing{false};
std::mutex g_timing_mu;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_timing_events;

// Records an event pair around the launches made during its lifetime when
// timing is enabled; does nothing otherwise.
class KernelTimer {
  public:
    explicit KernelTimer(hipStream_t st) : st_(st) {
        if (!g_timing.load(std::memory_order_relaxed)) return;
        if (hipEventCreate(&e0_) != hipSuccess || hipEventCreate(&e1_) != hipSuccess ||
            hipEventRecord(e0_, st_) != hipSuccess) {
            release();
            return;
        }
        on_ = true;
    }
    ~KernelTimer() {
        if (!on_) return;
        if (hipEventRecord(e1_, st_) != hipSuccess) {
            release();
            return;
        }
        std::lock_guard<std::mutex> lk(g_timing_mu);
        g_timing_events.emplace_back(e0_, e1_);
    }
    KernelTimer(const KernelTimer&) = delete;
    KernelTimer& operator=(const KernelTimer&) = delete;

  private:
    void release() {
        if (e0_) (void)hipEventDestroy(e0_);
        if (e1_) (void)hipEventDestroy(e1_);
        e0_ = e1_ = nullptr;
        on_ = false;
    }
    hipStream_t st_;
    hipEvent_t e0_ = nullptr, e1_ = nullptr;
    bool on_ = false;
};

// ----------------------------------------------------------------------------
// Launch helpers
// ----------------------------------------------------------------------------

int launch_fill_zero(void* p, size_t bytes, hipStream_t st) {
    if (bytes == 0) return TG_OK;
    int64_t nvec = int64_t(bytes / 16);
    int64_t blocks = (nvec + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(tg::tg_fill_zero, dim3(unsigned(blocks)), dim3(256), 0, st,
                       static_cast<unsigned char*>(p), int64_t(bytes));
    TG_HIP(hipGetLastError());
    return TG_OK;
}

template <typename T>
bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// B^T staging (BT[z][j][k] = B[z][k][j], nb batch items): 16-byte vectors when
// the shape, strides and pointers allow them, element by element otherwise.
// The callers have checked (K + 31) / 32 <= 65535.
template <typename T>
bool transpose_vectors(const T* B, const T* BT, int64_t K, int64_t N, int64_t sB, int64_t sBT) {
    constexpr int VW = tg::Vec16<T>::N;
    return K % VW == 0 && N % VW == 0 && sB % VW == 0 && sBT % VW == 0 && aligned16<T>(B) &&
           aligned16<T>(BT);
}

// cls (f64 only, and only where transpose_vectors holds): the column classes
// of B are ORed into cls[z*N + j] on the way (see tg_transpose_v).
template <typename T>
int launch_transpose(const T* B, T* BT, int64_t K, int64_t N, int64_t sB, int64_t sBT, int64_t nb,
                     hipStream_t st, uint32_t* cls = nullptr) {
    if (transpose_vectors<T>(B, BT, K, N, sB, sBT)) {
        dim3 grid(unsigned((N + 63) / 64), unsigned((K + 63) / 64), unsigned(nb));
        hipLaunchKernelGGL((tg::tg_transpose_v<T>), grid, dim3(256), 0, st, B, BT, K, N, sB, sBT,
                           cls);
    } else {
        if (cls != nullptr)
            return fail(TG_ERR_INVALID_ARGUMENT, "internal: column classes need the vector transpose");
        dim3 grid(unsigned((N + 31) / 32), unsigned((K + 31) / 32), unsigned(nb));
        hipLaunchKernelGGL((tg::tg_transpose<T>), grid, dim3(32, 8), 0, st, B, BT, K, N, sB, sBT);
    }
    TG_HIP(hipGetLastError());
    return TG_OK;
}

// Row-major problem description after the layout mapping.
struct Problem {
    const void* A;
    const void* B;
    void* C;
    int32_t* IDX;
    int64_t batch, M, N, K, sA, sB, sC;
};

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Workspace layout: [B^T staging (argmax)][split-K value partials][split-K
// index partials (argmax)], each region 256-byte aligned.
struct WsLayout {
    size_t bt = 0, pv = 0, pi = 0, total = 0;
};

WsLayout ws_layout(tg_dtype dt, int64_t batch, int64_t M, int64_t N, int64_t K, bool argmax,
                   int splits) {
    WsLayout w;
    const size_t es = size_t(elem_size(dt));
    const size_t bt = argmax ? round_up(size_t(batch) * size_t(K) * size_t(N) * es, 256) : 0;
    const size_t part = splits > 1 ? round_up(size_t(splits) * size_t(batch) * size_t(M) * size_t(N) * es, 256) : 0;
    w.bt = 0;
    w.pv = bt;
    w.pi = bt + part;
    w.total = bt + part + (argmax ? part : 0);
    return w;
}

// Workspace of the f64 direct-to-LDS kernel: B^T (batch x K x N, argmax
// only), then the row classes of A (batch x M) and column classes of B
// (batch x N).
size_t dl64_ws_bytes(int64_t batch, int64_t M, int64_t N, int64_t K, bool argmax) {
    return (argmax ? round_up(size_t(batch) * size_t(K) * size_t(N) * 8, 256) : 0) +
           round_up(size_t(batch) * size_t(M + N) * 4, 256);
}

// f64, large problems (tg_gemm_dl64): the operand class prepass and, with
// argmax, B^T staging; then the GEMM.  K % 32 == 0 and the rest of dl64_fits
// hold.
template <int SR>
int run_gemm_dl64(const Problem& p, void* ws, hipStream_t st) {
    using Cfg = tg::Dl64Cfg;
    const int64_t tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    const int64_t tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    if (tiles_m * tiles_n > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "output too large for one launch");
    if ((p.K + 31) / 32 > 65535 || (p.K + 255) / 256 > 65535)
        return fail(TG_ERR_DIMENSION_MISMATCH, "K too large for the staging grids");
    const double* A = static_cast<const double*>(p.A);
    const double* B = static_cast<const double*>(p.B);
    const bool argmax = p.IDX != nullptr;
    unsigned char* wsb = static_cast<unsigned char*>(ws);
    double* BT = argmax ? reinterpret_cast<double*>(wsb) : nullptr;
    const size_t bt_bytes = argmax ? round_up(size_t(p.batch) * size_t(p.K) * size_t(p.N) * 8, 256) : 0;
    uint32_t* cls = reinterpret_cast<uint32_t*>(wsb + bt_bytes);
    uint32_t* clsA = cls;
    uint32_t* clsB = cls + p.batch * p.M;
    // With argmax, the B^T transpose records the column classes when it runs
    // on 16-byte vectors (every batch chunk alike: sB and K*N are even).
    const bool cols_in_transpose =
        argmax && transpose_vectors<double>(B, BT, p.K, p.N, p.sB, p.K * p.N);
    hipLaunchKernelGGL(tg::tg_fill_zero, dim3(unsigned((p.batch * (p.M + p.N) * 4 / 16 + 255) / 256 + 1)),
                       dim3(256), 0, st, reinterpret_cast<unsigned char*>(cls), p.batch * (p.M + p.N) * 4);
    TG_HIP(hipGetLastError());
    {
        int64_t row_blocks = (p.batch * p.M + 3) / 4;
        if (row_blocks > 16384) row_blocks = 16384;
        int64_t col_blocks = cols_in_transpose ? 0 : ((p.N + 63) / 64) * ((p.K + 255) / 256) * p.batch;
        if (col_blocks > 16384) col_blocks = 16384;
        hipLaunchKernelGGL(tg::tg_class_prepass, dim3(unsigned(row_blocks + col_blocks)), dim3(256), 0,
                           st, A, p.M, p.K, p.sA, B, p.N, p.sB, p.batch, clsA,
                           cols_in_transpose ? nullptr : clsB, int(row_blocks));
        TG_HIP(hipGetLastError());
    }
    for (int64_t z0 = 0; argmax && z0 < p.batch; z0 += 65535) {
        const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
        const int rc = launch_transpose<double>(B + z0 * p.sB, BT + z0 * p.K * p.N, p.K, p.N, p.sB,
                                                p.K * p.N, nb, st,
                                                cols_in_transpose ? clsB + z0 * p.N : nullptr);
        if (rc != TG_OK) return rc;
    }
    KernelTimer timer(st);
    for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
        const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
        const dim3 grid(unsigned(tiles_m * tiles_n), 1, unsigned(nb));
        double* Cz = static_cast<double*>(p.C) + z0 * p.sC;
        if (argmax)
            hipLaunchKernelGGL((tg::tg_gemm_dl64<SR, true>), grid, dim3(256), Cfg::LDS_BYTES, st,
                               A + z0 * p.sA, B + z0 * p.sB, BT + z0 * p.K * p.N, Cz,
                               p.IDX + z0 * p.sC, clsA + z0 * p.M, clsB + z0 * p.N, p.M, p.N, p.K,
                               p.sA, p.sB, p.sC, int(tiles_m), int(tiles_n));
        else
            hipLaunchKernelGGL((tg::tg_gemm_dl64<SR, false>), grid, dim3(256), Cfg::TILE_BYTES, st,
                               A + z0 * p.sA, B + z0 * p.sB, nullptr, Cz, nullptr, clsA + z0 * p.M,
                               clsB + z0 * p.N, p.M, p.N, p.K, p.sA, p.sB, p.sC, int(tiles_m),
                               int(tiles_n));
        TG_HIP(hipGetLastError());
    }
    return TG_OK;
}

// Split argmax on 64 x 64 tiles whose chunk holds an even number of
// fragments runs its K slices in one workgroup: the number of slices (four
// when each keeps at least 256 k, else two), or 0 when the split runs as
// separate launches into the workspace partials.
inline int wg_slices(bool slices_ok, bool argmax, int splits, int64_t K) {
    constexpr int BK = tg::TG_CHUNK;
    if (!slices_ok || !argmax || (splits != 2 && splits != 4) || K % (2 * BK) != 0) return 0;
    return (K % (4 * BK) == 0 && K / 4 >= 256) ? 4 : 2;
}

// Direct-to-LDS kernel for 32-bit types (partial edge tiles allowed, see
// tg::dl_fits).  splits > 1 (full tiles only) runs K in that many slices into
// the workspace partials, then merges them.
template <int SR, typename T, int TM, int TN, int CL>
int run_gemm_dl(const Problem& p, void* ws, int splits, hipStream_t st) {
    using Cfg = tg::DlCfg<TM, TN>;
    const int64_t tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;  // the last ones may be partial
    const int64_t tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    if (tiles_m * tiles_n > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "output too large for one launch");
    const T* A = static_cast<const T*>(p.A);
    const T* B = static_cast<const T*>(p.B);
    T* C = static_cast<T*>(p.C);
    const bool argmax = p.IDX != nullptr;
    const WsLayout wl = ws_layout(std::is_same<T, float>::value ? TG_F32 : TG_I32, p.batch, p.M,
                                  p.N, p.K, argmax, splits);
    unsigned char* wsb = static_cast<unsigned char*>(ws);
    T* PV = splits > 1 ? reinterpret_cast<T*>(wsb + wl.pv) : nullptr;
    int32_t* PI = (splits > 1 && argmax) ? reinterpret_cast<int32_t*>(wsb + wl.pi) : nullptr;
    const int64_t MN = p.M * p.N;
    const int64_t sY = splits > 1 ? p.batch * MN : 0;
    const int64_t KS = p.K / splits;
    // Split-K problems are small: when all of B (every batch item) fits in
    // 4 MiB it stays in L2, and the resolve reads B's columns directly
    // (BDIRECT), with no B^T staged and one launch fewer.
    const bool bdirect = argmax && splits > 1 && TN == 4 && p.K % Cfg::BK == 0 &&
                         size_t(p.batch) * size_t(p.K) * size_t(p.N) * sizeof(T) <= (size_t(4) << 20);
    if (argmax && !bdirect) {  // B^T staging for the resolve, outside the timed GEMM launches
        if ((p.K + 31) / 32 > 65535)
            return fail(TG_ERR_DIMENSION_MISMATCH, "K too large for the transpose grid");
        for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
            const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
            T* BT = reinterpret_cast<T*>(wsb + wl.bt) + z0 * p.K * p.N;
            const int rc = launch_transpose<T>(B + z0 * p.sB, BT, p.K, p.N, p.sB, p.K * p.N, nb, st);
            if (rc != TG_OK) return rc;
        }
    }
    // 128 x 128 value-only tiles take 64 KB of dynamic LDS: raise the
    // kernel's limit once (no stream work, so also fine under capture).
    // The value-only 8 x 8 tiles run the pipelined main loop (tg::pipe_fits).
    constexpr bool kPipe = TM == 8 && TN == 8;
    const bool pipe = kPipe && !argmax && tg::pipe_fits(p.N, p.K);
    if constexpr (Cfg::TILE_BYTES > 48 * 1024) {
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&tg::tg_gemm_dl<SR, T, false, TM, TN, CL>),
            hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::TILE_BYTES);
        TG_HIP(attr);
        if constexpr (kPipe) {
            static const hipError_t attr_pipe = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&tg::tg_gemm_dl<SR, T, false, TM, TN, CL, false, false, 2>),
                hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::TILE_BYTES);
            TG_HIP(attr_pipe);
        }
    }
    // Split argmax on 64 x 64 tiles: the K slices of a tile run in one
    // workgroup, 256 threads per slice, and merge in LDS (no partials, no
    // merge launch).  Four slices (1024 threads, four waves per SIMD) when
    // each slice keeps at least 256 k, else two.
    constexpr bool kHalves = TM == 4 && TN == 4 && (Cfg::BK / CL) % 2 == 0;
    if (const int halves = wg_slices(kHalves, argmax, splits, p.K)) {
        if constexpr (kHalves) {
            const int64_t KSh = p.K / halves;
            static const hipError_t attr4 = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, false, 0, 4>),
                hipFuncAttributeMaxDynamicSharedMemorySize, 4 * Cfg::LDS_BYTES);
            static const hipError_t attr4d = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, true, 0, 4>),
                hipFuncAttributeMaxDynamicSharedMemorySize, 4 * Cfg::LDS_BYTES);
            TG_HIP(attr4);
            TG_HIP(attr4d);
            KernelTimer timer(st);
            for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
                const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
                const T* Az = A + z0 * p.sA;
                const T* Bz = B + z0 * p.sB;
                T* Cz = C + z0 * p.sC;
                int32_t* Iz = p.IDX + z0 * p.sC;
                const T* BT = reinterpret_cast<const T*>(wsb + wl.bt) + z0 * p.K * p.N;
                dim3 grid(unsigned(tiles_m * tiles_n), 1, unsigned(nb));
                if (halves == 4) {
                    if (bdirect)
                        hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, true, 0, 4>),
                                           grid, dim3(1024), 4 * Cfg::LDS_BYTES, st, Az, Bz, nullptr,
                                           Cz, Iz, p.M, p.N, p.K, p.sA, p.sB, p.sC, int(tiles_m),
                                           int(tiles_n), KSh, int64_t(0));
                    else
                        hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, false, 0, 4>),
                                           grid, dim3(1024), 4 * Cfg::LDS_BYTES, st, Az, Bz, BT, Cz,
                                           Iz, p.M, p.N, p.K, p.sA, p.sB, p.sC, int(tiles_m),
                                           int(tiles_n), KSh, int64_t(0));
                } else if (bdirect) {
                    hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, true, 0, 2>),
                                       grid, dim3(512), 2 * Cfg::LDS_BYTES, st, Az, Bz, nullptr, Cz,
                                       Iz, p.M, p.N, p.K, p.sA, p.sB, p.sC, int(tiles_m),
                                       int(tiles_n), KSh, int64_t(0));
                } else {
                    hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, false, 0, 2>),
                                       grid, dim3(512), 2 * Cfg::LDS_BYTES, st, Az, Bz, BT, Cz, Iz,
                                       p.M, p.N, p.K, p.sA, p.sB, p.sC, int(tiles_m), int(tiles_n),
                                       KSh, int64_t(0));
                }
                TG_HIP(hipGetLastError());
            }
        }
        return TG_OK;
    }
    KernelTimer timer(st);
    for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
        const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
        const T* Az = A + z0 * p.sA;
        const T* Bz = B + z0 * p.sB;
        // Split launches write dense partials (batch stride M*N).
        T* Cz = splits > 1 ? PV + z0 * MN : C + z0 * p.sC;
        int32_t* Iz = !argmax ? nullptr : splits > 1 ? PI + z0 * MN : p.IDX + z0 * p.sC;
        const int64_t sCk = splits > 1 ? MN : p.sC;
        dim3 grid(unsigned(tiles_m * tiles_n), unsigned(splits), unsigned(nb));
        const bool tailk = p.K % Cfg::BK != 0;  // the last k-tile is partial
        if (argmax) {
            const T* BT = reinterpret_cast<const T*>(wsb + wl.bt) + z0 * p.K * p.N;
            if constexpr (TM == 4 && TN == 4 && (Cfg::BK / CL) % 2 == 0) {
                if (bdirect) {
                    hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL, false, true>), grid,
                                       dim3(256), Cfg::LDS_BYTES, st, Az, Bz, nullptr, Cz, Iz, p.M,
                                       p.N, p.K, p.sA, p.sB, sCk, int(tiles_m), int(tiles_n), KS,
                                       sY);
                    TG_HIP(hipGetLastError());
                    continue;
                }
            }
            if constexpr (TM == 4 && (Cfg::BK / CL) % 2 == 0) {
                if (tailk) {
                    // 64 x 64 tiles only: the 64 x 128 kernel with the tail
                    // code would spill (the plan never picks it for a partial K).
                    if constexpr (TN == 4)
                        hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL, true>), grid,
                                           dim3(256), Cfg::LDS_BYTES, st, Az, Bz, BT, Cz, Iz, p.M,
                                           p.N, p.K, p.sA, p.sB, sCk, int(tiles_m), int(tiles_n),
                                           KS, sY);
                    else
                        return fail(TG_ERR_INVALID_ARGUMENT,
                                    "internal: 64x128 tiles need K % 32 == 0");
                } else
                    hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, true, TM, TN, CL>), grid, dim3(256),
                                       Cfg::LDS_BYTES, st, Az, Bz, BT, Cz, Iz, p.M, p.N, p.K,
                                       p.sA, p.sB, sCk, int(tiles_m), int(tiles_n), KS, sY);
            } else {
                return fail(TG_ERR_INVALID_ARGUMENT,
                            "internal: argmax tiles have 4 rows and an even chunk count per k-tile");
            }
        } else {
            if (tailk) {
                if constexpr (TM == 4 && TN == 4)
                    hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, false, TM, TN, CL, true>), grid,
                                       dim3(256), Cfg::TILE_BYTES, st, Az, Bz, nullptr, Cz,
                                       nullptr, p.M, p.N, p.K, p.sA, p.sB, sCk, int(tiles_m),
                                       int(tiles_n), KS, sY);
                else
                    return fail(TG_ERR_INVALID_ARGUMENT, "internal: wide tiles need K % 32 == 0");
            } else if (pipe) {
                if constexpr (kPipe)
                    hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, false, TM, TN, CL, false, false, 2>),
                                       grid, dim3(256), Cfg::TILE_BYTES, st, Az, Bz, nullptr, Cz,
                                       nullptr, p.M, p.N, p.K, p.sA, p.sB, sCk, int(tiles_m),
                                       int(tiles_n), KS, sY);
            } else
                hipLaunchKernelGGL((tg::tg_gemm_dl<SR, T, false, TM, TN, CL>), grid, dim3(256),
                                   Cfg::TILE_BYTES, st, Az, Bz, nullptr, Cz, nullptr, p.M, p.N,
                                   p.K, p.sA, p.sB, sCk, int(tiles_m), int(tiles_n), KS, sY);
        }
        TG_HIP(hipGetLastError());
    }
    if (splits > 1) {
        const int64_t nvec = p.batch * MN / 4;
        int64_t blocks = (nvec + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        const T* BT = argmax && !bdirect ? reinterpret_cast<const T*>(wsb + wl.bt) : nullptr;
        if (argmax)
            hipLaunchKernelGGL((tg::tg_merge_splits<SR, T, true>), dim3(unsigned(blocks)), dim3(256), 0,
                               st, PV, PI, C, p.IDX, splits, MN, p.batch, sY, p.sC, A, B, BT, p.N,
                               p.K, p.sA, p.sB);
        else
            hipLaunchKernelGGL((tg::tg_merge_splits<SR, T, false>), dim3(unsigned(blocks)), dim3(256), 0,
                               st, PV, nullptr, C, nullptr, splits, MN, p.batch, sY, p.sC, A, B,
                               BT, p.N, p.K, p.sA, p.sB);
        TG_HIP(hipGetLastError());
    }
    return TG_OK;
}

// Compute units of the current device (cached per device).
int current_cu_count() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lk(mu);
    if (int(cache.size()) <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

// Workgroups of tg_gemm_kres<SR, T, KT> resident per CU (LDS and register
// limits), from the runtime's occupancy calculator; 2 if that fails.
template <int SR, typename T, int KT>
int kres_per_cu() {
    static const int n = [] {
        int b = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, tg::tg_gemm_kres<SR, T, KT>, 256, 0) !=
                hipSuccess ||
            b <= 0) {
            (void)hipGetLastError();
            b = 2;
        }
        return b;
    }();
    return n;
}

template <int SR, typename T, int KT>
void launch_kres(const Problem& p, int64_t tiles_m, int64_t tiles_n, hipStream_t st) {
    // Persistent grid: every resident workgroup slot, rounded down to a
    // multiple of the column-tile count (each workgroup owns one column tile).
    const int64_t total = p.batch * tiles_m * tiles_n;
    int64_t grid = int64_t(kres_per_cu<SR, T, KT>()) * current_cu_count();
    grid = (grid / tiles_n) * tiles_n;
    if (grid < tiles_n) grid = tiles_n;
    if (grid > total) grid = total;
    hipLaunchKernelGGL((tg::tg_gemm_kres<SR, T, KT>), dim3(unsigned(grid)), dim3(256), 0, st,
                       static_cast<const T*>(p.A), static_cast<const T*>(p.B), static_cast<T*>(p.C),
                       p.IDX, p.N, p.sA, p.sB, p.sC, int(tiles_m), int(tiles_n), p.batch);
}

// Workgroups of tg_gemm_kres8<SR, KT> resident per CU; 1 if the query fails.
template <int SR, int KT>
int kres8_per_cu() {
    static const int n = [] {
        int b = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, tg::tg_gemm_kres8<SR, KT>, 256, 0) !=
                hipSuccess ||
            b <= 0) {
            (void)hipGetLastError();
            b = 1;
        }
        return b;
    }();
    return n;
}

template <int SR, int KT>
void launch_kres8(const Problem& p, int64_t tiles_m, int64_t tiles_n, hipStream_t st) {
    const int64_t total = p.batch * tiles_m * tiles_n;
    int64_t grid = int64_t(kres8_per_cu<SR, KT>()) * current_cu_count();
    grid = (grid / tiles_n) * tiles_n;
    if (grid < tiles_n) grid = tiles_n;
    if (grid > total) grid = total;
    hipLaunchKernelGGL((tg::tg_gemm_kres8<SR, KT>), dim3(unsigned(grid)), dim3(256), 0, st,
                       static_cast<const int32_t*>(p.A), static_cast<const int32_t*>(p.B),
                       static_cast<int32_t*>(p.C), p.IDX, p.N, p.sA, p.sB, p.sC, int(tiles_m),
                       int(tiles_n), p.batch);
}

// K-resident argmax kernel with 64 x 128 tiles (i32 MaxPlus/MinPlus).
template <int SR>
int run_gemm_kres8(const Problem& p, hipStream_t st) {
    using Cfg = tg::Kres8Cfg;
    const int64_t tiles_m = p.M / Cfg::BM;
    const int64_t tiles_n = p.N / Cfg::BN;
    if (tiles_m > 0x7fffffffLL || tiles_n > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "output too large for one launch");
    KernelTimer timer(st);
    switch (p.K / Cfg::BK) {
        case 2: launch_kres8<SR, 2>(p, tiles_m, tiles_n, st); break;
        case 3: launch_kres8<SR, 3>(p, tiles_m, tiles_n, st); break;
        case 4: launch_kres8<SR, 4>(p, tiles_m, tiles_n, st); break;
        default: return fail(TG_ERR_INVALID_ARGUMENT, "K-resident kernel: unsupported K");
    }
    TG_HIP(hipGetLastError());
    return TG_OK;
}

// K-resident argmax kernel with wave-private 16-row tiles (i32
// MaxPlus/MinPlus, N a multiple of 128): one 1024-thread workgroup per CU,
// the CUs split evenly over the column tiles.
template <int SR, int KT>
int launch_kresw(const Problem& p, int64_t tiles_n, hipStream_t st) {
    constexpr size_t lds = tg::kresw_lds_bytes(KT);
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&tg::tg_gemm_kresw<SR, KT>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    TG_HIP(attr);
    int64_t grid = (int64_t(current_cu_count()) / tiles_n) * tiles_n;
    if (grid < tiles_n) grid = tiles_n;
    // Fewer workgroups when the row tiles would not give each of a column
    // tile's workgroups one tile per wave.
    const int64_t per_col = (p.M / tg::KreswCfg::ROWS + tg::KreswCfg::WAVES - 1) / tg::KreswCfg::WAVES;
    if (grid > per_col * tiles_n) grid = per_col * tiles_n;
    hipLaunchKernelGGL((tg::tg_gemm_kresw<SR, KT>), dim3(unsigned(grid)), dim3(1024), lds, st,
                       static_cast<const int32_t*>(p.A), static_cast<const int32_t*>(p.B),
                       static_cast<int32_t*>(p.C), p.IDX, p.M, p.N, p.sA, p.sB, p.sC,
                       int(tiles_n), p.batch);
    return TG_OK;
}

template <int SR>
int run_gemm_kresw(const Problem& p, hipStream_t st) {
    using Cfg = tg::KreswCfg;
    const int64_t tiles_n = p.N / Cfg::BN;
    KernelTimer timer(st);
    int rc = TG_OK;
    switch (p.K / Cfg::BK) {
        case 2: rc = launch_kresw<SR, 2>(p, tiles_n, st); break;
        case 3: rc = launch_kresw<SR, 3>(p, tiles_n, st); break;
        case 4: rc = launch_kresw<SR, 4>(p, tiles_n, st); break;
        default: return fail(TG_ERR_INVALID_ARGUMENT, "K-resident kernel: unsupported K");
    }
    if (rc != TG_OK) return rc;
    TG_HIP(hipGetLastError());
    return TG_OK;
}

// Short-K kernel: 32 x 256 (64-bit types: 16 x 256) tiles written as 1 KB
// row runs.
template <int SR, typename T>
int run_gemm_shortk(const Problem& p, hipStream_t st) {
    using Cfg = tg::ShortkCfg<T>;
    const int64_t tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    const int64_t tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    if (tiles_m * tiles_n > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "output too large for one launch");
    const bool argmax = p.IDX != nullptr;
    KernelTimer timer(st);
    for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
        const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
        const T* Az = static_cast<const T*>(p.A) + z0 * p.sA;
        const T* Bz = static_cast<const T*>(p.B) + z0 * p.sB;
        T* Cz = static_cast<T*>(p.C) + z0 * p.sC;
        dim3 grid(unsigned(tiles_m * tiles_n), 1, unsigned(nb));
        if (argmax)
            hipLaunchKernelGGL((tg::tg_gemm_shortk<SR, T, true>), grid, dim3(256), 0, st, Az, Bz,
                               Cz, p.IDX + z0 * p.sC, p.M, p.N, p.K, p.sA, p.sB, p.sC,
                               int(tiles_n));
        else
            hipLaunchKernelGGL((tg::tg_gemm_shortk<SR, T, false>), grid, dim3(256), 0, st, Az, Bz,
                               Cz, nullptr, p.M, p.N, p.K, p.sA, p.sB, p.sC, int(tiles_n));
        TG_HIP(hipGetLastError());
    }
    return TG_OK;
}

// K-resident argmax kernel for short K (32-bit types): no B^T staging.
template <int SR, typename T>
int run_gemm_kres(const Problem& p, hipStream_t st) {
    using Cfg = tg::KresCfg;
    const int64_t tiles_m = p.M / Cfg::BM;
    const int64_t tiles_n = p.N / Cfg::BN;
    if (tiles_m > 0x7fffffffLL || tiles_n > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "output too large for one launch");
    KernelTimer timer(st);
    switch (p.K / Cfg::BK) {
        case 2: launch_kres<SR, T, 2>(p, tiles_m, tiles_n, st); break;
        case 3: launch_kres<SR, T, 3>(p, tiles_m, tiles_n, st); break;
        case 4: launch_kres<SR, T, 4>(p, tiles_m, tiles_n, st); break;
        default: return fail(TG_ERR_INVALID_ARGUMENT, "K-resident kernel: unsupported K");
    }
    TG_HIP(hipGetLastError());
    return TG_OK;
}

// Argmax problems with K up to this run the generic tiles kernel in its exact
// mode (per-product index tracking, no resolve, no B^T staging): at short K
// the chunked kernels' resolve, which re-reads A and B^T windows per output,
// costs several times the main loop.
constexpr int64_t kExactMaxK = 32;
// Argmax problems with partial tiles (M, N or K) that the direct-to-LDS kernels
// can run take the generic kernel's exact mode up to this K: measured on
// MI355X (f32 MaxPlus, 4100^2 and 1000^2), exact 124 us against 153 at K = 64,
// 233 against 188 at K = 128.
constexpr int64_t kExactPartialMaxK = 96;
// Argmax problems that reach the generic tiles kernel (no direct-to-LDS or
// K-resident kernel takes them) run its exact mode up to this K: 4 VALU ops
// per product against the chunked mode's ~2 plus its resolve.  Crossovers
// measured on MI355X (MaxPlus, M = N = 4096): f32 near K = 480, f64 near
// K = 700, i64 near K = 4096 (its 64-bit compare costs as much as the add).
template <typename T>
constexpr int64_t exact_tiles_max_k() {
    return sizeof(T) == 4 ? 384 : std::is_same<T, int64_t>::value ? 2048 : 512;
}

// Problems with K up to these run the short-K kernel (when N % 4 == 0 and B,
// C, IDX are 16-byte aligned).  Measured on MI355X (MaxPlus, against the
// kernels these problems took before): f32 65536 x 2048 x K, argmax K = 8
// 183 us against 251 (generic tiles, exact mode), K = 32 403 against 417,
// K = 48 567 against 554; value-only K = 8 104 against 143, K = 48 253
// against 336, K = 64 344 against 343 (direct-to-LDS); f64 8192^2 x K,
// argmax K = 8 163 against 236, K = 32 335 against 390; value-only K = 63
// 368 against 434.
constexpr int64_t kShortkArgmaxMaxK = 32;
constexpr int64_t kShortkValueMaxK = 63;

// The kernel a problem runs on.
enum class Path { SHORTK, KRESW, KRES8, KRES, DL_88_32, DL_48_16, DL_48_VALUE, DL_44_8, DL_44_16, DL_44_32, DL64, DL64_VALUE, TILES_EXACT, TILES_CHUNKED, TILES };

struct Plan {
    Path path = Path::TILES;
    int splits = 1;
};

// True when the path reads the workspace: B^T staging for the resolve of the
// chunked argmax kernels, and split-K partials.
bool uses_workspace(const Plan& pl, bool argmax) {
    switch (pl.path) {
        case Path::SHORTK:
        case Path::KRESW:
        case Path::KRES8:
        case Path::KRES:
        case Path::TILES_EXACT:
        case Path::TILES: return false;
        case Path::TILES_CHUNKED:
        case Path::DL64:
        case Path::DL64_VALUE: return true;
        default: return argmax || pl.splits > 1;
    }
}

// Chooses the kernel.  ws_bytes limits split K (the partials live in the
// workspace).
template <int SR, typename T>
Plan plan_typed(const Problem& p, size_t ws_bytes) {
    Plan pl;
    const bool argmax = p.IDX != nullptr;
    const bool exact = argmax && p.K <= kExactMaxK;
    if (p.K <= (argmax ? kShortkArgmaxMaxK : kShortkValueMaxK) &&
        tg::shortk_fits(p.M, p.N, p.K, p.sB, p.sC, p.B, p.C, p.IDX)) {
        pl.path = Path::SHORTK;
        return pl;
    }
    if constexpr (sizeof(T) == 4) {
        if constexpr (std::is_same<T, int32_t>::value && SR != tg::SR_MAXMUL) {
            if (argmax && tg::kresw_fits(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::KRESW;
                return pl;
            }
            if (argmax && tg::kres8_fits(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::KRES8;
                return pl;
            }
        }
        if (argmax && tg::kres_fits(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
            pl.path = Path::KRES;
            return pl;
        }
        // Partial tiles (M, N or K): short argmax problems take the generic
        // kernel's exact mode (no resolve); longer ones and value-only run
        // the direct-to-LDS kernels with clamped loads.
        const bool partial = !tg::dl_full_tiles<4, 4>(p.M, p.N, p.K);
        // Value-only with K below 64 and not a multiple of 32: most of the
        // direct-to-LDS kernel's padded last k-tile would be wasted work;
        // the generic kernel bounds its last tile instead.
        const bool short_tail = !argmax && p.K % 32 != 0 && p.K < 64;
        if (!exact && !short_tail && !(partial && argmax && p.K <= kExactPartialMaxK)) {
            // Direct-to-LDS kernels (value-only, or argmax beyond the exact
            // range).  Split K when the problem makes too few 64 x 64 tiles
            // and the workspace holds the partials (tg_gemm_workspace_size
            // includes them).
            const tg_dtype dt = std::is_same<T, float>::value ? TG_F32 : TG_I32;
            int splits = tg::dl_splits(p.M, p.N, p.K, p.batch);
            if (splits > 1 && ws_layout(dt, p.batch, p.M, p.N, p.K, argmax, splits).total > ws_bytes)
                splits = 1;
            const int64_t ks = p.K / splits;
            // Argmax chunk length.  The bookkeeping costs 2 VALU ops per output
            // per chunk (2K/CL); the resolve re-reads one chunk's A-row and
            // B^T-row segments per output from L2 and recomputes them, which
            // costs more than its ~4 ops per product suggest.  Measured on
            // MI355X (f32 MaxPlus, slices of 256 .. 4096 k): CL = 8 is fastest
            // up to 512 k per slice, CL = 16 above (CL = 32 is 4-18% slower
            // everywhere).
            const int cl = !argmax ? 32 : ks <= 512 ? 8 : 16;
            // 64 x 128 tiles for argmax problems big enough that the last
            // round of 768 resident workgroups is a small share of the work
            // (their main loop is the faster one); 64 x 64 tiles otherwise
            // (value-only runs four workgroups per CU, small problems get
            // twice the tiles).
            using W48 = tg::DlCfg<4, 8>;
            using W88 = tg::DlCfg<8, 8>;
            const bool wide = splits == 1 && argmax && cl == 16 && p.N % W48::BN == 0 &&
                              p.K % W48::BK == 0 &&
                              ((p.M + W48::BM - 1) / W48::BM) * (p.N / W48::BN) * p.batch >= 1536;
            // Value-only tile shape by how the tiles fill the resident slots
            // of the 256 CUs (128 x 128 tiles run two per CU, 512 slots;
            // 64 x 64 tiles four, 1024 slots).  128 x 128 tiles (8 x 8
            // outputs per thread) from two rounds up, or exactly one round
            // (2048 x 4096 x 1024: 241 against 267-279 us for 64 x 64; one
            // and a bit rounds, 3072^2 x 2048, take 855 against 593-628 us);
            // 64 x 128 tiles where 64 x 64 would make exactly one round
            // (2048^2 x 2048: 265-269 against 286-290 us; 5-8% at K = 1024 ..
            // 4096); 64 x 64 otherwise (0.75 or 1.25 rounds: 5-15% faster
            // than 64 x 128).
            constexpr int64_t kCus = 256;
            const int64_t t128 =
                ((p.M + W88::BM - 1) / W88::BM) * ((p.N + W88::BN - 1) / W88::BN) * p.batch;
            const int64_t t64 = ((p.M + 63) / 64) * ((p.N + 63) / 64) * p.batch;
            const bool big = splits == 1 && !argmax && p.K % W88::BK == 0 &&
                             (t128 >= 4 * kCus || t128 == 2 * kCus);
            const bool mid = splits == 1 && !argmax && !big && t64 == 4 * kCus &&
                             p.N % W48::BN == 0 && p.K % W48::BK == 0;
            pl.splits = splits;
            if (wide && tg::dl_fits<16>(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::DL_48_16;
                pl.splits = 1;
                return pl;
            }
            if (big && tg::dl_fits<32>(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::DL_88_32;
                pl.splits = 1;
                return pl;
            }
            if (mid && tg::dl_fits<16>(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::DL_48_VALUE;
                pl.splits = 1;
                return pl;
            }
            if (cl == 8 && tg::dl_fits<8>(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::DL_44_8;
                return pl;
            }
            if (cl == 16 && tg::dl_fits<16>(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::DL_44_16;
                return pl;
            }
            if (cl == 32 && tg::dl_fits<32>(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX)) {
                pl.path = Path::DL_44_32;
                return pl;
            }
            pl.splits = 1;
        }
    }
    if constexpr (std::is_same<T, double>::value) {
        // f64 on at least 256 tiles of 64 x 128 with the workspace for the
        // operand classes (and B^T with argmax): argmax beyond the exact
        // range, value-only from K = 256 (below that the class prepass and
        // its launches weigh on the product).
        const int64_t tiles = ((p.M + tg::Dl64Cfg::BM - 1) / tg::Dl64Cfg::BM) *
                              ((p.N + tg::Dl64Cfg::BN - 1) / tg::Dl64Cfg::BN) * p.batch;
        const bool deep = argmax ? !exact && p.K > exact_tiles_max_k<T>() : p.K >= 256;
        if (deep && tiles >= 256 &&
            tg::dl64_fits(p.M, p.N, p.K, p.sA, p.sB, p.sC, p.A, p.B, p.C, p.IDX) &&
            dl64_ws_bytes(p.batch, p.M, p.N, p.K, argmax) <= ws_bytes) {
            pl.path = argmax ? Path::DL64 : Path::DL64_VALUE;
            return pl;
        }
    }
    if (!argmax)
        pl.path = Path::TILES;
    else if (exact || p.K <= exact_tiles_max_k<T>())
        pl.path = Path::TILES_EXACT;
    else
        pl.path = Path::TILES_CHUNKED;
    return pl;
}

template <int SR, typename T>
int run_gemm_typed(const Problem& p, void* ws, size_t ws_bytes, hipStream_t st) {
    const Plan pl = plan_typed<SR, T>(p, ws_bytes);
    if (pl.path == Path::SHORTK) return run_gemm_shortk<SR, T>(p, st);
    if constexpr (std::is_same<T, double>::value) {
        if (pl.path == Path::DL64 || pl.path == Path::DL64_VALUE) return run_gemm_dl64<SR>(p, ws, st);
    }
    if constexpr (sizeof(T) == 4) {
        switch (pl.path) {
            case Path::KRESW:
                if constexpr (std::is_same<T, int32_t>::value && SR != tg::SR_MAXMUL)
                    return run_gemm_kresw<SR>(p, st);
                break;
            case Path::KRES8:
                if constexpr (std::is_same<T, int32_t>::value && SR != tg::SR_MAXMUL)
                    return run_gemm_kres8<SR>(p, st);
                break;
            case Path::KRES: return run_gemm_kres<SR, T>(p, st);
            case Path::DL_88_32: return run_gemm_dl<SR, T, 8, 8, 32>(p, ws, 1, st);
            case Path::DL_48_16: return run_gemm_dl<SR, T, 4, 8, 16>(p, ws, 1, st);
            case Path::DL_48_VALUE: return run_gemm_dl<SR, T, 4, 8, 16>(p, ws, 1, st);  // CL unused
            case Path::DL_44_8: return run_gemm_dl<SR, T, 4, 4, 8>(p, ws, pl.splits, st);
            case Path::DL_44_16: return run_gemm_dl<SR, T, 4, 4, 16>(p, ws, pl.splits, st);
            case Path::DL_44_32: return run_gemm_dl<SR, T, 4, 4, 32>(p, ws, pl.splits, st);
            default: break;
        }
    }
    using Cfg = tg::TileCfg<T>;
    const int64_t tiles_m = (p.M + Cfg::BM - 1) / Cfg::BM;
    const int64_t tiles_n = (p.N + Cfg::BN - 1) / Cfg::BN;
    if (tiles_m * tiles_n > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "output too large for one launch");
    const T* A = static_cast<const T*>(p.A);
    const T* B = static_cast<const T*>(p.B);
    T* C = static_cast<T*>(p.C);
    constexpr int VW = 16 / int(sizeof(T));
    const bool vec = (p.K % VW == 0) && (p.N % VW == 0) && (p.sA % VW == 0) &&
                     (p.sB % VW == 0) && aligned16<T>(A) && aligned16<T>(B);
    const bool argmax = p.IDX != nullptr;

    for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
        const int64_t nb = (p.batch - z0 < 65535) ? p.batch - z0 : 65535;
        const T* Az = A + z0 * p.sA;
        const T* Bz = B + z0 * p.sB;
        T* Cz = C + z0 * p.sC;
        int32_t* Iz = argmax ? p.IDX + z0 * p.sC : nullptr;
        dim3 grid(unsigned(tiles_m * tiles_n), 1, unsigned(nb));
        if (pl.path == Path::TILES_EXACT) {
            KernelTimer timer(st);
            if (vec)
                hipLaunchKernelGGL((tg::tg_gemm_tiles<SR, T, true, true, true>), grid, dim3(256), 0,
                                   st, Az, Bz, nullptr, Cz, Iz, p.M, p.N, p.K, p.sA, p.sB, p.sC,
                                   int(tiles_m), int(tiles_n));
            else
                hipLaunchKernelGGL((tg::tg_gemm_tiles<SR, T, true, false, true>), grid, dim3(256), 0,
                                   st, Az, Bz, nullptr, Cz, Iz, p.M, p.N, p.K, p.sA, p.sB, p.sC,
                                   int(tiles_m), int(tiles_n));
            TG_HIP(hipGetLastError());
        } else if (pl.path == Path::TILES_CHUNKED) {
            // B^T staging for the argmax epilogue (dense, batch stride K*N).
            T* BT = static_cast<T*>(ws);
            const int64_t sBT = p.K * p.N;
            if (p.K > 0) {
                if ((p.K + 31) / 32 > 65535)
                    return fail(TG_ERR_DIMENSION_MISMATCH, "K too large for the transpose grid");
                const int rc = launch_transpose<T>(Bz, BT, p.K, p.N, p.sB, sBT, nb, st);
                if (rc != TG_OK) return rc;
            }
            // 64-bit integers record 16-k chunks: their 128-byte windows halve
            // what the resolve reads (it misses L2), for one record per 64
            // instructions of products instead of 128.
            constexpr int CL = std::is_same<T, int64_t>::value ? 16 : tg::TG_CHUNK;
            KernelTimer timer(st);
            if (vec)
                hipLaunchKernelGGL((tg::tg_gemm_tiles<SR, T, true, true, false, CL>), grid, dim3(256),
                                   0, st, Az, Bz, BT, Cz, Iz, p.M, p.N, p.K, p.sA, p.sB, p.sC,
                                   int(tiles_m), int(tiles_n));
            else
                hipLaunchKernelGGL((tg::tg_gemm_tiles<SR, T, true, false, false, CL>), grid,
                                   dim3(256), 0, st, Az, Bz, BT, Cz, Iz, p.M, p.N, p.K, p.sA, p.sB,
                                   p.sC, int(tiles_m), int(tiles_n));
            TG_HIP(hipGetLastError());
        } else {
            KernelTimer timer(st);
            if (vec)
                hipLaunchKernelGGL((tg::tg_gemm_tiles<SR, T, false, true>), grid, dim3(256), 0, st,
                                   Az, Bz, nullptr, Cz, nullptr, p.M, p.N, p.K, p.sA, p.sB, p.sC,
                                   int(tiles_m), int(tiles_n));
            else
                hipLaunchKernelGGL((tg::tg_gemm_tiles<SR, T, false, false>), grid, dim3(256), 0,
                                   st, Az, Bz, nullptr, Cz, nullptr, p.M, p.N, p.K, p.sA, p.sB,
                                   p.sC, int(tiles_m), int(tiles_n));
            TG_HIP(hipGetLastError());
        }
    }
    return TG_OK;
}

template <int SR>
int run_gemm_sr(tg_dtype dt, const Problem& p, void* ws, size_t ws_bytes, hipStream_t st) {
    switch (dt) {
        case TG_F32: return run_gemm_typed<SR, float>(p, ws, ws_bytes, st);
        case TG_F64: return run_gemm_typed<SR, double>(p, ws, ws_bytes, st);
        case TG_I32: return run_gemm_typed<SR, int32_t>(p, ws, ws_bytes, st);
        case TG_I64: return run_gemm_typed<SR, int64_t>(p, ws, ws_bytes, st);
    }
    return fail(TG_ERR_INVALID_ARGUMENT, "bad dtype");
}

template <int SR>
Plan plan_sr(tg_dtype dt, const Problem& p, size_t ws_bytes) {
    switch (dt) {
        case TG_F32: return plan_typed<SR, float>(p, ws_bytes);
        case TG_F64: return plan_typed<SR, double>(p, ws_bytes);
        case TG_I32: return plan_typed<SR, int32_t>(p, ws_bytes);
        case TG_I64: return plan_typed<SR, int64_t>(p, ws_bytes);
    }
    return Plan{};
}

Plan plan_gemm(tg_semiring sr, tg_dtype dt, const Problem& p, size_t ws_bytes) {
    switch (sr) {
        case TG_MAXPLUS: return plan_sr<tg::SR_MAXPLUS>(dt, p, ws_bytes);
        case TG_MINPLUS: return plan_sr<tg::SR_MINPLUS>(dt, p, ws_bytes);
        case TG_MAXMUL: return plan_sr<tg::SR_MAXMUL>(dt, p, ws_bytes);
    }
    return Plan{};
}

const char* path_name(Path path) {
    switch (path) {
        case Path::SHORTK: return "shortk";
        case Path::KRESW: return "kresw";
        case Path::KRES8: return "kres8";
        case Path::KRES: return "kres";
        case Path::DL_88_32: return "dl_8x8_cl32";
        case Path::DL_48_16: return "dl_4x8_cl16";
        case Path::DL_48_VALUE: return "dl_4x8";
        case Path::DL_44_8: return "dl_4x4_cl8";
        case Path::DL_44_16: return "dl_4x4_cl16";
        case Path::DL_44_32: return "dl_4x4_cl32";
        case Path::DL64: return "dl64_4x8_cl16";
        case Path::DL64_VALUE: return "dl64_4x8";
        case Path::TILES_EXACT: return "tiles_exact";
        case Path::TILES_CHUNKED: return "tiles_chunked";
        case Path::TILES: return "tiles";
    }
    return "?";
}

int run_gemm(tg_semiring sr, tg_dtype dt, const Problem& p, void* ws, size_t ws_bytes,
             hipStream_t st) {
    switch (sr) {
        case TG_MAXPLUS: return run_gemm_sr<tg::SR_MAXPLUS>(dt, p, ws, ws_bytes, st);
        case TG_MINPLUS: return run_gemm_sr<tg::SR_MINPLUS>(dt, p, ws, ws_bytes, st);
        case TG_MAXMUL: return run_gemm_sr<tg::SR_MAXMUL>(dt, p, ws, ws_bytes, st);
    }
    return fail(TG_ERR_INVALID_ARGUMENT, "bad semiring");
}

// B^T staging for argmax problems: K x N' elements per batch item, where N'
// is the kernel's N after the layout mapping (n for row-major calls, m for
// column-major ones, whose operands are swapped).  The size does not depend
// on the layout: K x max(m, n) covers both.  This is the minimum workspace.
size_t bt_bytes_for(tg_dtype dt, int64_t batch, int64_t m, int64_t n, int64_t k, bool with_argmax) {
    if (!with_argmax || batch <= 0 || m <= 0 || n <= 0 || k <= 0) return 0;
    const int64_t wide = m > n ? m : n;
    return round_up(size_t(batch) * size_t(k) * size_t(wide) * size_t(elem_size(dt)), 256);
}

// Full workspace: the minimum plus the split-K partials (values, and indices
// for argmax) of 32-bit problems that make too few tiles (tg::dl_splits,
// taken for both orientations: column-major calls swap m and n).  A
// workspace of at least the minimum runs the same products unsplit.
size_t workspace_bytes_for(tg_dtype dt, int64_t batch, int64_t m, int64_t n, int64_t k,
                           bool with_argmax) {
    if (batch <= 0 || m <= 0 || n <= 0 || k <= 0) return 0;
    size_t w = bt_bytes_for(dt, batch, m, n, k, with_argmax);
    if (dt == TG_F64)  // operand classes of the f64 direct-to-LDS kernel
        w += round_up(size_t(batch) * size_t(m + n) * 4, 256);
    if (elem_size(dt) == 4) {
        const int s1 = tg::dl_splits(m, n, k, batch), s2 = tg::dl_splits(n, m, k, batch);
        const int s = s1 > s2 ? s1 : s2;
        if (s > 1) {
            const size_t part = round_up(size_t(s) * size_t(batch) * size_t(m) * size_t(n) * 4, 256);
            w += part * (with_argmax ? 2 : 1);
        }
    }
    return w;
}

// Validation shared by the forward entry points.  Returns TG_OK or an error.
int validate_forward(int sr, int dt, int layout, const void* A, const void* B, const void* C,
                     int64_t batch, int64_t m, int64_t n, int64_t k, int64_t sa, int64_t sb,
                     int64_t sc, bool strided) {
    if (!valid_semiring(sr)) return fail(TG_ERR_INVALID_ARGUMENT, "unknown semiring " + std::to_string(sr));
    if (!valid_dtype(dt)) return fail(TG_ERR_INVALID_ARGUMENT, "unknown dtype " + std::to_string(dt));
    if (!valid_layout(layout)) return fail(TG_ERR_INVALID_ARGUMENT, "unknown layout " + std::to_string(layout));
    if (batch < 0 || m < 0 || n < 0 || k < 0)
        return fail(TG_ERR_DIMENSION_MISMATCH,
                    "negative dimension: batch=" + std::to_string(batch) + " m=" + std::to_string(m) +
                        " n=" + std::to_string(n) + " k=" + std::to_string(k));
    if (m > 0x7fffffffLL || n > 0x7fffffffLL || k > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "dimension exceeds 2^31-1 (argmax is int32)");
    const int64_t out = m * n;
    if (batch > 0 && out > 0) {
        if (C == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "C is NULL");
        if (k > 0 && (A == nullptr || B == nullptr))
            return fail(TG_ERR_INVALID_ARGUMENT, "A or B is NULL");
    }
    if (strided && batch > 1) {
        if (sc < out)
            return fail(TG_ERR_DIMENSION_MISMATCH,
                        "stride_c (" + std::to_string(sc) + ") < m*n (" + std::to_string(out) +
                            "): output matrices would overlap");
        if (sa < 0 || sb < 0) return fail(TG_ERR_DIMENSION_MISMATCH, "negative input stride");
    }
    return TG_OK;
}

// Layout mapping: a column-major product C = A (x) B is the row-major
// product C^T = B^T (x) A^T over the same buffers (kernels.rs:370-430).
Problem make_problem(tg_layout layout, const void* A, const void* B, void* C, int32_t* argmax,
                     int64_t batch, int64_t m, int64_t n, int64_t k, int64_t sa, int64_t sb,
                     int64_t sc, bool strided) {
    Problem p;
    if (layout == TG_ROW_MAJOR) {
        p = Problem{A, B, C, argmax, batch, m, n, k, sa, sb, sc};
    } else {
        p = Problem{B, A, C, argmax, batch, n, m, k, sb, sa, sc};
    }
    if (!strided) {
        p.sA = p.M * p.K;
        p.sB = p.K * p.N;
        p.sC = p.M * p.N;
    }
    return p;
}

int gemm_impl(int device, tg_semiring sr, tg_dtype dt, tg_layout layout, const void* A,
              const void* B, void* C, int32_t* argmax, int64_t batch, int64_t m, int64_t n,
              int64_t k, int64_t sa, int64_t sb, int64_t sc, bool strided, void* ws,
              size_t ws_bytes, bool ws_given, void* stream) {
    int rc = validate_forward(sr, dt, layout, A, B, C, batch, m, n, k, sa, sb, sc, strided);
    if (rc != TG_OK) return rc;
    const bool with_argmax = argmax != nullptr;
    const size_t need = bt_bytes_for(dt, batch, m, n, k, with_argmax);
    if (ws_given && need > 0) {
        if (ws == nullptr || ws_bytes < need)
            return fail(TG_ERR_INVALID_ARGUMENT, "workspace too small: need " + std::to_string(need) +
                                                     " bytes, got " + std::to_string(ws_bytes));
        if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0)
            return fail(TG_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    }
    // A workspace the split-K partials cannot use (none, or misaligned when
    // no B^T staging is needed) runs the product unsplit.
    if (ws_given && (ws == nullptr || (reinterpret_cast<uintptr_t>(ws) & 255u) != 0)) ws_bytes = 0;
    rc = select_device(device);
    if (rc != TG_OK) return rc;
    if (batch == 0 || m == 0 || n == 0) return TG_OK;
    hipStream_t st = as_stream(stream);

    Problem p = make_problem(layout, A, B, C, argmax, batch, m, n, k, sa, sb, sc, strided);

    // The kernels stage B^T (K x p.N per batch item) in the workspace.
    if (need > 0 && need < size_t(p.batch) * size_t(p.K) * size_t(p.N) * size_t(elem_size(dt)))
        return fail(TG_ERR_INVALID_ARGUMENT, "internal: workspace size below K x N");
    void* work = ws;
    bool own = false;
    if (!ws_given) {
        // Allocate the full workspace only for the kernels that read it.
        ws_bytes = workspace_bytes_for(dt, batch, m, n, k, with_argmax);
        if (ws_bytes > 0 && !uses_workspace(plan_gemm(sr, dt, p, ws_bytes), with_argmax))
            ws_bytes = 0;
        if (ws_bytes > 0) {
            TG_HIP(hipMallocAsync(&work, ws_bytes, st));
            own = true;
        }
    }
    rc = run_gemm(sr, dt, p, work, ws_given || own ? ws_bytes : 0, st);
    if (own) {
        hipError_t e = hipFreeAsync(work, st);
        if (rc == TG_OK && e != hipSuccess) return hip_fail(e, "hipFreeAsync");
    }
    return rc;
}

// ----------------------------------------------------------------------------
// Workspace without allocation (tg_gemm_noalloc)
// ----------------------------------------------------------------------------

// The workspace of tg_gemm_noalloc: one fixed array in the code object's
// zero-initialised device data.  Each device that loads the library holds its
// own copy from the module's load until the process ends.  On the host the
// name `scratch` is only a stand-in, never a device address: host code uses
// the address hipGetSymbolAddress returns for the current device
// (scratch_address), in kernel arguments as everywhere else.
constexpr size_t kScratchBytes = TG_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices] = {};

// Device address of `scratch` on `device`, which must be the current device.
// Looked up once per device (tg_context_init, or the first tg_gemm_noalloc
// call on that device) and kept.
int scratch_address(int device, void** out) {
    if (device < 0 || device >= kScratchMaxDevices)
        return fail(TG_ERR_INVALID_ARGUMENT,
                    "tg_gemm_noalloc supports devices 0.." + std::to_string(kScratchMaxDevices - 1));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (ptr == nullptr) return fail(TG_ERR_DRIVER, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return TG_OK;
}

// Scratch bytes the planned path reads (0 when it reads none).  The plan is
// made with kScratchBytes as the workspace, so split K is only chosen when
// its partials fit; B^T staging alone may still exceed it.
size_t scratch_need(tg_dtype dt, const Problem& p, const Plan& pl) {
    const bool argmax = p.IDX != nullptr;
    if (!uses_workspace(pl, argmax)) return 0;
    // The f64 direct-to-LDS kernel's workspace: B^T (argmax) and the operand
    // classes of A's rows and B's columns (run_gemm_dl64).
    if (pl.path == Path::DL64 || pl.path == Path::DL64_VALUE)
        return dl64_ws_bytes(p.batch, p.M, p.N, p.K, argmax);
    return ws_layout(dt, p.batch, p.M, p.N, p.K, argmax, pl.splits).total;
}

// ----------------------------------------------------------------------------
// Backward
// ----------------------------------------------------------------------------

// Launch geometry of the deterministic backward kernels (tg_backward.hpp).
// Both kernels loop over their rows / column groups with a grid stride, so
// the grid is capped (kBwdMaxGrid workgroups) and no dimension of a launch
// grows with M, N or the batch.
constexpr int64_t kBwdMaxGrid = 16384;
constexpr size_t kBwdLdsBudget = 128 * 1024;  // bins of one grad_A row at most
constexpr size_t kBwdLdsLimit = 160 * 1024;   // the CU's LDS
// grad_B takes its keys in passes (8 columns per group) when the columns'
// bins do not fit eight at a time, a pass re-reads no more bytes than it
// writes (the group's M rows of index and dC against its keys' gradients)
// and there are at most kBwdMaxPasses of them.  Measured (bit-identical,
// f32 unless noted): 1024 x 4096 x 32768 770 -> 220 us, x 16384 227 -> 107,
// f64 1024 x 4096 x 16384 550 -> 206; 4096 x 1024 x 16384 (re-reads twice
// the writes) 93 -> 129 and 62 passes at K = 262144 1.05 -> 1.39 ms, hence
// the two limits.
constexpr int64_t kBwdMaxPasses = 16;

struct BwdGeometry {
    bool global = false;  // bins in the gradient itself (K too large for LDS)
    int waves = 1;        // waves per workgroup
    size_t lds = 0;       // dynamic LDS bytes per workgroup
    int64_t grid = 0;     // workgroups
    int64_t groups_n = 0; // grad_B: column groups per batch item
    int64_t groups = 0;   // grad_B: column groups in total
    int64_t kp = 0;       // grad_B: keys per pass (K: one pass)
};

// grad_A: one wave per row; a wave's LDS is its row's K bins plus its stage
// (tg::kRowStageElems elements).  Four waves per workgroup while that is at
// most 8 KB, two while at most 16 KB, else one (18 KB at K = 4096 f32: eight
// workgroups per CU); global bins beyond the LDS budget.
BwdGeometry bwd_rows_geometry(int64_t rows, int64_t K, size_t es) {
    BwdGeometry g;
    const size_t row_bytes = size_t(K) * es;
    const size_t stage_bytes = size_t(tg::kRowStageElems) * es;
    const size_t wave_bytes = row_bytes + stage_bytes;
    if (row_bytes > kBwdLdsBudget) {
        g.global = true;
        g.waves = 4;
    } else {
        g.waves = wave_bytes <= 8 * 1024 ? 4 : wave_bytes <= 16 * 1024 ? 2 : 1;
    }
    g.lds = size_t(g.waves) * (g.global ? stage_bytes : wave_bytes);
    const int64_t need = (rows + g.waves - 1) / g.waves;
    g.grid = need < kBwdMaxGrid ? need : kBwdMaxGrid;
    return g;
}

// grad_B: one wave per column, W <= 8 adjacent columns per workgroup: the
// most whose bins, the staged tiles of argmax and dC (tg::kBwdTileRows x W)
// and the waves' stages fit the CU's 160 KB (8 at K = 4096 f32: 154 KB).
// Longer columns over few rows keep 8 columns and take their keys in passes
// (kp: keys per pass, see kBwdMaxPasses); otherwise fewer columns, and
// global bins when not even one column's fit.
BwdGeometry bwd_cols_geometry(int64_t batch, int64_t M, int64_t N, int64_t K, size_t es) {
    BwdGeometry g;
    auto lds_for = [&](int64_t w, int64_t kp, bool global) {
        return (global ? 0 : size_t(w) * size_t(kp) * es) +
               size_t(tg::kBwdTileRows) * size_t(w + 1) * (4 + es) +
               size_t(w) * size_t(tg::kStageElems) * es;
    };
    g.kp = K;
    // Keys per pass with 8 columns: what the LDS holds, a multiple of 4.
    const size_t fixed8 = lds_for(8, 0, false);
    const int64_t kp8 = int64_t((kBwdLdsLimit - fixed8) / (8 * es)) & ~int64_t(3);
    const bool one_pass = lds_for(8, K, false) <= kBwdLdsLimit;
    const int64_t passes = kp8 > 0 ? (K + kp8 - 1) / kp8 : 0;
    if (!one_pass && kp8 > 0 && M * int64_t(4 + es) <= kp8 * int64_t(es) &&
        passes <= kBwdMaxPasses) {
        // Long columns, few rows: 8 columns in passes over the keys.
        g.kp = kp8;
        g.waves = 8;
        g.lds = lds_for(8, kp8, false);
    } else {
        int64_t w = size_t(K) * es > kBwdLdsBudget ? 0 : 8;
        while (w >= 1 && lds_for(w, K, false) > kBwdLdsLimit) --w;
        if (w < 1) {
            g.global = true;
            w = 8;
        }
        g.waves = int(w);
        g.lds = lds_for(w, K, g.global);
    }
    const int64_t w = g.waves;
    g.groups_n = (N + w - 1) / w;
    g.groups = batch * g.groups_n;
    g.grid = g.groups < kBwdMaxGrid ? g.groups : kBwdMaxGrid;
    return g;
}

// Raises a kernel's dynamic LDS limit once (needed above 64 KB).
template <typename K>
int allow_lds(K* kernel, size_t bytes) {
    if (bytes <= 64 * 1024) return TG_OK;
    TG_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes)));
    return TG_OK;
}

// A gradient with no contributions (the product has no rows or no columns):
// `batch` matrices of len elements, stride apart, all +0.  The scatter
// kernels would read their first (clamped) contribution at index -1.
template <typename T>
int zero_gradient(T* out, int64_t len, int64_t batch, int64_t stride, hipStream_t st) {
    const int64_t total = len * batch;
    if (total == 0) return TG_OK;
    if ((batch == 1 || stride == len) && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
        // One contiguous run: 16-byte stores.
        const int64_t bytes = total * int64_t(sizeof(T));
        int64_t blocks = (bytes / 16 + 255) / 256;
        if (blocks > 8192) blocks = 8192;
        if (blocks < 1) blocks = 1;
        hipLaunchKernelGGL(tg::tg_fill_zero, dim3(unsigned(blocks)), dim3(256), 0, st,
                           reinterpret_cast<unsigned char*>(out), bytes);
        TG_HIP(hipGetLastError());
        return TG_OK;
    }
    int64_t bx = (len + 255) / 256;
    if (bx > 4096) bx = 4096;
    const int64_t by = batch < 65535 ? batch : 65535;
    hipLaunchKernelGGL((tg::tg_fill_zero_runs<T>), dim3(unsigned(bx), unsigned(by)), dim3(256), 0, st,
                       out, len, batch, stride);
    TG_HIP(hipGetLastError());
    return TG_OK;
}

template <typename T, bool MULT>
int run_backward_rows(const T* G, const int32_t* I, const T* O, T* GA, int64_t batch, int64_t M,
                      int64_t N, int64_t K, int64_t sC, int64_t sO, int64_t sA, hipStream_t st) {
    if (N == 0) return zero_gradient(GA, M * K, batch, sA, st);
    const BwdGeometry g = bwd_rows_geometry(batch * M, K, sizeof(T));
    if (g.grid == 0) return TG_OK;
    if (g.global) {
        hipLaunchKernelGGL((tg::tg_bwd_rows<T, MULT, true>), dim3(unsigned(g.grid)),
                           dim3(64 * g.waves), g.lds, st, G, I, O, GA, M, N, K, sC, sO, sA,
                           batch * M);
    } else {
        int rc = allow_lds(&tg::tg_bwd_rows<T, MULT, false>, g.lds);
        if (rc != TG_OK) return rc;
        hipLaunchKernelGGL((tg::tg_bwd_rows<T, MULT, false>), dim3(unsigned(g.grid)),
                           dim3(64 * g.waves), g.lds, st, G, I, O, GA, M, N, K, sC, sO, sA,
                           batch * M);
    }
    TG_HIP(hipGetLastError());
    return TG_OK;
}

template <typename T, bool MULT>
int run_backward_cols(const T* G, const int32_t* I, const T* O, T* GB, int64_t batch, int64_t M,
                      int64_t N, int64_t K, int64_t sC, int64_t sO, int64_t sB, hipStream_t st) {
    if (M == 0) return zero_gradient(GB, K * N, batch, sB, st);
    const BwdGeometry g = bwd_cols_geometry(batch, M, N, K, sizeof(T));
    if (g.grid == 0) return TG_OK;
    if (g.global) {
        // The bins are grad_B itself, zero-filled first in one coalesced
        // pass (1024 x 4096 x 65536 f32: 1.76 ms with each wave zeroing its
        // column, 0.48 ms this way).
        int rc = zero_gradient(GB, K * N, batch, sB, st);
        if (rc != TG_OK) return rc;
        rc = allow_lds(&tg::tg_bwd_cols<T, MULT, true>, g.lds);
        if (rc != TG_OK) return rc;
        hipLaunchKernelGGL((tg::tg_bwd_cols<T, MULT, true>), dim3(unsigned(g.grid)),
                           dim3(64 * g.waves), g.lds, st, G, I, O, GB, M, N, K, sC, sO, sB,
                           g.groups_n, g.groups, g.kp);
    } else {
        int rc = allow_lds(&tg::tg_bwd_cols<T, MULT, false>, g.lds);
        if (rc != TG_OK) return rc;
        hipLaunchKernelGGL((tg::tg_bwd_cols<T, MULT, false>), dim3(unsigned(g.grid)),
                           dim3(64 * g.waves), g.lds, st, G, I, O, GB, M, N, K, sC, sO, sB,
                           g.groups_n, g.groups, g.kp);
    }
    TG_HIP(hipGetLastError());
    return TG_OK;
}

// which: 0 = grad wrt the left operand (rows of C), 1 = wrt the right operand.
// Operates on the row-major problem.
template <typename T>
int run_backward_typed(int which, bool mult, const void* G, const int32_t* I, const void* O,
                       void* OUT, int64_t batch, int64_t M, int64_t N, int64_t K, int64_t sC,
                       int64_t sO, int64_t sOut, hipStream_t st) {
    const T* g = static_cast<const T*>(G);
    const T* o = static_cast<const T*>(O);
    T* out = static_cast<T*>(OUT);
    if (which == 0) {
        if (mult) return run_backward_rows<T, true>(g, I, o, out, batch, M, N, K, sC, sO, sOut, st);
        return run_backward_rows<T, false>(g, I, o, out, batch, M, N, K, sC, sO, sOut, st);
    }
    if (mult) return run_backward_cols<T, true>(g, I, o, out, batch, M, N, K, sC, sO, sOut, st);
    return run_backward_cols<T, false>(g, I, o, out, batch, M, N, K, sC, sO, sOut, st);
}

// Public-level backward: `want_a` selects grad wrt A (else B); `other` is B
// (for grad A) or A (for grad B) under the MaxMul rule, NULL otherwise.
int backward_impl(int device, tg_dtype dt, tg_layout layout, bool want_a, const void* grad_c,
                  const int32_t* argmax, const void* other, void* out, int64_t batch, int64_t m,
                  int64_t n, int64_t k, int64_t s_c, int64_t s_other, int64_t s_out, bool strided,
                  bool mult, void* stream) {
    if (!valid_dtype(dt)) return fail(TG_ERR_INVALID_ARGUMENT, "unknown dtype " + std::to_string(dt));
    if (dt != TG_F32 && dt != TG_F64)
        return fail(TG_ERR_UNSUPPORTED, std::string("backward is defined for f32/f64 only, got ") +
                                            dtype_name(dt));
    if (!valid_layout(layout)) return fail(TG_ERR_INVALID_ARGUMENT, "unknown layout " + std::to_string(layout));
    if (batch < 0 || m < 0 || n < 0 || k < 0) return fail(TG_ERR_DIMENSION_MISMATCH, "negative dimension");
    if (m > 0x7fffffffLL || n > 0x7fffffffLL || k > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "dimension exceeds 2^31-1");
    const int64_t out_elems = want_a ? m * k : k * n;
    if (batch > 0 && out_elems > 0 && out == nullptr)
        return fail(TG_ERR_INVALID_ARGUMENT, "gradient output is NULL");
    if (batch > 0 && m * n > 0 && (grad_c == nullptr || argmax == nullptr))
        return fail(TG_ERR_INVALID_ARGUMENT, "grad_c or argmax is NULL");
    if (mult && batch > 0 && m * n > 0 && k > 0 && other == nullptr)
        return fail(TG_ERR_INVALID_ARGUMENT, "MaxMul backward needs the other operand");
    if (strided && batch > 1) {
        if (s_out < out_elems)
            return fail(TG_ERR_DIMENSION_MISMATCH, "gradient stride smaller than one matrix");
        if (s_c < 0 || s_other < 0) return fail(TG_ERR_DIMENSION_MISMATCH, "negative stride");
    }
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    if (batch == 0 || out_elems == 0) return TG_OK;
    if (!strided) {
        s_c = m * n;
        s_other = want_a ? k * n : m * k;
        s_out = out_elems;
    }
    hipStream_t st = as_stream(stream);
    // Row-major problem C (M x N) = L (M x K) (x) R (K x N).  Column-major
    // data is the row-major transposed problem C^T = B^T (x) A^T, in which
    // A's gradient is the right operand's gradient and vice versa.
    int which;
    int64_t M, N;
    if (layout == TG_ROW_MAJOR) {
        which = want_a ? 0 : 1;
        M = m;
        N = n;
    } else {
        which = want_a ? 1 : 0;
        M = n;
        N = m;
    }
    if (dt == TG_F32)
        return run_backward_typed<float>(which, mult, grad_c, argmax, other, out, batch, M, N, k,
                                         s_c, s_other, s_out, st);
    return run_backward_typed<double>(which, mult, grad_c, argmax, other, out, batch, M, N, k, s_c,
                                      s_other, s_out, st);
}

}  // namespace

// ============================================================================
// Exported C ABI
// ============================================================================

extern "C" {

int tg_version(void) { return kAbiVersion; }

const char* tg_status_string(int status) {
    switch (status) {
        case TG_OK: return "success";
        case TG_ERR_DRIVER: return "HIP driver/runtime error";
        case TG_ERR_COMPILE: return "kernel compilation error";
        case TG_ERR_NO_DEVICE: return "no HIP device available";
        case TG_ERR_DIMENSION_MISMATCH: return "dimension mismatch";
        case TG_ERR_KERNEL_NOT_FOUND: return "kernel not found";
        case TG_ERR_INVALID_ARGUMENT: return "invalid argument";
        case TG_ERR_UNSUPPORTED: return "unsupported operation";
    }
    return "unknown status";
}

const char* tg_last_error(void) { return g_last_error.c_str(); }

int tg_device_count(int* count) {
    if (count == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "count is NULL");
    return device_count_cached(count);
}

int tg_context_init(int device) {
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipFree(nullptr));  // forces runtime/context initialisation
    if (device < kScratchMaxDevices) {  // tg_gemm_noalloc's workspace address
        void* unused = nullptr;
        rc = scratch_address(device, &unused);
        if (rc != TG_OK) return rc;
    }
    return TG_OK;
}

int tg_device_name(int device, char* buf, size_t len) {
    if (buf == nullptr || len == 0) return fail(TG_ERR_INVALID_ARGUMENT, "buffer is NULL");
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    hipDeviceProp_t prop;
    TG_HIP(hipGetDeviceProperties(&prop, device));
    std::snprintf(buf, len, "HIP Device %d (%s, %s)", device, prop.name, prop.gcnArchName);
    return TG_OK;
}

int tg_malloc(int device, void** ptr, size_t bytes) {
    if (ptr == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "ptr is NULL");
    *ptr = nullptr;
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    if (bytes == 0) return TG_OK;
    TG_HIP(hipMalloc(ptr, bytes));
    return TG_OK;
}

int tg_free(int device, void* ptr) {
    if (ptr == nullptr) return TG_OK;
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipFree(ptr));
    return TG_OK;
}

int tg_memcpy_htod(int device, void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return TG_OK;
    if (dst == nullptr || src == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "NULL pointer");
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return TG_OK;
}

int tg_memcpy_dtoh(int device, void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return TG_OK;
    if (dst == nullptr || src == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "NULL pointer");
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return TG_OK;
}

int tg_memcpy_dtod(int device, void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return TG_OK;
    if (dst == nullptr || src == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "NULL pointer");
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
    return TG_OK;
}

int tg_memset_zero(int device, void* ptr, size_t bytes, void* stream) {
    if (bytes == 0) return TG_OK;
    if (ptr == nullptr) return fail(TG_ERR_INVALID_ARGUMENT, "ptr is NULL");
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    return launch_fill_zero(ptr, bytes, as_stream(stream));
}

int tg_synchronize(int device) {
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipDeviceSynchronize());
    return TG_OK;
}

int tg_stream_synchronize(int device, void* stream) {
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    TG_HIP(hipStreamSynchronize(as_stream(stream)));
    return TG_OK;
}

int tg_kernel_timing_enable(int on) {
    g_timing.store(on != 0);
    return TG_OK;
}

int tg_kernel_timing_read(double* total_ms, int64_t* launches) {
    if (total_ms == nullptr || launches == nullptr)
        return fail(TG_ERR_INVALID_ARGUMENT, "total_ms or launches is NULL");
    std::vector<std::pair<hipEvent_t, hipEvent_t>> evs;
    {
        std::lock_guard<std::mutex> lk(g_timing_mu);
        evs.swap(g_timing_events);
    }
    double sum = 0.0;
    int rc = TG_OK;
    for (auto& e : evs) {
        float ms = 0.0f;
        hipError_t err = hipEventSynchronize(e.second);
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, e.first, e.second);
        if (err != hipSuccess && rc == TG_OK) rc = hip_fail(err, "hipEventElapsedTime");
        sum += ms;
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
    }
    *total_ms = sum;
    *launches = int64_t(evs.size());
    return rc;
}

int tg_gemm(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout, const void* A,
            const void* B, void* C, int32_t* argmax, int64_t m, int64_t n, int64_t k,
            void* stream) {
    return gemm_impl(device, semiring, dtype, layout, A, B, C, argmax, 1, m, n, k, 0, 0, 0, false,
                     nullptr, 0, false, stream);
}

int tg_gemm_noalloc(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                    const void* A, const void* B, void* C, int32_t* argmax, int64_t m, int64_t n,
                    int64_t k, void* stream) {
    int rc = validate_forward(semiring, dtype, layout, A, B, C, 1, m, n, k, 0, 0, 0, false);
    if (rc != TG_OK) return rc;
    const Problem p = make_problem(layout, A, B, C, argmax, 1, m, n, k, 0, 0, 0, false);
    // Host-only planning first, so an oversized problem is rejected before
    // any device work.
    const bool empty = m == 0 || n == 0;
    const Plan pl = empty ? Plan{} : plan_gemm(semiring, dtype, p, kScratchBytes);
    const size_t need = empty ? 0 : scratch_need(dtype, p, pl);
    if (need > kScratchBytes)
        return fail(TG_ERR_INVALID_ARGUMENT,
                    "tg_gemm_noalloc: this problem needs " + std::to_string(need) +
                        " bytes of workspace, above the fixed " + std::to_string(kScratchBytes) +
                        "-byte scratch; use tg_gemm or tg_gemm_ws");
    rc = select_device(device);
    if (rc != TG_OK) return rc;
    if (empty) return TG_OK;
    void* ws = nullptr;
    rc = scratch_address(device, &ws);
    if (rc != TG_OK) return rc;
    return run_gemm(semiring, dtype, p, ws, kScratchBytes, as_stream(stream));
}

size_t tg_gemm_noalloc_bytes(tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                             const void* A, const void* B, const void* C, const int32_t* argmax,
                             int64_t m, int64_t n, int64_t k) {
    if (validate_forward(semiring, dtype, layout, A, B, C, 1, m, n, k, 0, 0, 0, false) != TG_OK)
        return ~size_t(0);
    if (m == 0 || n == 0) return 0;
    const Problem p = make_problem(layout, A, B, const_cast<void*>(C), const_cast<int32_t*>(argmax),
                                   1, m, n, k, 0, 0, 0, false);
    return scratch_need(dtype, p, plan_gemm(semiring, dtype, p, kScratchBytes));
}

size_t tg_gemm_workspace_size(tg_dtype dtype, int64_t batch, int64_t m, int64_t n, int64_t k,
                              int with_argmax) {
    if (!valid_dtype(dtype)) return 0;
    return workspace_bytes_for(dtype, batch, m, n, k, with_argmax != 0);
}

const char* tg_gemm_plan(tg_semiring semiring, tg_dtype dtype, tg_layout layout, const void* A,
                         const void* B, const void* C, const int32_t* argmax, int64_t batch,
                         int64_t m, int64_t n, int64_t k, int64_t stride_a, int64_t stride_b,
                         int64_t stride_c, size_t workspace_bytes) {
    static thread_local std::string name;
    const bool strided = stride_a != 0 || stride_b != 0 || stride_c != 0;
    if (validate_forward(semiring, dtype, layout, A, B, C, batch, m, n, k, stride_a, stride_b,
                         stride_c, strided) != TG_OK)
        return "invalid";
    if (batch == 0 || m == 0 || n == 0) return "none";
    const Problem p = make_problem(layout, A, B, const_cast<void*>(C), const_cast<int32_t*>(argmax),
                                   batch, m, n, k, stride_a, stride_b, stride_c, strided);
    const Plan pl = plan_gemm(semiring, dtype, p, workspace_bytes);
    name = path_name(pl.path);
    const bool slices_ok = pl.path == Path::DL_44_8 || pl.path == Path::DL_44_16;
    if (const int s = wg_slices(slices_ok, argmax != nullptr, pl.splits, p.K))
        name += " slices " + std::to_string(s);
    else if (pl.splits > 1)
        name += " split " + std::to_string(pl.splits);
    return name.c_str();
}

const char* tg_backward_plan(tg_dtype dtype, tg_layout layout, int want_a, int64_t batch,
                             int64_t m, int64_t n, int64_t k) {
    static thread_local std::string name;
    if ((dtype != TG_F32 && dtype != TG_F64) || !valid_layout(layout) || batch < 0 || m < 0 ||
        n < 0 || k < 0)
        return "invalid";
    const size_t es = size_t(elem_size(dtype));
    // Row-major problem after the layout mapping (see backward_impl).
    const bool rows = (layout == TG_ROW_MAJOR) == (want_a != 0);
    const int64_t M = layout == TG_ROW_MAJOR ? m : n, N = layout == TG_ROW_MAJOR ? n : m;
    const BwdGeometry g = rows ? bwd_rows_geometry(batch * M, k, es)
                               : bwd_cols_geometry(batch, M, N, k, es);
    name = std::string(rows ? "rows" : "cols") + (g.global ? " global" : " lds") +
           " waves=" + std::to_string(g.waves) + " lds=" + std::to_string(g.lds) +
           " grid=" + std::to_string(g.grid);
    if (!rows && g.kp < k) name += " passes=" + std::to_string((k + g.kp - 1) / g.kp);
    return name.c_str();
}

int tg_gemm_ws(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout, const void* A,
               const void* B, void* C, int32_t* argmax, int64_t m, int64_t n, int64_t k,
               void* workspace, size_t workspace_bytes, void* stream) {
    return gemm_impl(device, semiring, dtype, layout, A, B, C, argmax, 1, m, n, k, 0, 0, 0, false,
                     workspace, workspace_bytes, true, stream);
}

int tg_gemm_strided_batched(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                            const void* A, const void* B, void* C, int32_t* argmax, int64_t batch,
                            int64_t m, int64_t n, int64_t k, int64_t stride_a, int64_t stride_b,
                            int64_t stride_c, void* stream) {
    return gemm_impl(device, semiring, dtype, layout, A, B, C, argmax, batch, m, n, k, stride_a,
                     stride_b, stride_c, true, nullptr, 0, false, stream);
}

int tg_gemm_strided_batched_ws(int device, tg_semiring semiring, tg_dtype dtype, tg_layout layout,
                               const void* A, const void* B, void* C, int32_t* argmax,
                               int64_t batch, int64_t m, int64_t n, int64_t k, int64_t stride_a,
                               int64_t stride_b, int64_t stride_c, void* workspace,
                               size_t workspace_bytes, void* stream) {
    return gemm_impl(device, semiring, dtype, layout, A, B, C, argmax, batch, m, n, k, stride_a,
                     stride_b, stride_c, true, workspace, workspace_bytes, true, stream);
}

int tg_backward_a(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                  const int32_t* argmax, void* grad_a, int64_t m, int64_t n, int64_t k,
                  void* stream) {
    return backward_impl(device, dtype, layout, true, grad_c, argmax, nullptr, grad_a, 1, m, n, k,
                         0, 0, 0, false, false, stream);
}

int tg_backward_b(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                  const int32_t* argmax, void* grad_b, int64_t m, int64_t n, int64_t k,
                  void* stream) {
    return backward_impl(device, dtype, layout, false, grad_c, argmax, nullptr, grad_b, 1, m, n, k,
                         0, 0, 0, false, false, stream);
}

int tg_maxmul_backward_a(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                         const int32_t* argmax, const void* B, void* grad_a, int64_t m, int64_t n,
                         int64_t k, void* stream) {
    return backward_impl(device, dtype, layout, true, grad_c, argmax, B, grad_a, 1, m, n, k, 0, 0,
                         0, false, true, stream);
}

int tg_maxmul_backward_b(int device, tg_dtype dtype, tg_layout layout, const void* grad_c,
                         const int32_t* argmax, const void* A, void* grad_b, int64_t m, int64_t n,
                         int64_t k, void* stream) {
    return backward_impl(device, dtype, layout, false, grad_c, argmax, A, grad_b, 1, m, n, k, 0, 0,
                         0, false, true, stream);
}

int tg_backward_a_strided_batched(int device, tg_dtype dtype, tg_layout layout,
                                  const void* grad_c, const int32_t* argmax, const void* other,
                                  void* grad_a, int64_t batch, int64_t m, int64_t n, int64_t k,
                                  int64_t stride_c, int64_t stride_other, int64_t stride_a,
                                  void* stream) {
    return backward_impl(device, dtype, layout, true, grad_c, argmax, other, grad_a, batch, m, n, k,
                         stride_c, stride_other, stride_a, true, other != nullptr, stream);
}

int tg_backward_b_strided_batched(int device, tg_dtype dtype, tg_layout layout,
                                  const void* grad_c, const int32_t* argmax, const void* other,
                                  void* grad_b, int64_t batch, int64_t m, int64_t n, int64_t k,
                                  int64_t stride_c, int64_t stride_other, int64_t stride_b,
                                  void* stream) {
    return backward_impl(device, dtype, layout, false, grad_c, argmax, other, grad_b, batch, m, n,
                         k, stride_c, stride_other, stride_b, true, other != nullptr, stream);
}

int tg_transpose(int device, tg_dtype dtype, const void* src, void* dst, int64_t batch,
                 int64_t rows, int64_t cols, void* stream) {
    if (!valid_dtype(dtype)) return fail(TG_ERR_INVALID_ARGUMENT, "unknown dtype " + std::to_string(dtype));
    if (batch < 0 || rows < 0 || cols < 0) return fail(TG_ERR_DIMENSION_MISMATCH, "negative dimension");
    if (rows > 0x7fffffffLL || cols > 0x7fffffffLL)
        return fail(TG_ERR_DIMENSION_MISMATCH, "dimension exceeds 2^31-1");
    if ((rows + 31) / 32 > 65535) return fail(TG_ERR_DIMENSION_MISMATCH, "rows too large for the transpose grid");
    const int64_t elems = rows * cols;
    if (batch > 0 && elems > 0 && (src == nullptr || dst == nullptr))
        return fail(TG_ERR_INVALID_ARGUMENT, "src or dst is NULL");
    int rc = select_device(device);
    if (rc != TG_OK) return rc;
    if (batch == 0 || elems == 0) return TG_OK;
    hipStream_t st = as_stream(stream);
    auto run = [&](auto tag) {
        using T = decltype(tag);
        const T* s = static_cast<const T*>(src);
        T* d = static_cast<T*>(dst);
        for (int64_t z0 = 0; z0 < batch; z0 += 65535) {
            const int64_t nb = (batch - z0 < 65535) ? batch - z0 : 65535;
            const int r = launch_transpose<T>(s + z0 * elems, d + z0 * elems, rows, cols, elems, elems,
                                              nb, st);
            if (r != TG_OK) return r;
        }
        return int(TG_OK);
    };
    switch (dtype) {
        case TG_F32: return run(float());
        case TG_F64: return run(double());
        case TG_I32: return run(int32_t());
        default: return run(int64_t());
    }
}

}  // extern "C"
