// tg_gemm_shortk.hpp -- tropical GEMM for short K (gfx950).
//
// At short K the product costs a few VALU ops per output against 4 (value) +
// 4 (argmax) bytes written per output, so the kernel is shaped for the
// writes rather than for operand reuse:
//   * 32 x 256 output tiles (16 x 256 for 64-bit types) taken in row-major
//     tile order; wave w of the 256-thread workgroup owns tile rows
//     R*w .. R*w+R-1 (R = 8, or 4 for 64-bit types) and lane l owns columns
//     4l .. 4l+3, so the wave's stores cover 1 KB (2 KB) runs of one row.
//     (A store probe on MI355X writing 2 x 512 MB: 1 KB row runs reach the
//     hipMemset rate, 6.5 TB/s; the 256 B runs of 128 x 64 tiles 5.8 TB/s.)
//   * A is wave-uniform: a wave reads its R rows' k values with scalar loads
//     (32 bytes per row and block) and the VALU takes them as SGPR operands.
//   * B rows are 16-byte vector loads, 1 KB per wave and k, served from L1/L2
//     (B is K x N, small at short K, and re-read by every wave).
//   * No LDS and at most 128 VGPRs (f32 argmax: 124), so 4 waves per SIMD
//     keep the products of some waves in flight while others store.
// ARGMAX: every product in k order updates (value, k) under the reference's
// select rule (ttake: strict improvement for non-NaN values, which keeps the
// first k attaining the optimum, core/argmax.rs:24-33 and
// core/kernel.rs:119-167; a NaN product replaces, as on the CPU); outputs
// that never beat the tropical zero keep it with argmax 0.
// Value-only: max3/min3 chains from the tropical zero (f32: NaN-propagating,
// with the serial rule for outputs that end NaN; f64: the select rule per
// product, since v_max_f64 drops NaN).
//
// Host-checked requirements: N % 4 == 0, B, C (and IDX) 16-byte aligned with
// batch strides sB, sC multiples of 4; any M >= 1, K >= 1.
// grid = (ceil(M / BM) * ceil(N / 256), 1, batch), block = 256.
#pragma once

#include <type_traits>

#include "tg_device.hpp"
#include "tg_kernels.hpp"

namespace tg {

template <typename T>
struct ShortkCfg {
    static constexpr int R = sizeof(T) == 4 ? 8 : 4;  // rows per wave
    static constexpr int KB = 32 / int(sizeof(T));    // k per scalar-load block
    static constexpr int BM = 4 * R, BN = 256;
};

template <int SR, typename T, bool ARGMAX>
__global__ __launch_bounds__(256) void tg_gemm_shortk(
    const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C,
    int32_t* __restrict__ IDX, int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB,
    int64_t sC, int tiles_n) {
    using Cfg = ShortkCfg<T>;
    constexpr int R = Cfg::R, KB = Cfg::KB;
    constexpr int VN = Vec16<T>::N;  // elements per 16-byte vector
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int tm = int(blockIdx.x) / tiles_n;
    const int tn = int(blockIdx.x) - tm * tiles_n;
    const int64_t z = blockIdx.z;
    A += z * sA;
    B += z * sB;
    C += z * sC;
    if constexpr (ARGMAX) IDX += z * sC;

    const int64_t r0 = int64_t(tm) * Cfg::BM + w * R;
    const int64_t col = int64_t(tn) * Cfg::BN + lane * 4;
    const bool col_ok = col < N;
    const int64_t colc = col_ok ? col : N - 4;  // in-range column quad for loads
    // Row pointers, wave-uniform; rows past M read row M-1 and store nothing.
    const T* arow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) arow[r] = A + (r0 + r < M ? r0 + r : M - 1) * K;

    T acc[R][4];
    int32_t ix[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[r][j] = tzero<SR, T>();
            ix[r][j] = 0;
        }

    // NK consecutive k from k0: A values through scalar loads, B quads
    // through vector loads, then the products in k order.
    auto block = [&](int64_t k0, auto nk) {
        constexpr int NK = decltype(nk)::value;
        T a[R][NK];
        T b[NK][4];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int kk = 0; kk < NK; ++kk) a[r][kk] = arow[r][k0 + kk];
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int h = 0; h < 4 / VN; ++h) {
                const Vec16<T> v =
                    *reinterpret_cast<const Vec16<T>*>(B + (k0 + kk) * N + colc + h * VN);
#pragma unroll
                for (int e = 0; e < VN; ++e) b[kk][h * VN + e] = v.v[e];
            }
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
            const int32_t kg = int32_t(k0 + kk);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                // The four compares of a row come before their selects, so no
                // select waits on the compare just issued (no hazard s_nop).
                T p[4];
                bool better[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) p[j] = tmul<SR, T>(a[r][kk], b[kk][j]);
                if constexpr (ARGMAX) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) better[j] = ttake<SR, T>(p[j], acc[r][j]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[r][j] = better[j] ? p[j] : acc[r][j];
                        ix[r][j] = better[j] ? kg : ix[r][j];
                    }
                } else if constexpr (std::is_same<T, double>::value) {
                    // v_max_f64 would drop a NaN product: the select rule.
#pragma unroll
                    for (int j = 0; j < 4; ++j) better[j] = ttake<SR, T>(p[j], acc[r][j]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[r][j] = better[j] ? p[j] : acc[r][j];
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[r][j] = tjoin<SR, T>(acc[r][j], p[j]);
                }
            }
        }
    };
    int64_t k0 = 0;
    for (; k0 + KB <= K; k0 += KB) block(k0, std::integral_constant<int, KB>());
    for (; k0 < K; ++k0) block(k0, std::integral_constant<int, 1>());

    if (!col_ok) return;
    if constexpr (!ARGMAX && std::is_same<T, float>::value) {
        // An f32 value chain that met a NaN product ends NaN: recompute it
        // with the reference's serial rule (K is short here).
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (tisnan(acc[r][j]) && r0 + r < M) {
                    int32_t unused;
                    cpu_select<SR, T>(A + (r0 + r) * K, 1, B + col + j, N, K, acc[r][j], unused);
                }
    }
    // Non-temporal stores where one instruction writes a contiguous 1 KB run
    // (32-bit C, and the argmax): 2-3% faster with argmax and 15% value-only
    // (65536 x 2048 x 16) than plain stores.  64-bit C stays plain: there a
    // 16-byte store covers every other 16 bytes of the run, and non-temporal
    // stores of such halves took f64 argmax (32768 x 2048 x 8) 137 -> 234 us.
    typedef uint32_t U4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r0 + r >= M) break;
        const int64_t off = (r0 + r) * N + col;
        if constexpr (VN == 4) {
            __builtin_nontemporal_store(*reinterpret_cast<const U4*>(acc[r]),
                                        reinterpret_cast<U4*>(C + off));
        } else {
#pragma unroll
            for (int h = 0; h < 4 / VN; ++h)
                reinterpret_cast<Vec16<T>*>(C + off)[h] =
                    reinterpret_cast<const Vec16<T>*>(acc[r])[h];
        }
        if constexpr (ARGMAX)
            __builtin_nontemporal_store(*reinterpret_cast<const U4*>(ix[r]),
                                        reinterpret_cast<U4*>(IDX + off));
    }
}

// Host-side shape check for tg_gemm_shortk (alignment of B, C, IDX and the
// batch strides; A needs only 4-byte alignment).
inline bool shortk_fits(int64_t M, int64_t N, int64_t K, int64_t sB, int64_t sC, const void* B,
                        const void* C, const void* IDX) {
    auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return M > 0 && N > 0 && K > 0 && N % 4 == 0 && sB % 4 == 0 && sC % 4 == 0 && al(B) &&
           al(C) && (IDX == nullptr || al(IDX)) && K <= 0x7fffffffLL;
}

}  // namespace tg
