// tg_device.hpp -- device-side semiring algebra shared by every kernel.
//
// Semantics follow the reference CPU path (paths relative to the reference root):
//   tropical zero / one and scalar ops   crates/tropical-gemm/src/types/scalar.rs:32-126
//   MaxPlus / MinPlus / MaxMul           types/max_plus.rs:29-74, min_plus.rs:28-74,
//                                        max_mul.rs:28-73
// Integers use two's-complement wrapping (release-build Rust `+`/`*`), not the
// reference GPU's +-46340 saturating sentinels (tropical_gemm.cu:18-50).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace tg {

enum : int { SR_MAXPLUS = 0, SR_MINPLUS = 1, SR_MAXMUL = 2 };

// Tropical zero: the accumulator's initial value and the result when no
// product beats it (core/argmax.rs:24-33 initialises C with it).
template <int SR, typename T>
__device__ __forceinline__ T tzero() {
    if constexpr (std::is_floating_point<T>::value) {
        if constexpr (SR == SR_MAXPLUS) return -static_cast<T>(__builtin_huge_val());
        else if constexpr (SR == SR_MINPLUS) return static_cast<T>(__builtin_huge_val());
        else return T(0);
    } else {
        using U = typename std::make_unsigned<T>::type;
        constexpr U hi = U(1) << (sizeof(T) * 8 - 1);
        if constexpr (SR == SR_MAXPLUS) return static_cast<T>(hi);        // MIN
        else if constexpr (SR == SR_MINPLUS) return static_cast<T>(hi - 1);  // MAX
        else return T(0);
    }
}

// Tropical product (x): one IEEE add/mul for floats, wrapping add/mul for ints.
template <int SR, typename T>
__device__ __forceinline__ T tmul(T a, T b) {
    if constexpr (std::is_floating_point<T>::value) {
        if constexpr (SR == SR_MAXMUL) return a * b;
        else return a + b;
    } else {
        using U = typename std::make_unsigned<T>::type;
        if constexpr (SR == SR_MAXMUL) return static_cast<T>(static_cast<U>(a) * static_cast<U>(b));
        else return static_cast<T>(static_cast<U>(a) + static_cast<U>(b));
    }
}

// Tropical sum (+) of a chain: max or min.  Two nested calls become one
// three-operand instruction: on f32 v_maximum3_f32 / v_minimum3_f32, which
// return NaN when any operand is NaN (IEEE 754-2019 maximum/minimum), so a
// chain that met a NaN product ends NaN and the kernel can hand that output
// to the exact rule below (same issue rate as v_max3_f32, measured); on i32
// v_max3_i32 / v_min3_i32.  f64 has no NaN-propagating max on gfx950: its
// chunked kernel checks its operands for values that can make a NaN
// product instead.
template <int SR, typename T>
__device__ __forceinline__ T tjoin(T acc, T p) {
    if constexpr (std::is_same<T, float>::value) {
        if constexpr (SR == SR_MINPLUS) return __builtin_elementwise_minimum(acc, p);
        else return __builtin_elementwise_maximum(acc, p);
    } else if constexpr (std::is_same<T, double>::value) {
        if constexpr (SR == SR_MINPLUS) return __builtin_fmin(acc, p);
        else return __builtin_fmax(acc, p);
    } else {
        if constexpr (SR == SR_MINPLUS) return p < acc ? p : acc;
        else return p > acc ? p : acc;
    }
}

// Strict improvement test used at chunk boundaries: the new running value
// beats the value held before the chunk.  Equal values never replace, which is
// the reference's "keep acc iff acc >= p" (max) / "acc <= p" (min) rule for
// non-NaN values (chains that met a NaN are resolved by cpu_select instead).
template <int SR, typename T>
__device__ __forceinline__ bool tbetter(T cand, T acc) {
    if constexpr (SR == SR_MINPLUS) return cand < acc;
    else return cand > acc;
}

// The reference CPU select rule for one product, NaN included: replace
// (acc, idx) by (p, k) iff the reference would not keep acc, i.e. iff
// !(acc >= p) for MaxPlus/MaxMul and !(acc <= p) for MinPlus
// (types/max_plus.rs:66-73, min_plus.rs:66-73, max_mul.rs:65-72).  A NaN
// product therefore replaces any acc, and any product replaces a NaN acc.
// For integers and non-NaN floats this is the strict improvement of tbetter.
template <int SR, typename T>
__device__ __forceinline__ bool ttake(T p, T acc) {
    if constexpr (SR == SR_MINPLUS) return !(acc <= p);
    else return !(acc >= p);
}

// The reference CPU rule over one output's whole k range, serially: a[k * sa]
// and b[k * sb] for k ascending, from the tropical zero with index 0
// (core/argmax.rs:24-33, core/kernel.rs:119-167).  The exact fallback for
// outputs whose fast chain met a NaN product.
template <int SR, typename T>
__device__ __forceinline__ void cpu_select(const T* a, int64_t sa, const T* b, int64_t sb, int64_t K,
                                        T& acc, int32_t& idx) {
    T v = tzero<SR, T>();
    int32_t ix = 0;
    for (int64_t k = 0; k < K; ++k) {
        const T p = tmul<SR, T>(a[k * sa], b[k * sb]);
        if (ttake<SR, T>(p, v)) {
            v = p;
            ix = int32_t(k);
        }
    }
    acc = v;
    idx = ix;
}

// True for a value that is NaN (floats only).
template <typename T>
__device__ __forceinline__ bool tisnan(T x) {
    if constexpr (std::is_floating_point<T>::value) return x != x;
    else return false;
}

}  // namespace tg
