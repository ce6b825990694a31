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

// Value-only tropical sum (+): max or min.  Two nested calls on floats
// become one v_max3_f32 / v_min3_f32; on i32 one v_max3_i32 / v_min3_i32.
template <int SR, typename T>
__device__ __forceinline__ T tjoin(T acc, T p) {
    if constexpr (std::is_same<T, float>::value) {
        if constexpr (SR == SR_MINPLUS) return __builtin_fminf(acc, p);
        else return __builtin_fmaxf(acc, p);
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
// the reference's "keep acc iff acc >= p" (max) / "acc <= p" (min) rule.
template <int SR, typename T>
__device__ __forceinline__ bool tbetter(T cand, T acc) {
    if constexpr (SR == SR_MINPLUS) return cand < acc;
    else return cand > acc;
}

}  // namespace tg
