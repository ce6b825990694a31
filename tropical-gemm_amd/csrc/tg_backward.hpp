// tg_backward.hpp -- deterministic argmax-scatter backward (gfx950).
//
// Reference: the CPU backward visits i then j ascending and accumulates
// grad_A[i, argmax[i,j]] += dC[i,j] and grad_B[argmax[i,j], j] += dC[i,j]
// (crates/tropical-gemm/src/api.rs:563-582, 627-646), the MaxMul rule first
// multiplying dC[i,j] by the winning B or A value
// (crates/tropical-gemm-python/src/lib.rs:877-950); indices outside [0, K)
// are skipped.  Every gradient element is therefore a sequential f32/f64
// sum, starting from +0, of its contributions in ascending j (grad_A) or
// ascending i (grad_B).  Floating-point addition is not associative, so these
// kernels reproduce that order exactly instead of using atomics: the result
// is bit-identical to the reference and the same from run to run.
//
// Ordering inside a wave: a block of 64 consecutive contributions (one per
// lane, in lane order) is grouped by target bin with 64-bit ballots over the
// bits of the bin index (wave_match_rank: a lane's rank is the number of
// earlier lanes with the same bin); then the block is applied in rounds,
// round r adding the contributions of rank r.  Within a round all targets
// differ, and the rounds run in program order, so each bin sees its
// contributions in lane order; blocks run in sequence.  A block costs one
// round per repetition of its most repeated bin (one or two for spread
// indices); a block that repeats a bin more than kRoundsMax times sums each
// bin serially in a wave-uniform register instead (a near-constant argmax:
// the sequential chain the sum needs anyway).
//
// grad_A (tg_bwd_rows): one wave per row of C at a time, its K bins in LDS
// (rows are independent; the wave walks j in blocks of 64).
// grad_B (tg_bwd_cols): one wave per column of C, its K bins in LDS; a
// workgroup of W waves takes W adjacent columns and stages 64-row tiles of
// argmax and dC for them through LDS (coalesced row segments), and each wave
// walks i in blocks of 64.
// Both loop over their rows/columns with a grid stride, so any M, N and batch
// fit the launch (grid sizes come from bwd_*_geometry on the host).  Bins
// that do not fit LDS live in the gradient itself (GLOBAL instantiations):
// the same order, with coherent loads and stores to global memory.
#pragma once

#include "tg_kernels.hpp"

namespace tg {

// Rank of this lane's key among the active lanes of the wave holding the
// same key (the number of lower lanes with an equal key).  nbits: bits that
// can differ between keys (keys < 2^nbits).
__device__ __forceinline__ int wave_match_rank(uint32_t key, bool active, int nbits) {
    uint64_t match = __ballot(active);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1u;
        const uint64_t m = __ballot(active && bit);
        match &= bit ? m : ~m;
    }
    const int lane = threadIdx.x & 63;
    const uint64_t below = lane == 0 ? 0 : (~uint64_t(0) >> (64 - lane));
    return __popcll(match & below);
}

// Bits needed for keys in [0, K).
__host__ __device__ inline int key_bits(int64_t K) {
    int b = 0;
    while (b < 31 && (int64_t(1) << b) < K) ++b;
    return b;
}

// Wave-wide maximum of a small non-negative int.
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int y = __shfl_xor(x, off, 64);
        x = y > x ? y : x;
    }
    return x;
}

// Lane l's value of x (wave-uniform result).
template <typename T>
__device__ __forceinline__ T read_lane(T x, int l) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, x);
        const uint32_t lo = __builtin_amdgcn_readlane(uint32_t(u), l);
        const uint32_t hi = __builtin_amdgcn_readlane(uint32_t(u >> 32), l);
        return __builtin_bit_cast(T, (uint64_t(hi) << 32) | lo);
    }
}

// bins[key * es] += g in lane order among equal keys (see the header
// comment).  Up to kRoundsMax repetitions of a key: rounds of distinct-bin
// read-add-writes.  A block that repeats one bin more often than that (a
// near-constant argmax) sums each bin's contributions serially instead: the
// bin is read once, its lanes' values are added one by one in lane order in
// a wave-uniform register, and the sum is written once.
// GLOBAL: the bins are in global memory, read and written with relaxed
// device-scope atomics (coherent, in this wave's program order per address).
constexpr int kRoundsMax = 8;

template <typename T, bool GLOBAL>
__device__ __forceinline__ void ordered_add(T* bins, int64_t es, int32_t key, T g, bool active,
                                            int rank) {
    auto ld = [&](int64_t k) {
        if constexpr (GLOBAL)
            return __hip_atomic_load(bins + k * es, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            return bins[k];
    };
    auto st = [&](int64_t k, T v) {
        if constexpr (GLOBAL)
            __hip_atomic_store(bins + k * es, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            bins[k] = v;
    };
    // Global bins: this wave's stores complete before its next loads, so a
    // bin written by one lane is read back by another from L2.
    auto order = [&]() {
        if constexpr (GLOBAL) __threadfence_block();
    };
    if (wave_max(active ? rank : 0) < kRoundsMax) {
        for (int r = 0;; ++r) {
            const bool go = active && rank == r;
            if (__ballot(go) == 0) break;
            if (go) st(key, ld(key) + g);
            order();
        }
        return;
    }
    uint64_t todo = __ballot(active);
    while (todo) {
        const int leader = __builtin_ctzll(todo);
        const int32_t k = __builtin_amdgcn_readlane(key, leader);
        uint64_t grp = __ballot(active && key == k);
        todo &= ~grp;
        T acc = read_lane(ld(k), 0);  // every lane read the same bin
        while (grp) {
            acc = acc + read_lane(g, __builtin_ctzll(grp));
            grp &= grp - 1;
        }
        if ((threadIdx.x & 63) == 0) st(k, acc);
        order();
    }
}

// ---------------------------------------------------------------------------
// grad_A.  rows = batch * M; row rr is (z = rr / M, i = rr % M).  Each wave
// owns one row at a time; LDS: K bins per wave (dynamic, waves * K * T).
//   MULT: MaxMul rule, g *= B[z][k][j] (OTHER = B, row-major K x N).
// GLOBAL: the bins are the grad_A row itself (K too large for LDS).
// grid: any size (grid-stride over rows), block = 64 * waves.
// ---------------------------------------------------------------------------
template <typename T, bool MULT, bool GLOBAL>
__global__ __launch_bounds__(256) void tg_bwd_rows(const T* __restrict__ G,
                                                   const int32_t* __restrict__ IDX,
                                                   const T* __restrict__ OTHER, T* GA, int64_t M,
                                                   int64_t N, int64_t K, int64_t sC, int64_t sO,
                                                   int64_t sA, int64_t rows) {
    extern __shared__ __align__(16) unsigned char bwd_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves = blockDim.x >> 6;
    const int nbits = key_bits(K);
    for (int64_t rr = int64_t(blockIdx.x) * waves + wave; rr < rows;
         rr += int64_t(gridDim.x) * waves) {
        const int64_t z = rr / M, i = rr - z * M;
        const T* g_row = G + z * sC + i * N;
        const int32_t* k_row = IDX + z * sC + i * N;
        const T* other = MULT ? OTHER + z * sO : nullptr;
        T* out = GA + z * sA + i * K;
        T* bins = GLOBAL ? out : reinterpret_cast<T*>(bwd_lds) + int64_t(wave) * K;
        if constexpr (GLOBAL) {
            for (int64_t k = lane; k < K; k += 64)
                __hip_atomic_store(bins + k, T(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            for (int64_t k = lane; k < K; k += 64) bins[k] = T(0);
        }
        // Contributions in blocks of 64 consecutive j, the next block's
        // loads issued before the current one is applied.
        int32_t kn = lane < N ? k_row[lane] : -1;
        T gn = lane < N ? g_row[lane] : T(0);
        for (int64_t j0 = 0; j0 < N; j0 += 64) {
            const int32_t key = kn;
            T g = gn;
            const int64_t jn = j0 + 64 + lane;
            kn = jn < N ? k_row[jn] : -1;
            gn = jn < N ? g_row[jn] : T(0);
            const bool active = key >= 0 && int64_t(key) < K;
            if (MULT && active) g = g * other[int64_t(key) * N + j0 + lane];
            const int rank = wave_match_rank(uint32_t(key), active, nbits);
            ordered_add<T, GLOBAL>(bins, 1, key, g, active, rank);
        }
        if constexpr (!GLOBAL) {
            for (int64_t k = lane; k < K; k += 64) out[k] = bins[k];
        }
    }
}

// ---------------------------------------------------------------------------
// grad_B.  Column groups: batch * ceil(N / W) groups of W adjacent columns,
// W = waves per workgroup; group gg is (z = gg / groups_n, columns
// c0 = (gg % groups_n) * W ...).  Wave w owns column c0 + w and its K bins
// (LDS, or the grad_B column itself with GLOBAL).  Per 64-row block the
// workgroup stages argmax and dC for its W columns in LDS (row stride W + 1:
// the column reads of 64 lanes hit distinct banks), then each wave applies
// its column's 64 contributions in row order.
//   MULT: MaxMul rule, g *= A[z][i][k] (OTHER = A, row-major M x K).
// LDS: W * K bins (not with GLOBAL) + 64 (W + 1) (4 + sizeof(T)) bytes.
// grid: any size (grid-stride over column groups), block = 64 * W, W <= 8.
// ---------------------------------------------------------------------------
template <typename T, bool MULT, bool GLOBAL>
__global__ __launch_bounds__(512) void tg_bwd_cols(const T* __restrict__ G,
                                                   const int32_t* __restrict__ IDX,
                                                   const T* __restrict__ OTHER, T* GB, int64_t M,
                                                   int64_t N, int64_t K, int64_t sC, int64_t sO,
                                                   int64_t sB, int64_t groups_n, int64_t groups) {
    extern __shared__ __align__(16) unsigned char bwd_lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int W = blockDim.x >> 6;
    const int stride = W + 1;
    const int nbits = key_bits(K);
    T* bins_all = reinterpret_cast<T*>(bwd_lds);
    const int64_t bins_bytes = GLOBAL ? 0 : int64_t(W) * K * int64_t(sizeof(T));
    T* tile_g = reinterpret_cast<T*>(bwd_lds + bins_bytes);
    int32_t* tile_k = reinterpret_cast<int32_t*>(bwd_lds + bins_bytes + 64 * stride * sizeof(T));
    for (int64_t gg = blockIdx.x; gg < groups; gg += gridDim.x) {
        const int64_t z = gg / groups_n;
        const int64_t c0 = (gg - z * groups_n) * W;
        const int64_t c = c0 + wave;
        const T* gz = G + z * sC;
        const int32_t* kz = IDX + z * sC;
        const T* other = MULT ? OTHER + z * sO : nullptr;
        T* outz = GB + z * sB;
        T* bins = GLOBAL ? outz + c : bins_all + int64_t(wave) * K;
        const int64_t es = GLOBAL ? N : 1;
        if (c < N) {
            if constexpr (GLOBAL) {
                for (int64_t k = lane; k < K; k += 64)
                    __hip_atomic_store(bins + k * es, T(0), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            } else {
                for (int64_t k = lane; k < K; k += 64) bins[k] = T(0);
            }
        }
        for (int64_t i0 = 0; i0 < M; i0 += 64) {
            // Stage the 64 x W block (row i0 + r, column c0 + q) of argmax and dC.
            for (int e = tid; e < 64 * W; e += blockDim.x) {
                const int r = e / W, q = e - (e / W) * W;
                const int64_t i = i0 + r, cc = c0 + q;
                const bool ok = i < M && cc < N;
                tile_k[r * stride + q] = ok ? kz[i * N + cc] : -1;
                tile_g[r * stride + q] = ok ? gz[i * N + cc] : T(0);
            }
            __syncthreads();
            if (c < N) {
                const int32_t key = tile_k[lane * stride + wave];
                T g = tile_g[lane * stride + wave];
                const bool active = key >= 0 && int64_t(key) < K;
                if (MULT && active) g = g * other[(i0 + lane) * K + key];
                const int rank = wave_match_rank(uint32_t(key), active, nbits);
                ordered_add<T, GLOBAL>(bins, es, key, g, active, rank);
            }
            __syncthreads();
        }
        if constexpr (!GLOBAL) {
            // The W columns leave together: row k of the group is W
            // consecutive elements of grad_B.
            for (int64_t e = tid; e < int64_t(W) * K; e += blockDim.x) {
                const int64_t k = e / W;
                const int q = int(e - k * W);
                if (c0 + q < N) outz[k * N + c0 + q] = bins_all[int64_t(q) * K + k];
            }
            __syncthreads();  // the next group zeroes the bins
        }
    }
}

}  // namespace tg
