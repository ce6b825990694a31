// tg_kernels.hpp -- gfx950 kernels of the tropical GEMM path.
//
// Kernel map (reference kernel each one replaces, tropical_gemm.cu):
//   tg_gemm_tiles      value-only and argmax GEMM for every dtype/semiring
//                      (TROPICAL_GEMM_{F32,F64,I32,I64} 86-520,
//                       TROPICAL_GEMM_ARGMAX_* 526-996, batched 1094-1219)
//   tg_transpose       B -> B^T staging for the argmax epilogue (new)
//   tg_fill_zero       zero fill used instead of hipMemsetAsync
// The backward scatters (TROPICAL_BACKWARD_A/B 1002-1036) are in
// tg_backward.hpp.
//
// All matrices are row-major here; the host layer maps column-major calls
// onto row-major ones with the operand swap C^T = B^T (x) A^T
// (kernels.rs:370-430 does the same trick in the other direction).
//
// Argmax scheme ("chunked argmax").  K is cut into chunks of CL consecutive k
// (TG_CHUNK = 32, one LDS k-tile, or an even part of it: 16 for 64-bit
// integers).  Inside a chunk each output folds its
// products into a chunk maximum with max/min only (two products per
// v_max3/v_min3).  At the chunk end one compare against the running value
// records the chunk index if the chunk strictly improved it.  Because max/min
// select an operand exactly and earlier chunks only lose on strict
// improvement, the first k attaining the final value lies in the recorded
// chunk; the kernel's epilogue finds it by recomputing that chunk's <= CL
// products (reading A and B^T rows) and takes the first k whose product
// equals the final value, writing both the index and that product's bits (so
// a -0/+0 tie keeps the first occurrence's sign, exactly like the CPU select
// rule).  The per-(i,j,k) VALU cost is one (x), half a max3 and 2/CL for the
// records instead of the four operations of a per-k compare-and-select.
#pragma once

#include "tg_device.hpp"

namespace tg {

constexpr int TG_CHUNK = 32;   // k per LDS tile == the default argmax chunk length
constexpr int TG_THREADS = 256;

// Tile shapes.  4-byte types: 128 x 64 output tile, 8 x 4 outputs per thread.
// 8-byte types: 64 x 64 output tile, 4 x 4 outputs per thread.
template <typename T>
struct TileCfg;
template <>
struct TileCfg<float> {
    static constexpr int BM = 128, BN = 64, TM = 8, TN = 4;
};
template <>
struct TileCfg<int32_t> {
    static constexpr int BM = 128, BN = 64, TM = 8, TN = 4;
};
template <>
struct TileCfg<double> {
    static constexpr int BM = 64, BN = 64, TM = 4, TN = 4;
};
template <>
struct TileCfg<int64_t> {
    static constexpr int BM = 64, BN = 64, TM = 4, TN = 4;
};

// 16-byte vector type of T (4 x 32-bit or 2 x 64-bit lanes).
template <typename T>
struct Vec16 {
    static constexpr int N = 16 / sizeof(T);
    T v[N];
};

// Block -> output tile.  Consecutive workgroup ids go round-robin over the 8
// XCDs; remap so each XCD owns a contiguous range of tiles, then walk that
// range in groups of 8 tile-rows so co-resident workgroups of one XCD share
// A and B panels in that XCD's L2.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    int lin = bid;
    if ((total & 7) == 0) lin = (bid & 7) * (total >> 3) + (bid >> 3);
    constexpr int GROUP = 8;
    const int per_group = GROUP * tiles_n;
    const int group = lin / per_group;
    const int first_m = group * GROUP;
    const int rem = tiles_m - first_m;
    const int gsize = rem < GROUP ? rem : GROUP;
    const int in_group = lin - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

// ---------------------------------------------------------------------------
// Main GEMM kernel.
//   ARGMAX=false : C = A (x) B.
//   ARGMAX=true  : C = A (x) B and IDX = the first k attaining C.  The main
//                  loop folds each chunk of CL consecutive k into a chunk
//                  maximum cm and records the chunk when cm strictly beats
//                  the running value; the epilogue then re-reads that
//                  chunk's A-row and B^T-row segments (BT from tg_transpose)
//                  and takes the first k whose product equals the final value.
//   CL           : argmax chunk length, TG_CHUNK / SUB.  Shorter chunks cost
//                  more records and shorten the windows the resolve reads
//                  (which miss L2): 64-bit integers use 16.
//   VEC          : K and N are multiples of 16/sizeof(T) and A, B, BT are
//                  16-byte aligned, so tiles and argmax windows use 16-byte
//                  global loads.
//   EXACT        : (with ARGMAX) every product updates (value, index) on a
//                  strict improvement, in k order: no chunk records, no
//                  resolve and no B^T.  For short K, where the resolve's
//                  re-reads of A and B^T would outweigh the main loop.
// grid = (tiles_m * tiles_n, 1, batch), block = 256.
// ---------------------------------------------------------------------------
template <int SR, typename T, bool ARGMAX, bool VEC, bool EXACT = false, int CL = TG_CHUNK>
__global__ __launch_bounds__(TG_THREADS) void tg_gemm_tiles(
    const T* __restrict__ A, const T* __restrict__ B, const T* __restrict__ BT,
    T* __restrict__ C, int32_t* __restrict__ IDX, int64_t M, int64_t N, int64_t K, int64_t sA,
    int64_t sB, int64_t sC, int tiles_m, int tiles_n) {
    using Cfg = TileCfg<T>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, TM = Cfg::TM, TN = Cfg::TN, BK = TG_CHUNK;
    constexpr int VW = Vec16<T>::N;          // elements per 16-byte vector
    constexpr int PAD = VW;                  // keeps 16-byte alignment of LDS rows
    constexpr int NVA = BM * BK / VW / TG_THREADS;  // 16-byte vectors of A per thread
    constexpr int NVB = BK * BN / VW / TG_THREADS;  // 16-byte vectors of B per thread
    static_assert(NVA >= 1 && NVB >= 1, "tile too small for the block");
    static_assert(TM % 4 == 0 && TN % 4 == 0, "micro-tile must be made of 4-wide groups");
    static_assert(ARGMAX || !EXACT, "EXACT is an argmax mode");
    static_assert(BK % CL == 0 && CL % 8 == 0, "argmax chunks split the k-tile evenly");
    constexpr int SUB = BK / CL;  // argmax chunks per k-tile

    __shared__ __align__(16) T As[2][BK][BM + PAD];
    __shared__ __align__(16) T Bs[2][BK][BN + PAD];

    const int tid = threadIdx.x;
    const int tx = tid & 15;
    const int ty = tid >> 4;
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t row0 = int64_t(tm) * BM;
    const int64_t col0 = int64_t(tn) * BN;
    const int64_t z = blockIdx.z;
    A += z * sA;
    B += z * sB;
    C += z * sC;
    if (ARGMAX) {
        IDX += z * sC;
        if (!EXACT) BT += z * (N * K);
    }

    // ---- global -> register staging ------------------------------------
    // f64 chains use v_max_f64 / v_min_f64, which drop NaN operands, so a
    // NaN product would vanish from a chain.  NaN products come only from NaN
    // operands or from infinities meeting (+inf + -inf; 0 * inf for MaxMul):
    // the loads classify every in-bounds operand (one v_cmp_class each into
    // wave masks), and a tile whose operands could make a NaN product is
    // recomputed with the reference's serial rule in the epilogue.
    // The wave's findings are bits of one wave-uniform word (A: nan, c1, c2
    // at bits 0-2; B at 3-5): one combined class test per operand, and the
    // three separate ones only when the wave holds a special value (64-bit
    // ballot masks per class kept the SGPRs busy enough to spill).
    constexpr bool CHECK = std::is_same<T, double>::value && !EXACT;
    constexpr int CLS1 = SR == SR_MAXMUL ? 516 : 512;  // +-inf | +inf
    constexpr int CLS2 = SR == SR_MAXMUL ? 96 : 4;     // +-0   | -inf
    uint32_t fl = 0;
    __shared__ int danger_flags;
    if (CHECK && tid == 0) danger_flags = 0;
    auto classify = [&](bool inb, T x, int o) {
        if constexpr (CHECK) {
            if (__any(inb && __builtin_amdgcn_class(x, 3 | CLS1 | CLS2))) {
                fl |= (__any(inb && __builtin_amdgcn_class(x, 3)) ? 1u : 0u) << o;
                fl |= (__any(inb && __builtin_amdgcn_class(x, CLS1)) ? 2u : 0u) << o;
                fl |= (__any(inb && __builtin_amdgcn_class(x, CLS2)) ? 4u : 0u) << o;
            }
        }
    };
    Vec16<T> ra[NVA], rb[NVB];
    auto load_tiles = [&](int64_t k0) {
#pragma unroll
        for (int v = 0; v < NVA; ++v) {
            const int L = v * TG_THREADS + tid;
            const int r = L / (BK / VW);
            const int kq = (L % (BK / VW)) * VW;
            const int64_t gr = row0 + r;
            const int64_t gk = k0 + kq;
            if constexpr (VEC) {
                if (gr < M && gk < K) {
                    ra[v] = *reinterpret_cast<const Vec16<T>*>(A + gr * K + gk);
                } else {
#pragma unroll
                    for (int e = 0; e < VW; ++e) ra[v].v[e] = T(0);
                }
            } else {
#pragma unroll
                for (int e = 0; e < VW; ++e)
                    ra[v].v[e] = (gr < M && gk + e < K) ? A[gr * K + gk + e] : T(0);
            }
#pragma unroll
            for (int e = 0; e < VW; ++e) classify(gr < M && gk + e < K, ra[v].v[e], 0);
        }
#pragma unroll
        for (int v = 0; v < NVB; ++v) {
            const int L = v * TG_THREADS + tid;
            const int kr = L / (BN / VW);
            const int nq = (L % (BN / VW)) * VW;
            const int64_t gk = k0 + kr;
            const int64_t gc = col0 + nq;
            if constexpr (VEC) {
                if (gk < K && gc < N) {
                    rb[v] = *reinterpret_cast<const Vec16<T>*>(B + gk * N + gc);
                } else {
#pragma unroll
                    for (int e = 0; e < VW; ++e) rb[v].v[e] = T(0);
                }
            } else {
#pragma unroll
                for (int e = 0; e < VW; ++e)
                    rb[v].v[e] = (gk < K && gc + e < N) ? B[gk * N + gc + e] : T(0);
            }
#pragma unroll
            for (int e = 0; e < VW; ++e) classify(gk < K && gc + e < N, rb[v].v[e], 3);
        }
    };
    auto store_tiles = [&](int buf) {
#pragma unroll
        for (int v = 0; v < NVA; ++v) {
            const int L = v * TG_THREADS + tid;
            const int r = L / (BK / VW);
            const int kq = (L % (BK / VW)) * VW;
#pragma unroll
            for (int e = 0; e < VW; ++e) As[buf][kq + e][r] = ra[v].v[e];
        }
#pragma unroll
        for (int v = 0; v < NVB; ++v) {
            const int L = v * TG_THREADS + tid;
            const int kr = L / (BN / VW);
            const int nq = (L % (BN / VW)) * VW;
            *reinterpret_cast<Vec16<T>*>(&Bs[buf][kr][nq]) = rb[v];
        }
    };

    // ---- accumulators ------------------------------------------------------
    // acc: running value; ch: last chunk that strictly improved it (-1: none,
    // i.e. the tropical zero was never beaten).  EXACT: ch is the argmax
    // itself, 0 until a product beats the zero.
    T acc[TM][TN];
    int32_t ch[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            acc[i][j] = tzero<SR, T>();
            ch[i][j] = EXACT ? 0 : -1;
        }

    auto load_frag = [&](int buf, int kk, T (&a)[TM], T (&b)[TN]) {
#pragma unroll
        for (int g = 0; g < TM / 4; ++g) {
#pragma unroll
            for (int e = 0; e < 4; ++e) a[g * 4 + e] = As[buf][kk][g * 64 + ty * 4 + e];
        }
#pragma unroll
        for (int g = 0; g < TN / 4; ++g) {
#pragma unroll
            for (int e = 0; e < 4; ++e) b[g * 4 + e] = Bs[buf][kk][g * 64 + tx * 4 + e];
        }
    };

    const int64_t ntiles = (K + BK - 1) / BK;
    if (ntiles > 0) {
        load_tiles(0);
        store_tiles(0);
    }
    __syncthreads();

    for (int64_t t = 0; t < ntiles; ++t) {
        const int buf = int(t & 1);
        const int64_t k0 = t * BK;
        if (t + 1 < ntiles) load_tiles(k0 + BK);

        if constexpr (EXACT) {
            // Every product in k order under the reference's select rule
            // (ttake: strict improvement for non-NaN values, so the first k
            // is kept; a NaN product replaces, as on the CPU).
            auto step = [&](int kk) {
                T a0[TM], b0[TN];
                load_frag(buf, kk, a0, b0);
                const int32_t kg = int32_t(k0 + kk);
                if constexpr (sizeof(T) == 8) {
                    // A row's compares come before their selects, so no
                    // select waits on the compare just issued (no hazard
                    // s_nop): 7% faster for 64-bit types.  For 32-bit types
                    // the grouping needs 175 VGPRs instead of 155 (2 waves per
                    // SIMD instead of 3) and was 9-15% slower.
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        T p[TN];
                        bool better[TN];
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            p[j] = tmul<SR, T>(a0[i], b0[j]);
                            better[j] = ttake<SR, T>(p[j], acc[i][j]);
                        }
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            acc[i][j] = better[j] ? p[j] : acc[i][j];
                            ch[i][j] = better[j] ? kg : ch[i][j];
                        }
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const T p = tmul<SR, T>(a0[i], b0[j]);
                            const bool better = ttake<SR, T>(p, acc[i][j]);
                            acc[i][j] = better ? p : acc[i][j];
                            ch[i][j] = better ? kg : ch[i][j];
                        }
                }
            };
            const int kcnt = k0 + BK <= K ? BK : int(K - k0);
#pragma unroll 4
            for (int kk = 0; kk < kcnt; ++kk) step(kk);
            if (t + 1 < ntiles) store_tiles(buf ^ 1);
            __syncthreads();
            continue;
        }
        // Chunk maximum (minimum for MinPlus) over each chunk's products, then
        // its record.  Strict improvement only: an equal chunk maximum keeps
        // the earlier chunk, which is the reference's "keep acc iff acc >= p"
        // rule.
        auto fold = [&](T (&cm)[TM][TN], int32_t chunk) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (ARGMAX) {
                        if (tbetter<SR, T>(cm[i][j], acc[i][j])) ch[i][j] = chunk;
                    }
                    acc[i][j] = tjoin<SR, T>(acc[i][j], cm[i][j]);
                }
        };
        const bool full = k0 + BK <= K;
        const int kcnt = full ? BK : int(K - k0);
#pragma unroll
        for (int s = 0; s < SUB; ++s) {
            const int kb = s * CL;
            if (kb >= kcnt) break;
            T cm[TM][TN];
            if (full) {
                T a0[TM], b0[TN], a1[TM], b1[TN];
                load_frag(buf, kb, a0, b0);
                load_frag(buf, kb + 1, a1, b1);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        cm[i][j] = tjoin<SR, T>(tmul<SR, T>(a0[i], b0[j]), tmul<SR, T>(a1[i], b1[j]));
                // Remaining products two at a time: one max3/min3 per pair.
#pragma unroll
                for (int kk = kb + 2; kk < kb + CL; kk += 2) {
                    load_frag(buf, kk, a0, b0);
                    load_frag(buf, kk + 1, a1, b1);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const T p0 = tmul<SR, T>(a0[i], b0[j]);
                            const T p1 = tmul<SR, T>(a1[i], b1[j]);
                            cm[i][j] = tjoin<SR, T>(tjoin<SR, T>(cm[i][j], p0), p1);
                        }
                }
            } else {
                // Ragged last k-tile: only k < K may enter the reduction.
                const int ke = kb + CL < kcnt ? kb + CL : kcnt;
                T a0[TM], b0[TN];
                load_frag(buf, kb, a0, b0);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) cm[i][j] = tmul<SR, T>(a0[i], b0[j]);
                for (int kk = kb + 1; kk < ke; ++kk) {
                    load_frag(buf, kk, a0, b0);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            cm[i][j] = tjoin<SR, T>(cm[i][j], tmul<SR, T>(a0[i], b0[j]));
                }
            }
            fold(cm, int32_t(t * SUB + s));
        }

        if (t + 1 < ntiles) store_tiles(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue ------------------------------------------------------------
    // Outputs computed with the reference's serial rule instead of the fast
    // chain: f32 chains that met a NaN product (they end NaN), and every
    // output of an f64 tile whose operands could make one (CHECK above).
    bool danger = false;
    if constexpr (CHECK) {
        const int w = int(fl);
        if ((tid & 63) == 0 && w != 0) atomicOr(&danger_flags, w);
        __syncthreads();
        const int f = danger_flags;
        danger = (f & 1) || (f & 8) || ((f & 2) && (f & 32)) || ((f & 4) && (f & 16));
    }
    auto exact = [&](int64_t gr, int64_t gc, T& v, int32_t& ix) {
        if constexpr (ARGMAX && !EXACT)
            cpu_select<SR, T>(A + gr * K, 1, BT + gc * K, 1, K, v, ix);
        else
            cpu_select<SR, T>(A + gr * K, 1, B + gc, N, K, v, ix);
    };
    // Row i of the thread's values and indices as they stand in acc / ch (the
    // chunked argmax writes a row's resolved outputs back there first, so the
    // row's registers are free after its stores).  Each thread's columns come in
    // groups of 4 consecutive ones: one 16-byte store per group and array
    // when the rows are 16-byte aligned, element stores at the ragged right
    // edge or otherwise.
    const bool vec_out = N % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & 15u) == 0 &&
                         (!ARGMAX || (reinterpret_cast<uintptr_t>(IDX) & 15u) == 0);
    auto store_row = [&](const int i) {
        const int64_t gr = row0 + (i / 4) * 64 + ty * 4 + (i % 4);
        if (gr >= M) return;
#pragma unroll
        for (int g = 0; g < TN / 4; ++g) {
            const int64_t gc = col0 + g * 64 + tx * 4;
            if (vec_out && gc + 3 < N) {
                T cv[4];
                int32_t iv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    cv[e] = acc[i][g * 4 + e];
                    iv[e] = ch[i][g * 4 + e];
                }
                static_assert(sizeof(cv) % 16 == 0, "4 values make whole 16-byte vectors");
#pragma unroll
                for (int w = 0; w < int(sizeof(cv)) / 16; ++w) {
                    if constexpr (!ARGMAX) {
                        // Value-only: non-temporal (streaming) stores,
                        // 8-15% faster at short K on MI355X; with argmax
                        // they were 10-20% slower, so plain stores there.
                        typedef int v4i_t __attribute__((ext_vector_type(4)));
                        v4i_t x;
                        __builtin_memcpy(&x, reinterpret_cast<const char*>(cv) + 16 * w, 16);
                        __builtin_nontemporal_store(
                            x, reinterpret_cast<v4i_t*>(C + gr * N + gc) + w);
                    } else {
                        reinterpret_cast<Vec16<T>*>(C + gr * N + gc)[w] =
                            reinterpret_cast<const Vec16<T>*>(cv)[w];
                    }
                }
                if constexpr (ARGMAX)
                    *reinterpret_cast<Vec16<int32_t>*>(IDX + gr * N + gc) =
                        *reinterpret_cast<const Vec16<int32_t>*>(iv);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (gc + e < N) {
                        C[gr * N + gc + e] = acc[i][g * 4 + e];
                        if constexpr (ARGMAX) IDX[gr * N + gc + e] = ch[i][g * 4 + e];
                    }
                }
            }
        }
    };
    if constexpr (!ARGMAX || EXACT) {
        if constexpr (!EXACT) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int64_t gr = row0 + (i / 4) * 64 + ty * 4 + (i % 4);
                    const int64_t gc = col0 + (j / 4) * 64 + tx * 4 + (j % 4);
                    if ((danger || tisnan(acc[i][j])) && gr < M && gc < N) {
                        int32_t ix;
                        exact(gr, gc, acc[i][j], ix);
                    }
                }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) store_row(i);
    } else {
        // Exact argmax inside the recorded chunk.  Products in the chunk
        // before it never equal the final value (that chunk would not have
        // been beaten strictly), so a 16-byte-aligned window of CL products
        // ending at K may be searched for the ragged last chunk.  The value
        // written is the bits of the first equal product, so a -0/+0 tie
        // keeps the first occurrence's sign like the CPU rule.
        constexpr int NW = CL / VW;  // 16-byte vectors per window
        // Outputs with windows in flight: two while a window is one 128-byte
        // line per operand.
        constexpr int G = CL * int(sizeof(T)) <= 128 ? 2 : 1;
        const bool vec_windows = VEC && K >= CL;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t gr = row0 + (i / 4) * 64 + ty * 4 + (i % 4);
            const int64_t grl = gr < M ? gr : M - 1;  // clamped row for loads
#pragma unroll
            for (int j0 = 0; j0 < TN; j0 += G) {
                T val[G];
                int32_t idx[G];
                int64_t gc[G];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    gc[g] = col0 + ((j0 + g) / 4) * 64 + tx * 4 + ((j0 + g) % 4);
                    val[g] = acc[i][j0 + g];
                    idx[g] = 0;
                }
                if (vec_windows) {
                    Vec16<T> av[G][NW], bv[G][NW];
                    const T* ap[G];
                    const T* bp[G];
                    int64_t ws[G];
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const int64_t gcl = gc[g] < N ? gc[g] : N - 1;
                        const int64_t c = ch[i][j0 + g] < 0 ? 0 : ch[i][j0 + g];
                        ws[g] = (c * CL < K - CL) ? c * CL : K - CL;
                        ap[g] = A + grl * K + ws[g];
                        bp[g] = BT + gcl * K + ws[g];
#pragma unroll
                        for (int w = 0; w < NW; ++w) {
                            av[g][w] = reinterpret_cast<const Vec16<T>*>(ap[g])[w];
                            bv[g][w] = reinterpret_cast<const Vec16<T>*>(bp[g])[w];
                        }
                    }
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const T target = val[g];
                        // Last match scanning downwards == first match.  Groups
                        // of 8 compares keep few lane masks live at once.
                        int32_t f = 0;
#pragma unroll
                        for (int q = CL / 8 - 1; q >= 0; --q) {
#pragma unroll
                            for (int kk = q * 8 + 7; kk >= q * 8; --kk) {
                                const T p = tmul<SR, T>(av[g][kk / VW].v[kk % VW],
                                                        bv[g][kk / VW].v[kk % VW]);
                                f = (p == target) ? kk : f;
                            }
                            __builtin_amdgcn_sched_barrier(0);
                        }
                        idx[g] = int32_t(ws[g] + f);
                        if constexpr (std::is_floating_point<T>::value) {
                            // Equal values have equal bits except +0/-0: take
                            // the sign of the first zero product (rare branch).
                            if (target == T(0)) val[g] = tmul<SR, T>(ap[g][f], bp[g][f]);
                        }
                    }
                } else {
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        const int32_t c = ch[i][j0 + g];
                        if (gr < M && gc[g] < N && c >= 0) {
                            const T target = val[g];
                            const int64_t k0 = int64_t(c) * CL;
                            const int64_t k1 = (k0 + CL < K) ? k0 + CL : K;
                            idx[g] = int32_t(k0);
                            for (int64_t k = k0; k < k1; ++k) {
                                const T p = tmul<SR, T>(A[gr * K + k], BT[gc[g] * K + k]);
                                if (p == target) {
                                    idx[g] = int32_t(k);
                                    val[g] = p;
                                    break;
                                }
                            }
                        }
                    }
                }
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    if (ch[i][j0 + g] < 0) {  // the tropical zero was never beaten
                        val[g] = tzero<SR, T>();
                        idx[g] = 0;
                    }
                    if (gr < M && gc[g] < N && (danger || tisnan(acc[i][j0 + g])))
                        exact(gr, gc[g], val[g], idx[g]);
                    acc[i][j0 + g] = val[g];
                    ch[i][j0 + g] = idx[g];
                }
            }
            store_row(i);
        }
    }
}

// ---------------------------------------------------------------------------
// BT[z][j][k] = B[z][k][j]   (K x N -> N x K), 32 x 32 tiles through LDS.
// grid = (ceil(N/32), ceil(K/32), batch), block = (32, 8).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void tg_transpose(const T* __restrict__ B, T* __restrict__ BT,
                                                    int64_t K, int64_t N, int64_t sB, int64_t sBT) {
    __shared__ T tile[32][33];
    const int64_t z = blockIdx.z;
    B += z * sB;
    BT += z * sBT;
    const int64_t n0 = int64_t(blockIdx.x) * 32;
    const int64_t k0 = int64_t(blockIdx.y) * 32;
    const int x = threadIdx.x, y = threadIdx.y;
#pragma unroll
    for (int r = y; r < 32; r += 8) {
        const int64_t k = k0 + r, n = n0 + x;
        if (k < K && n < N) tile[r][x] = B[k * N + n];
    }
    __syncthreads();
#pragma unroll
    for (int r = y; r < 32; r += 8) {
        const int64_t n = n0 + r, k = k0 + x;
        if (k < K && n < N) BT[n * K + k] = tile[x][r];
    }
}

// Operand classes for the NaN check of the f64 kernel: bits of a row of A or
// a column of B.
enum : uint32_t { TG_CLS_NAN = 1, TG_CLS_PINF = 2, TG_CLS_NINF = 4, TG_CLS_ZERO = 8 };

__device__ __forceinline__ uint32_t tclass(double x) {
    uint32_t c = 0;
    if (x != x) c |= TG_CLS_NAN;
    if (x == __builtin_huge_val()) c |= TG_CLS_PINF;
    if (x == -__builtin_huge_val()) c |= TG_CLS_NINF;
    if (x == 0.0) c |= TG_CLS_ZERO;
    return c;
}

// ---------------------------------------------------------------------------
// The same with 16-byte vectors (VW = 16 / sizeof(T) elements) on 64 x 64
// tiles: every load reads VW columns of a row of B, every store writes VW
// k of a row of B^T.  Requires K and N multiples of VW, 16-byte aligned B and
// BT, and batch strides multiples of VW (then a vector is either wholly in
// the matrix or wholly out).  The LDS rows are padded to 65 elements, which
// spreads the column reads of a wave over the banks.  With T = double and
// cls non-null, the loads also OR the class bits of each column of B into
// cls[z*N + j] (zeroed beforehand; atomics only for columns with a bit set),
// so the f64 kernel needs no separate column pass.
// grid = (ceil(N/64), ceil(K/64), batch), block = 256.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void tg_transpose_v(const T* __restrict__ B, T* __restrict__ BT,
                                                      int64_t K, int64_t N, int64_t sB, int64_t sBT,
                                                      uint32_t* __restrict__ cls) {
    constexpr int VW = Vec16<T>::N;
    constexpr int TS = 64, LD = TS + 1;
    constexpr int VPR = TS / VW;    // vectors per tile row
    constexpr int RPP = 256 / VPR;  // tile rows per pass
    __shared__ T tile[TS * LD];
    const int64_t z = blockIdx.z;
    B += z * sB;
    BT += z * sBT;
    const int64_t n0 = int64_t(blockIdx.x) * TS;
    const int64_t k0 = int64_t(blockIdx.y) * TS;
    const int v = threadIdx.x % VPR, r = threadIdx.x / VPR;
    uint32_t cl[VW] = {};
#pragma unroll
    for (int rr = r; rr < TS; rr += RPP) {  // rr: k in the tile, v: a vector of n
        const int64_t k = k0 + rr, n = n0 + v * VW;
        if (k < K && n < N) {
            const Vec16<T> x = *reinterpret_cast<const Vec16<T>*>(B + k * N + n);
#pragma unroll
            for (int e = 0; e < VW; ++e) {
                tile[rr * LD + v * VW + e] = x.v[e];
                if constexpr (std::is_same<T, double>::value) cl[e] |= tclass(x.v[e]);
            }
        }
    }
    if constexpr (std::is_same<T, double>::value) {
        if (cls != nullptr) {
#pragma unroll
            for (int e = 0; e < VW; ++e)
                if (cl[e]) atomicOr(cls + z * N + n0 + v * VW + e, cl[e]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int rr = r; rr < TS; rr += RPP) {  // rr: n in the tile, v: a vector of k
        const int64_t n = n0 + rr, k = k0 + v * VW;
        if (n < N && k < K) {
            Vec16<T> y;
#pragma unroll
            for (int e = 0; e < VW; ++e) y.v[e] = tile[(v * VW + e) * LD + rr];
            *reinterpret_cast<Vec16<T>*>(BT + n * K + k) = y;
        }
    }
}

// ---------------------------------------------------------------------------
// Zero fill (16-byte stores + byte tail).  Used instead of hipMemsetAsync so
// that the library records no memset nodes when a caller captures a graph.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void tg_fill_zero(unsigned char* __restrict__ p, int64_t bytes) {
    const int64_t nvec = bytes / 16;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t v = int64_t(blockIdx.x) * 256 + threadIdx.x; v < nvec; v += stride)
        reinterpret_cast<uint4*>(p)[v] = make_uint4(0u, 0u, 0u, 0u);
    const int64_t tail0 = nvec * 16;
    for (int64_t b = tail0 + int64_t(blockIdx.x) * 256 + threadIdx.x; b < bytes; b += stride) p[b] = 0;
}

// Zeroes `batch` runs of `len` elements, run z starting at p + z * stride
// (element stores: any alignment, gaps between the runs untouched).  Grid:
// x strides over a run, y over the runs.
template <typename T>
__global__ __launch_bounds__(256) void tg_fill_zero_runs(T* __restrict__ p, int64_t len,
                                                          int64_t batch, int64_t stride) {
    const int64_t step = int64_t(gridDim.x) * 256;
    for (int64_t z = blockIdx.y; z < batch; z += gridDim.y) {
        T* run = p + z * stride;
        for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < len; e += step) run[e] = T(0);
    }
}

}  // namespace tg
