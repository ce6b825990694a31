// tg_gemm_kres.hpp -- K-resident tropical GEMM with argmax for short K (gfx950).
//
// Same contract as tg_gemm_dl with ARGMAX=true, for 32-bit types and
// K <= 32 * KRES_KT_MAX (tall-skinny products such as Viterbi steps, where
// K is small and M is large).  The whole K extent of the workgroup's A rows
// and B columns stays in LDS for the life of the workgroup, so the argmax
// epilogue resolves every recorded chunk from LDS: no B^T staging kernel, no
// global re-reads and no chunk sort.
//
// Layouts (one slot per 32-k tile t, never overwritten):
//   A tile t  64 rows x 32 k, row-major (128 B rows); the 16-byte quad q of
//             row r sits at quad position q ^ ((r >> 2) & 7), so the four
//             rows a wave reads at one k fall in different banks.
//   B tile t  32 k x 64 cols, row-major (256 B rows).
// All tiles are requested up front with global_load_lds_dwordx4 and waited
// for once.
//
// Each thread owns 4 consecutive rows (ty*4 + i) and 4 consecutive columns
// (tx*4 + j).  Argmax chunks are KRES_CL = 8 consecutive k: with K <= 128
// that balances the per-chunk bookkeeping (3 ops per output per chunk)
// against the resolve (about 4 ops per product of one chunk).
#pragma once

#include "tg_gemm_dl.hpp"

namespace tg {

constexpr int KRES_KT_MAX = 4;  // K <= 128

struct KresCfg {
    static constexpr int BM = 64, BN = 64, BK = 32, TM = 4, TN = 4, CL = 8;
    static constexpr int A_TILE = BM * BK;            // elements per A k-tile
    static constexpr int B_TILE = BK * BN;            // elements per B k-tile
    static constexpr int NBI = BK * BN * 4 / 1024 / 4;  // 1 KB B loads per wave per tile
    static constexpr int RPI = 256 / BN;              // B k-rows per 1 KB load
    static constexpr int LPR = BN / 4;                // lanes per B k-row
};

// True when tg_gemm_kres can run the problem: full 64 x 64 tiles, K a
// multiple of 32 from 64 up to 32 * KRES_KT_MAX, 16-byte aligned operands,
// outputs and batch strides.  (K = 32 goes to tg_gemm_dl: with a single
// k-tile the compiler interleaves the epilogue with the main loop and
// spills.)
inline bool kres_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, int64_t sC,
                      const void* A, const void* B, const void* C, const void* IDX) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return M > 0 && N > 0 && K > 0 && M % KresCfg::BM == 0 && N % KresCfg::BN == 0 &&
           K % KresCfg::BK == 0 && K >= 2 * KresCfg::BK &&
           K <= int64_t(KresCfg::BK) * KRES_KT_MAX && sA % 4 == 0 &&
           sB % 4 == 0 && sC % 4 == 0 && a16(A) && a16(B) && a16(C) && a16(IDX);
}

// grid = (tiles_m * tiles_n, 1, batch), block = 256.  K = 32 * KT.
template <int SR, typename T, int KT>
__global__ __launch_bounds__(TG_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void tg_gemm_kres(
    const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C,
    int32_t* __restrict__ IDX, int64_t M, int64_t N, int64_t sA, int64_t sB, int64_t sC,
    int tiles_m, int tiles_n) {
    static_assert(sizeof(T) == 4, "K-resident kernel is for 32-bit types");
    static_assert(KT >= 2 && KT <= KRES_KT_MAX, "K-resident tile count");
    using Cfg = KresCfg;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, TM = Cfg::TM, TN = Cfg::TN;
    constexpr int CL = Cfg::CL, NBI = Cfg::NBI;
    constexpr int K = KT * BK;
    constexpr int CPT = BK / CL;  // chunks per k-tile
    __shared__ __align__(16) T As[KT * Cfg::A_TILE];
    __shared__ __align__(16) T Bs[KT * Cfg::B_TILE];
    (void)M;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    IDX += z * sC;

    // Every tile's direct loads, in tile order.  A: 8 rows per 1 KB
    // instruction, wave w issues instructions 2w, 2w+1 of each tile.  B: RPI
    // k-rows per instruction, wave w issues NBI*w .. NBI*w + NBI-1.
    {
        const T* srcA[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int r = (wave * 2 + q) * 8 + (lane >> 3);
            const int qsrc = (lane & 7) ^ ((r >> 2) & 7);
            srcA[q] = A + (row0 + r) * K + qsrc * 4;
        }
        const T* srcB[NBI];
#pragma unroll
        for (int q = 0; q < NBI; ++q) {
            const int kr = (wave * NBI + q) * Cfg::RPI + lane / Cfg::LPR;
            srcB[q] = B + int64_t(kr) * N + col0 + (lane % Cfg::LPR) * 4;
        }
#pragma unroll
        for (int t = 0; t < KT; ++t) {
#pragma unroll
            for (int q = 0; q < 2; ++q)
                lds_load16(srcA[q] + t * BK, As + t * Cfg::A_TILE + (wave * 2 + q) * 256);
#pragma unroll
            for (int q = 0; q < NBI; ++q)
                lds_load16(srcB[q] + int64_t(t) * BK * N,
                           Bs + t * Cfg::B_TILE + (wave * NBI + q) * 256);
        }
    }

    // All of this wave's loads have landed; the barrier makes the other
    // waves' loads visible.  (The compiler makes LDS reads wait for every
    // outstanding direct-to-LDS load anyway, so per-tile waits would not
    // overlap anything inside the workgroup: the second workgroup resident
    // on the CU overlaps its loads with this one's compute instead.)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // Fragment reads of tile t.  A: row ty*4+i, k pair (kk, kk+1) at its
    // swizzled quad; B: k rows kk, kk+1 at columns tx*4 .. tx*4+3.
    const int swz = ty & 7;
    auto load_frag = [&](int t, int kk, T (&a)[TM][2], T (&b)[2][TN]) {
        const T* as = As + t * Cfg::A_TILE;
        const T* bs = Bs + t * Cfg::B_TILE;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int off = (ty * 4 + i) * BK + (((kk >> 2) ^ swz) << 2) + (kk & 3);
            a[i][0] = as[off];
            a[i][1] = as[off + 1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < TN; ++j) b[h][j] = bs[(kk + h) * BN + tx * 4 + j];
    };
    auto store_row = [&](int i, const Vec16<T>& cv, const Vec16<int32_t>& iv) {
        const int64_t gr = row0 + ty * 4 + i;
        const int64_t gc = col0 + tx * 4;
        *reinterpret_cast<Vec16<T>*>(C + gr * N + gc) = cv;
        *reinterpret_cast<Vec16<int32_t>*>(IDX + gr * N + gc) = iv;
    };

    // ---- packed paths: i32 MaxPlus / MinPlus with small magnitudes ---------
    // When every |a| and |b| of the workgroup is below 2^22, the key
    //   MaxPlus: (a + b) * 256 + (255 - k)     MinPlus: (a + b) * 256 + k
    // cannot overflow, orders first by the product and then by k (smaller k
    // wins ties under max, and under min), and so carries the exact value and
    // the first-k argmax through a value-only max3/min3 chain.  A = a * 256
    // and B = b * 256 + (255 - k) (or + k) are rewritten in LDS once; the
    // result is C = key >> 8 and argmax = 255 - (key & 255) (or key & 255).
    // Below 2^15 every key is an integer under 2^24 in magnitude, so the keys
    // are held as f32 (exact adds and max3/min3 on integers), which issues
    // about 1.4x faster than the i32 add + max3 mix on gfx950.  Any larger
    // magnitude in the workgroup falls back to the chunked path.
    if constexpr (std::is_same<T, int32_t>::value && SR != SR_MAXMUL) {
        constexpr int AV = KT * Cfg::A_TILE / 4;  // 16-byte slots of A
        constexpr int BV = KT * Cfg::B_TILE / 4;  // 16-byte slots of B
        static_assert(AV % TG_THREADS == 0 && BV % TG_THREADS == 0, "slot split");
        static_assert(K <= 256, "k must fit in the key's low byte");
        auto below = [](int32_t x, int bits) {
            return uint32_t(x + (1 << (bits - 1))) < (1u << bits);
        };
        int ok15 = 1, ok22 = 1;
#pragma unroll
        for (int q = 0; q < AV / TG_THREADS; ++q) {
            const Vec16<T> v = reinterpret_cast<const Vec16<T>*>(As)[q * TG_THREADS + tid];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ok15 &= below(v.v[e], 16);
                ok22 &= below(v.v[e], 23);
            }
        }
#pragma unroll
        for (int q = 0; q < BV / TG_THREADS; ++q) {
            const Vec16<T> v = reinterpret_cast<const Vec16<T>*>(Bs)[q * TG_THREADS + tid];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ok15 &= below(v.v[e], 16);
                ok22 &= below(v.v[e], 23);
            }
        }
        const bool f32_keys = __syncthreads_and(ok15) != 0;
        const bool i32_keys = !f32_keys && __syncthreads_and(ok22) != 0;
        if (f32_keys || i32_keys) {
            // Rewrite A and B in place (f32 bit patterns or i32 keys).
#pragma unroll
            for (int q = 0; q < AV / TG_THREADS; ++q) {
                Vec16<T>* pv = reinterpret_cast<Vec16<T>*>(As) + q * TG_THREADS + tid;
                Vec16<T> v = *pv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int32_t x = int32_t(uint32_t(v.v[e]) << 8);
                    v.v[e] = f32_keys ? __float_as_int(float(x)) : x;
                }
                *pv = v;
            }
#pragma unroll
            for (int q = 0; q < BV / TG_THREADS; ++q) {
                const int slot = q * TG_THREADS + tid;
                const int el = slot * 4;
                const int k = (el / Cfg::B_TILE) * BK + (el % Cfg::B_TILE) / BN;
                const int low = SR == SR_MINPLUS ? k : 255 - k;
                Vec16<T>* pv = reinterpret_cast<Vec16<T>*>(Bs) + slot;
                Vec16<T> v = *pv;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int32_t x = int32_t((uint32_t(v.v[e]) << 8) + uint32_t(low));
                    v.v[e] = f32_keys ? __float_as_int(float(x)) : x;
                }
                *pv = v;
            }
            __syncthreads();
            // Value-only chain over the keys; U is the key type (f32 or i32).
            auto run = [&](auto zero) {
                using U = decltype(zero);
                const U* au = reinterpret_cast<const U*>(As);
                const U* bu = reinterpret_cast<const U*>(Bs);
                U key[TM][TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) key[i][j] = zero;
#pragma unroll 1
                for (int t = 0; t < KT; ++t) {
#pragma unroll
                    for (int kk = 0; kk < BK; kk += 2) {
                        U a[TM][2], b[2][TN];
#pragma unroll
                        for (int i = 0; i < TM; ++i) {
                            const int off = t * Cfg::A_TILE + (ty * 4 + i) * BK +
                                            (((kk >> 2) ^ swz) << 2) + (kk & 3);
                            a[i][0] = au[off];
                            a[i][1] = au[off + 1];
                        }
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int j = 0; j < TN; ++j)
                                b[h][j] = bu[t * Cfg::B_TILE + (kk + h) * BN + tx * 4 + j];
#pragma unroll
                        for (int i = 0; i < TM; ++i)
#pragma unroll
                            for (int j = 0; j < TN; ++j)
                                key[i][j] = tjoin<SR, U>(
                                    tjoin<SR, U>(key[i][j], tmul<SR, U>(a[i][0], b[0][j])),
                                    tmul<SR, U>(a[i][1], b[1][j]));
                    }
                }
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    Vec16<T> cv;
                    Vec16<int32_t> iv;
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const int32_t ik = int32_t(key[i][j]);  // exact: an integer key
                        cv.v[j] = ik >> 8;
                        iv.v[j] = SR == SR_MINPLUS ? (ik & 255) : 255 - (ik & 255);
                    }
                    store_row(i, cv, iv);
                }
            };
            if (f32_keys)
                run(tzero<SR, float>());
            else
                run(tzero<SR, int32_t>());
            return;
        }
    }

    // ---- chunked path --------------------------------------------------------
    // acc: running value; ch: last chunk that strictly improved it (-1: the
    // tropical zero was never beaten).  Each chunk folds its products into a
    // fresh max3/min3 chain that starts from acc, so the running value needs
    // no separate update: the chunk improved acc iff the chain's result beats
    // acc strictly (the reference's "keep acc iff acc >= p").
    T acc[TM][TN];
    int32_t ch[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            acc[i][j] = tzero<SR, T>();
            ch[i][j] = -1;
        }

#pragma unroll 1
    for (int t = 0; t < KT; ++t) {
#pragma unroll
        for (int s = 0; s < CPT; ++s) {
            T an[TM][TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) an[i][j] = acc[i][j];
#pragma unroll
            for (int kk = s * CL; kk < (s + 1) * CL; kk += 2) {
                T a[TM][2], b[2][TN];
                load_frag(t, kk, a, b);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const T p0 = tmul<SR, T>(a[i][0], b[0][j]);
                        const T p1 = tmul<SR, T>(a[i][1], b[1][j]);
                        an[i][j] = tjoin<SR, T>(tjoin<SR, T>(an[i][j], p0), p1);
                    }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if (tbetter<SR, T>(an[i][j], acc[i][j])) ch[i][j] = t * CPT + s;
                    acc[i][j] = an[i][j];
                }
        }
    }

    // Epilogue: resolve each output inside its recorded chunk, from LDS.  The
    // chunk holds the final value as its own extremum and no earlier product
    // reaches it, so the first k in the chunk whose product equals the final
    // value is the argmax.  For floats the value written is that product's
    // bits (a -0/+0 tie keeps the first occurrence's sign, as the CPU does);
    // for integers it is the final value itself.  Branch-free: outputs whose
    // zero was never beaten resolve chunk 0 and are overwritten.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int r = ty * 4 + i;
        Vec16<T> cv;
        Vec16<int32_t> iv;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int c = ch[i][j];
            const int k0 = (c < 0 ? 0 : c) * CL;
            const int t = k0 / BK;
            const int kq = k0 % BK;
            const T* as = As + t * Cfg::A_TILE + r * BK;
            const T* bs = Bs + t * Cfg::B_TILE + kq * BN + tx * 4 + j;
            const Vec16<T> a0 = *reinterpret_cast<const Vec16<T>*>(as + (((kq >> 2) ^ swz) << 2));
            const Vec16<T> a1 =
                *reinterpret_cast<const Vec16<T>*>(as + ((((kq >> 2) + 1) ^ swz) << 2));
            T p[CL];
#pragma unroll
            for (int kk = 0; kk < CL; ++kk) {
                const T av = kk < 4 ? a0.v[kk] : a1.v[kk - 4];
                p[kk] = tmul<SR, T>(av, bs[kk * BN]);
            }
            // Last match scanning downwards == first match.
            int f = CL - 1;
            T v = p[CL - 1];
#pragma unroll
            for (int kk = CL - 2; kk >= 0; --kk) {
                const bool e = p[kk] == acc[i][j];
                f = e ? kk : f;
                if constexpr (std::is_floating_point<T>::value) v = e ? p[kk] : v;
            }
            if constexpr (!std::is_floating_point<T>::value) v = acc[i][j];
            cv.v[j] = c < 0 ? tzero<SR, T>() : v;
            iv.v[j] = c < 0 ? 0 : k0 + f;
        }
        store_row(i, cv, iv);
    }
}

}  // namespace tg
