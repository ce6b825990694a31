// tg_gemm_kres.hpp -- K-resident tropical GEMM with argmax for short K (gfx950).
//
// Same contract as tg_gemm_dl with ARGMAX=true, for 32-bit types and
// K in {64, 96, 128} (tall-skinny products such as Viterbi steps, where K is
// small and M is large).  The whole K extent of a tile's A rows and B columns
// stays in LDS, so the argmax is resolved from LDS: no B^T staging kernel, no
// global re-reads and no chunk sort.
//
// Persistent: the grid holds every resident workgroup slot (two per CU for
// K = 128).  Workgroup w (renumbered per XCD) owns column tile w % tiles_n
// and walks the row tiles (over all batch items) with a stride of
// gridDim.x / tiles_n.  Its B panel (K x 64) stays in LDS across
// row tiles and is reloaded only when the batch item or the path changes; the
// next row tile's A panel (64 x K) is prefetched into registers while the
// current one computes, then range-checked and written to LDS.
//
// LDS layouts (one slot per 32-k tile t):
//   A tile t  64 rows x 32 k, row-major (128 B rows); the 16-byte quad q of
//             row r sits at quad position q ^ ((r >> 2) & 7), so the four
//             rows a wave reads at one k fall in different banks.
//   B tile t  32 k x 64 cols, row-major (256 B rows).
// Each thread owns 4 consecutive rows (ty*4 + i) and 4 consecutive columns
// (tx*4 + j).
//
// Paths, chosen per row tile from the magnitudes in its A and B panels:
//   f32 keys  i32 MaxPlus/MinPlus, every |x| < 2^15: value-only chain on keys
//             (a+b)*256 + (255-k) (MinPlus: + k), exact integers below 2^24
//             held as f32 (the f32 add + max3 mix issues ~1.4x faster than
//             the i32 one on gfx950);
//   i32 keys  every |x| < 2^22: the same keys as i32;
//   chunked   anything else, and every float problem: chunked argmax with
//             chunks of 8 k (bookkeeping ~2 ops per output per chunk, resolve
//             ~4 ops per product of one chunk), resolved from LDS.
#pragma once

#include "tg_gemm_dl.hpp"

namespace tg {

constexpr int KRES_KT_MAX = 4;  // K <= 128

struct KresCfg {
    static constexpr int BM = 64, BN = 64, BK = 32, TM = 4, TN = 4, CL = 8;
    static constexpr int A_TILE = BM * BK;              // elements per A k-tile
    static constexpr int B_TILE = BK * BN;              // elements per B k-tile
    static constexpr int NBI = BK * BN * 4 / 1024 / 4;  // 1 KB B loads per wave per k-tile
    static constexpr int RPI = 256 / BN;                // B k-rows per 1 KB load
    static constexpr int LPR = BN / 4;                  // lanes per B k-row
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
           K <= int64_t(KresCfg::BK) * KRES_KT_MAX && sA % 4 == 0 && sB % 4 == 0 &&
           sC % 4 == 0 && a16(A) && a16(B) && a16(C) && a16(IDX);
}

// grid = (G, 1, 1) with G a multiple of tiles_n, block = 256.  K = 32 * KT.
template <int SR, typename T, int KT>
__global__ __launch_bounds__(TG_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void tg_gemm_kres(
    const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C,
    int32_t* __restrict__ IDX, int64_t N, int64_t sA, int64_t sB, int64_t sC, int tiles_m,
    int tiles_n, int64_t batch) {
    static_assert(sizeof(T) == 4, "K-resident kernel is for 32-bit types");
    static_assert(KT >= 2 && KT <= KRES_KT_MAX, "K-resident tile count");
    using Cfg = KresCfg;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, TM = Cfg::TM, TN = Cfg::TN;
    constexpr int CL = Cfg::CL, NBI = Cfg::NBI;
    constexpr int K = KT * BK;
    constexpr int CPT = BK / CL;                           // chunks per k-tile
    constexpr int AQ = BM * K / 4 / TG_THREADS;            // 16-byte A slots per thread
    constexpr int BQ = KT * Cfg::B_TILE / 4 / TG_THREADS;  // 16-byte B slots per thread
    constexpr bool KEYS = std::is_same<T, int32_t>::value && SR != SR_MAXMUL;
    constexpr int FORM_ORIG = 0, FORM_F32 = 1, FORM_I32 = 2;
    static_assert(K <= 256, "k must fit in the key's low byte");
    __shared__ __align__(16) T As[KT * Cfg::A_TILE];
    __shared__ __align__(16) T Bs[KT * Cfg::B_TILE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tx = tid & 15;
    const int ty = tid >> 4;
    const int swz = ty & 7;
    // Consecutive workgroup ids go round-robin over the 8 XCDs.  Renumber so
    // each XCD holds a contiguous range: the workgroups that share a row tile
    // (one per column tile) then sit on one XCD and read its A panel through
    // the same L2, so A is fetched from HBM once.
    int lb = int(blockIdx.x);
    if ((gridDim.x & 7) == 0 && (int(gridDim.x >> 3) % tiles_n) == 0)
        lb = int(blockIdx.x & 7) * int(gridDim.x >> 3) + int(blockIdx.x >> 3);
    const int tn = lb % tiles_n;
    const int64_t step = int64_t(gridDim.x) / tiles_n;
    const int64_t total = batch * tiles_m;
    const int64_t col0 = int64_t(tn) * BN;
    int64_t r = int64_t(lb) / tiles_n;
    if (r >= total) return;

    // ---- staging helpers ----------------------------------------------------
    // A panel of row tile rr: 64 x K contiguous elements (row stride K), so
    // slot s of it is elements 4s .. 4s+3; thread tid holds slots q*256+tid.
    Vec16<T> pre[AQ];
    auto load_a = [&](int64_t rr) {
        const int64_t z = rr / tiles_m;
        const int64_t tm = rr - z * tiles_m;
        const T* ap = A + z * sA + tm * BM * K;
#pragma unroll
        for (int q = 0; q < AQ; ++q)
            pre[q] = *reinterpret_cast<const Vec16<T>*>(ap + (q * TG_THREADS + tid) * 4);
    };
    auto store_a = [&](int form) {
#pragma unroll
        for (int q = 0; q < AQ; ++q) {
            const int s = q * TG_THREADS + tid;
            const int row = s / (K / 4);
            const int qg = s % (K / 4);
            Vec16<T> v = pre[q];
            if (form != FORM_ORIG) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int32_t x = int32_t(uint32_t(v.v[e]) << 8);
                    v.v[e] = form == FORM_F32 ? __float_as_int(float(x)) : x;
                }
            }
            *reinterpret_cast<Vec16<T>*>(As + (qg >> 3) * Cfg::A_TILE + row * BK +
                                         (((qg & 7) ^ ((row >> 2) & 7)) << 2)) = v;
        }
    };
    // B panel of batch item z, straight into LDS; ends with a barrier.
    auto load_b = [&](int64_t z) {
        const T* bz = B + z * sB;
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
            for (int q = 0; q < NBI; ++q) {
                const int kr = (wave * NBI + q) * Cfg::RPI + lane / Cfg::LPR;
                lds_load16(bz + int64_t(t * BK + kr) * N + col0 + (lane % Cfg::LPR) * 4,
                           Bs + t * Cfg::B_TILE + (wave * NBI + q) * 256);
            }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    auto below = [](int32_t x, int bits) {
        return uint32_t(x) + (1u << (bits - 1)) < (1u << bits);  // unsigned: no overflow
    };
    // Rewrites B in LDS into keys: b*256 + (255 - k) (MinPlus: + k); ends
    // with a barrier.
    auto rewrite_b = [&](int form) {
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const int slot = q * TG_THREADS + tid;
            const int el = slot * 4;
            const int k = (el / Cfg::B_TILE) * BK + (el % Cfg::B_TILE) / BN;
            const int low = SR == SR_MINPLUS ? k : 255 - k;
            Vec16<T>* pv = reinterpret_cast<Vec16<T>*>(Bs) + slot;
            Vec16<T> v = *pv;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int32_t x = int32_t((uint32_t(v.v[e]) << 8) + uint32_t(low));
                v.v[e] = form == FORM_F32 ? __float_as_int(float(x)) : x;
            }
            *pv = v;
        }
        __syncthreads();
    };

    // Fragment reads of k-tile t as element type U (the keys may be f32):
    // A row ty*4+i, k pair (kk, kk+1) at its swizzled quad; B k rows kk, kk+1
    // at columns tx*4 .. tx*4+3.
    auto frag = [&](auto zero, int t, int kk, auto (&a)[TM][2], auto (&b)[2][TN]) {
        using U = decltype(zero);
        const U* as = reinterpret_cast<const U*>(As) + t * Cfg::A_TILE;
        const U* bs = reinterpret_cast<const U*>(Bs) + t * Cfg::B_TILE;
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

    int64_t zb = -1;        // batch item whose B panel is in LDS
    int bform = FORM_ORIG;  // form of the B panel in LDS
    int bok15 = 0, bok22 = 0;
    load_a(r);
    for (; r < total; r += step) {
        const int64_t z = r / tiles_m;
        const int64_t tm = r - z * tiles_m;
        int form = FORM_ORIG;
        if (z != zb) {
            __syncthreads();  // every wave is done with the previous B panel
            load_b(z);
            bform = FORM_ORIG;
            zb = z;
            if constexpr (KEYS) {
                int ok15 = 1, ok22 = 1;
#pragma unroll
                for (int q = 0; q < BQ; ++q) {
                    const Vec16<T> v = reinterpret_cast<const Vec16<T>*>(Bs)[q * TG_THREADS + tid];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        ok15 &= below(v.v[e], 16);
                        ok22 &= below(v.v[e], 23);
                    }
                }
                bok15 = __syncthreads_and(ok15);
                bok22 = __syncthreads_and(ok22);
            }
        }
        if constexpr (KEYS) {
            int aok15 = 1, aok22 = 1;
#pragma unroll
            for (int q = 0; q < AQ; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    aok15 &= below(pre[q].v[e], 16);
                    aok22 &= below(pre[q].v[e], 23);
                }
            // Also the barrier after the previous tile's use of As.
            if (__syncthreads_and(bok15 && aok15))
                form = FORM_F32;
            else if (__syncthreads_and(bok22 && aok22))
                form = FORM_I32;
        } else {
            __syncthreads();  // every wave is done with the previous A panel
        }
        if (form != bform) {
            if (bform != FORM_ORIG) load_b(z);  // restore the original B panel
            if (form != FORM_ORIG) rewrite_b(form);
            bform = form;
        }
        store_a(form);
        __syncthreads();
        if (r + step < total) load_a(r + step);  // lands while this tile computes

        T* Ct = C + z * sC + tm * BM * N;
        int32_t* It = IDX + z * sC + tm * BM * N;
        // Outputs are written once and not read back by this kernel: non-temporal
        // 16-byte stores keep them from displacing the A/B panels in L2.
        typedef int v4i_t __attribute__((ext_vector_type(4)));
        auto stream16 = [](void* p, const void* v) {
            v4i_t x;
            __builtin_memcpy(&x, v, 16);
            __builtin_nontemporal_store(x, reinterpret_cast<v4i_t*>(p));
        };
        auto store_row = [&](int i, const Vec16<T>& cv, const Vec16<int32_t>& iv) {
            const int64_t off = int64_t(ty * 4 + i) * N + col0 + tx * 4;
            stream16(Ct + off, &cv);
            stream16(It + off, &iv);
        };

        if constexpr (KEYS) {
            if (form != FORM_ORIG) {
                // Value-only chain over the keys; U is the key type (f32 or i32).
                auto run = [&](auto zero) {
                    using U = decltype(zero);
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
                            frag(zero, t, kk, a, b);
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
                if (form == FORM_F32)
                    run(tzero<SR, float>());
                else
                    run(tzero<SR, int32_t>());
                continue;
            }
        }

        // ---- chunked path -------------------------------------------------
        // acc: running value; ch: last chunk that strictly improved it (-1:
        // the tropical zero was never beaten).  Each chunk folds its products
        // into a max3/min3 chain that starts from acc, so the running value
        // needs no separate update: the chunk improved acc iff the chain's
        // result beats acc strictly (the reference's "keep acc iff acc >= p").
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
                    frag(T(0), t, kk, a, b);
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

        // Resolve each output inside its recorded chunk, from LDS.  The chunk
        // holds the final value as its own extremum and no earlier product
        // reaches it, so the first k in the chunk whose product equals the
        // final value is the argmax.  For floats the value written is that
        // product's bits (a -0/+0 tie keeps the first occurrence's sign, as
        // the CPU does); for integers it is the final value itself.
        // Branch-free: outputs whose zero was never beaten resolve chunk 0
        // and are overwritten.
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = ty * 4 + i;
            Vec16<T> cv;
            Vec16<int32_t> iv;
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int c = ch[i][j];
                const int k0 = (c < 0 ? 0 : c) * CL;
                const int t = k0 / BK;
                const int kq = k0 % BK;
                const T* as = As + t * Cfg::A_TILE + row * BK;
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
                if constexpr (std::is_floating_point<T>::value) {
                    if (tisnan(acc[i][j])) {
                        // The chain met a NaN product: the reference's serial
                        // rule over the whole (LDS-resident) k range.
                        T x = tzero<SR, T>();
                        int32_t ix = 0;
                        for (int k = 0; k < KT * BK; ++k) {
                            const int tt = k / BK, q = k % BK;
                            const T ak = As[tt * Cfg::A_TILE + row * BK + (((q >> 2) ^ swz) << 2) + (q & 3)];
                            const T bk = Bs[tt * Cfg::B_TILE + q * BN + tx * 4 + j];
                            const T pk = tmul<SR, T>(ak, bk);
                            if (ttake<SR, T>(pk, x)) {
                                x = pk;
                                ix = k;
                            }
                        }
                        cv.v[j] = x;
                        iv.v[j] = ix;
                    }
                }
            }
            store_row(i, cv, iv);
        }
    }
}

}  // namespace tg
