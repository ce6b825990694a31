// tg_gemm_dl64.hpp -- direct-to-LDS tropical GEMM for f64 (gfx950).
//
// Same contract as tg_gemm_tiles (tg_kernels.hpp), with or without argmax,
// for large f64 problems.  The byte layout is that of tg_gemm_dl's 64 x 128 tiles
// (tg_gemm_dl.hpp) with 8-byte elements: a 16-byte quad holds two k.
//   A tile  64 rows x 16 k, 128-byte rows; quad q of row r stored at quad
//           position q ^ ((r >> 2) & 7) (the four rows a wave reads at one k
//           pair fall in different banks).
//   B tile  16 k x 128 columns, row-major (1 KB per k-row).
// Two LDS buffers of 24 KB: the loads of k-tile t+1 overlap the compute of
// k-tile t.  16 x 16 threads; thread (tx, ty) owns rows ty*4 + i (i < 4) and
// columns (j >> 2) * 64 + tx*4 + (j & 3) (j < 8).  Per pair of k it reads 4
// ds_read_b128 of A and 8 of B for 64 products: 3 bytes of LDS per product.
// Per product one v_add_f64 and one v_max_f64 (v_min_f64): f64 has no
// three-input max on gfx950.  With argmax about 210 VGPRs: two waves per
// SIMD, which the issue probe measures at 92% of the f64 add+max ceiling;
// value-only (no chunk-start copies, no records) three.
//
// Argmax: one chunk per k-tile (CL = 16).  The running value alternates
// between acc and alt from k-tile to k-tile, and a k-tile is recorded where
// its chain strictly beats the value before it (as tg_gemm_dl); the epilogue
// resolves the first k inside the recorded chunk from the A-row and B^T-row
// windows.
//
// NaN: v_max_f64 / v_min_f64 return the other operand of a NaN, so a chain
// never shows a NaN product.  A prepass (tg_class_prepass; with argmax the
// B^T transpose does the columns) records per row of A and per column of B
// whether it holds a NaN, +inf,
// -inf or a zero; an output whose row and column could meet in a NaN product
// (a NaN operand, +inf with -inf for MaxPlus / MinPlus, a zero with an
// infinity for MaxMul) is recomputed after the stores with the reference's
// serial rule (cpu_select over the whole k range).
//
// Host-checked requirements (dl64_fits): K % 32 == 0 (k-tiles in pairs),
// N % 4 == 0, 16-byte aligned A, B, C, IDX (if any) and batch strides
// multiples of 4;
// chunk indices below 2^16.  Partial tiles in M and N: loads clamp into the
// matrix, stores skip rows past M and 4-column groups past N.
#pragma once

#include "tg_gemm_dl.hpp"

namespace tg {

struct Dl64Cfg {
    static constexpr int TM = 4, TN = 8, BM = 64, BN = 128, BK = 16, CL = 16;
    static constexpr int NAI = BM * BK * 8 / 4096;  // 1 KB A loads per wave (2)
    static constexpr int NBI = BK * BN * 8 / 4096;  // 1 KB B loads per wave (4)
    static constexpr int A_BYTES = BM * BK * 8;     // 8 KB
    static constexpr int B_BYTES = BK * BN * 8;     // 16 KB
    static constexpr int TILE_BYTES = 2 * (A_BYTES + B_BYTES);
    static constexpr int OUTS = BM * BN;
    static constexpr int NB = 256;  // chunk buckets of the epilogue sort
    static constexpr int HIST_OFF = 0;
    static constexpr int CHS_OFF = HIST_OFF + NB * 4;
    static constexpr int LIST_OFF = CHS_OFF + OUTS * 2;
    static constexpr int MISC_OFF = LIST_OFF + OUTS * 2;
    static constexpr int LDS_BYTES = (MISC_OFF + 64 > TILE_BYTES) ? MISC_OFF + 64 : TILE_BYTES;
};

// True when a row of class ca and a column of class cb can make a NaN
// product at some k (conservative: the k need not coincide).
template <int SR>
__device__ __forceinline__ bool nan_danger(uint32_t ca, uint32_t cb) {
    if ((ca | cb) & TG_CLS_NAN) return true;
    if constexpr (SR == SR_MAXMUL) {
        const uint32_t inf = TG_CLS_PINF | TG_CLS_NINF;
        return ((ca & TG_CLS_ZERO) && (cb & inf)) || ((ca & inf) && (cb & TG_CLS_ZERO));
    } else {
        return ((ca & TG_CLS_PINF) && (cb & TG_CLS_NINF)) || ((ca & TG_CLS_NINF) && (cb & TG_CLS_PINF));
    }
}

// Operand classes, one launch: blocks [0, row_blocks) take the rows of A
// (batch x M x K, batch stride sA) into clsA[z*M + i], one wave per row at a
// time; the other blocks take the columns of B (batch x K x N, batch stride
// sB) into clsB[z*N + j] (skipped when clsB is null: the f64 argmax path
// gets them from the B^T transpose, which reads B anyway), in segments of 64
// columns x 256 k, 4 k-lanes per column.  Both arrays zeroed beforehand.
// Grid-stride over rows and segments; block = 256.
__global__ __launch_bounds__(256) void tg_class_prepass(const double* __restrict__ A, int64_t M,
                                                        int64_t K, int64_t sA,
                                                        const double* __restrict__ B, int64_t N,
                                                        int64_t sB, int64_t batch,
                                                        uint32_t* __restrict__ clsA,
                                                        uint32_t* __restrict__ clsB,
                                                        int row_blocks) {
    const int lane = threadIdx.x & 63;
    if (int(blockIdx.x) < row_blocks) {
        const int64_t waves = int64_t(row_blocks) * 4;
        for (int64_t w = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6); w < batch * M; w += waves) {
            const int64_t z = w / M, i = w - z * M;
            const double* row = A + z * sA + i * K;
            uint32_t c = 0;
            for (int64_t k = lane; k < K; k += 64) c |= tclass(row[k]);
            uint32_t all = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if (__ballot((c >> b) & 1u)) all |= 1u << b;
            if (lane == 0) clsA[w] = all;
        }
        return;
    }
    if (clsB == nullptr) return;
    const int64_t nbx = (N + 63) / 64, nby = (K + 255) / 256;
    const int64_t per_z = nbx * nby, segs = per_z * batch;
    const int64_t cblocks = int64_t(gridDim.x) - row_blocks;
    for (int64_t sg = int64_t(blockIdx.x) - row_blocks; sg < segs; sg += cblocks) {
        const int64_t z = sg / per_z, r = sg - z * per_z;
        const int64_t by = r / nbx, bx = r - by * nbx;
        const int64_t j = bx * 64 + lane;
        const int64_t k0 = by * 256 + (threadIdx.x >> 6);
        if (j < N) {
            const double* col = B + z * sB + j;
            uint32_t c = 0;
            for (int64_t k = k0; k < K && k < k0 + 256; k += 4) c |= tclass(col[k * N]);
            if (c) atomicOr(clsB + z * N + j, c);
        }
    }
}

// Chunk records of four f64 outputs (record4 with 64-bit compares): ch[q] = c
// where cand[q] strictly beats prev[q].
template <int SR>
__device__ __forceinline__ void record4_f64(int32_t& c0, int32_t& c1, int32_t& c2, int32_t& c3,
                                            double n0, double n1, double n2, double n3, double p0,
                                            double p1, double p2, double p3, int32_t cv) {
    uint64_t m0, m1, m2, m3;
#define TG_RECORD4_F64_ASM(CMP)                                                                \
    asm volatile(CMP " %0, %8, %12\n\t" CMP " %1, %9, %13\n\t" CMP " %2, %10, %14\n\t" CMP    \
                     " %3, %11, %15\n\t"                                                       \
                     "v_cndmask_b32_e64 %4, %4, %16, %0\n\t"                                    \
                     "v_cndmask_b32_e64 %5, %5, %16, %1\n\t"                                    \
                     "v_cndmask_b32_e64 %6, %6, %16, %2\n\t"                                    \
                     "v_cndmask_b32_e64 %7, %7, %16, %3"                                        \
                 : "=&s"(m0), "=&s"(m1), "=&s"(m2), "=&s"(m3), "+v"(c0), "+v"(c1), "+v"(c2), \
                   "+v"(c3)                                                                     \
                 : "v"(n0), "v"(n1), "v"(n2), "v"(n3), "v"(p0), "v"(p1), "v"(p2), "v"(p3),      \
                   "v"(cv))
    if constexpr (SR == SR_MINPLUS) TG_RECORD4_F64_ASM("v_cmp_lt_f64_e64");
    else TG_RECORD4_F64_ASM("v_cmp_gt_f64_e64");
#undef TG_RECORD4_F64_ASM
}

// True when tg_gemm_dl64 can run the problem (see the header comment).
inline bool dl64_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, int64_t sC,
                      const void* A, const void* B, const void* C, const void* IDX) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return M > 0 && N > 0 && K > 0 && K % 32 == 0 && N % 4 == 0 && K / Dl64Cfg::CL < 0xFFFF &&
           K < (int64_t(1) << 25) && N < (int64_t(1) << 27) && sA % 4 == 0 && sB % 4 == 0 &&
           sC % 4 == 0 && a16(A) && a16(B) && a16(C) && (IDX == nullptr || a16(IDX));
}

// grid = (tiles_m * tiles_n, 1, batch), block = 256, LDS = Dl64Cfg::LDS_BYTES
// (argmax) or Dl64Cfg::TILE_BYTES (value-only: BT and IDX unused).
// clsA / clsB: row / column classes (batch x M, batch x N).
template <int SR, bool ARGMAX>
__global__ __launch_bounds__(TG_THREADS) __attribute__((amdgpu_waves_per_eu(ARGMAX ? 2 : 3))) void tg_gemm_dl64(
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ BT,
    double* __restrict__ C, int32_t* __restrict__ IDX, const uint32_t* __restrict__ clsA,
    const uint32_t* __restrict__ clsB, int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB,
    int64_t sC, int tiles_m, int tiles_n) {
    using T = double;
    using Cfg = Dl64Cfg;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, TM = Cfg::TM, TN = Cfg::TN;
    constexpr int NAI = Cfg::NAI, NBI = Cfg::NBI, CL = Cfg::CL;
    static_assert(CL == BK, "one argmax chunk per k-tile");
    extern __shared__ __align__(16) unsigned char dl64_lds[];
    T* const As0 = reinterpret_cast<T*>(dl64_lds);
    T* const Bs0 = reinterpret_cast<T*>(dl64_lds + 2 * Cfg::A_BYTES);

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
    if constexpr (ARGMAX) {
        IDX += z * sC;
        BT += z * (N * K);
    }
    clsA += z * M;
    clsB += z * N;
    auto trow = [&](int i) { return ty * 4 + i; };
    auto tcol = [&](int j) { return (j >> 2) * 64 + tx * 4 + (j & 3); };

    // Direct loads of k-tile t.  A: 8 rows (128 B each) per 1 KB
    // instruction, wave w issuing instructions NAI*w .. NAI*w + NAI-1; B: one
    // k-row (1 KB) per instruction, wave w issuing NBI*w .. NBI*w + NBI-1.
    // Addresses: a wave-uniform base plus a 32-bit per-lane byte offset.
    // Rows past M read row M-1 and column pairs past N the last pair: in
    // bounds, feeding only outputs that are never stored.
    uint32_t offA[NAI];
#pragma unroll
    for (int q = 0; q < NAI; ++q) {
        const int64_t rb = row0 + (wave * NAI + q) * 8;
        const int64_t gr = rb + (lane >> 3);
        const int r = int(gr - row0);
        const int qsrc = (lane & 7) ^ ((r >> 2) & 7);
        offA[q] = uint32_t(((gr < M ? gr : M - 1) - (rb < M ? rb : M - 1)) * K * 8 + qsrc * 16);
    }
    auto a_base = [&](int q) {
        const int64_t rb = row0 + (wave * NAI + q) * 8;
        return reinterpret_cast<const unsigned char*>(A + (rb < M ? rb : M - 1) * K);
    };
    const int64_t gcB = col0 + lane * 2;
    const uint32_t offB = uint32_t((gcB < N ? gcB : N - 2) * 8);
    auto b_base = [&](int q, int64_t k0) {
        return reinterpret_cast<const unsigned char*>(B + (k0 + wave * NBI + q) * N);
    };
    auto issue_loads = [&](int64_t t, int buf) {
        T* adst = As0 + buf * (BM * BK);
        T* bdst = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int q = 0; q < NAI; ++q)
            lds_load16(a_base(q) + t * BK * 8 + offA[q], adst + (wave * NAI + q) * 128);
#pragma unroll
        for (int q = 0; q < NBI; ++q)
            lds_load16(b_base(q, t * BK) + offB, bdst + (wave * NBI + q) * 128);
    };

    T acc[TM][TN], alt[TM][TN];
    int32_t ch[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            acc[i][j] = tzero<SR, T>();
            alt[i][j] = tzero<SR, T>();
            ch[i][j] = -1;
        }

    // A: row trow(i), k pair (kk, kk + 1) = quad kk >> 1 at its swizzled
    // position (the swizzle is ty & 7 for all of a thread's rows).
    int swz_t = ty & 7;
    auto load_frag = [&](int buf, int kk, T (&a)[TM][2], T (&b)[2][TN]) {
        const T* as = As0 + buf * (BM * BK);
        const T* bs = Bs0 + buf * (BK * BN);
        const int q = (((kk >> 1) ^ swz_t) << 1);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const Vec16<T> v = *reinterpret_cast<const Vec16<T>*>(as + trow(i) * BK + q);
            a[i][0] = v.v[0];
            a[i][1] = v.v[1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < TN; j += 2) {
                const Vec16<T> v = *reinterpret_cast<const Vec16<T>*>(bs + (kk + h) * BN + tcol(j));
                b[h][j] = v.v[0];
                b[h][j + 1] = v.v[1];
            }
    };
    // Value-only chains: v_max_f64 / v_min_f64 as written.  Through the
    // compiler's maxnum the loop-carried value gets a canonicalizing max per
    // k-tile, and the loop spilled; every operand here is an add result or a
    // max of them, so it is canonical already.
    auto join_f64 = [](T x, T y) {
        T r;
        if constexpr (SR == SR_MINPLUS)
            asm("v_min_f64 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
        else
            asm("v_max_f64 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
        return r;
    };
    // The k-tile t (one chunk) in buffer buf: a chain from `from` into `to`,
    // recorded where `to` strictly beats `from` (value-only: in place, no
    // record).
    auto chunk = [&](int64_t t, int buf, const T (&from)[TM][TN], T (&to)[TM][TN]) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            T a[TM][2], b[2][TN];
            load_frag(buf, kk, a, b);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const T p0 = tmul<SR, T>(a[i][0], b[0][j]);
                    const T p1 = tmul<SR, T>(a[i][1], b[1][j]);
                    const T st = kk == 0 ? from[i][j] : to[i][j];
                    if constexpr (ARGMAX)
                        to[i][j] = tjoin<SR, T>(tjoin<SR, T>(st, p0), p1);
                    else
                        to[i][j] = join_f64(join_f64(st, p0), p1);
                }
        }
        if constexpr (ARGMAX) {
            int32_t cv;
            asm volatile("v_mov_b32 %0, %1" : "=v"(cv) : "s"(int32_t(t)));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; j += 4)
                    record4_f64<SR>(ch[i][j], ch[i][j + 1], ch[i][j + 2], ch[i][j + 3], to[i][j],
                                    to[i][j + 1], to[i][j + 2], to[i][j + 3], from[i][j],
                                    from[i][j + 1], from[i][j + 2], from[i][j + 3], cv);
        }
    };

    // k-tiles in pairs: the even one runs acc -> alt, the odd one alt -> acc.
    const int64_t nkt = K / BK;
    issue_loads(0, 0);
    for (int64_t t = 0; t < nkt; t += 2) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t tt = t + h;
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tt + 1 < nkt) issue_loads(tt + 1, h ^ 1);
            asm volatile("" : "+v"(swz_t));
            if constexpr (!ARGMAX)
                chunk(tt, h, acc, acc);
            else if (h == 0)
                chunk(tt, 0, acc, alt);
            else
                chunk(tt, 1, alt, acc);
        }
    }

    // ---- epilogue ------------------------------------------------------------
    auto store_row = [&](int i, const T (&v)[TN], const int32_t (&ix)[TN]) {
        const int64_t gr = row0 + trow(i);
        if (gr >= M) return;
#pragma unroll
        for (int g = 0; g < TN / 4; ++g) {
            const int64_t gc = col0 + g * 64 + tx * 4;
            if (gc >= N) continue;  // N is a multiple of 4: whole groups only
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                Vec16<T> cv;
                cv.v[0] = v[g * 4 + 2 * h];
                cv.v[1] = v[g * 4 + 2 * h + 1];
                *reinterpret_cast<Vec16<T>*>(C + gr * N + gc + 2 * h) = cv;
            }
            Vec16<int32_t> iv;
#pragma unroll
            for (int e = 0; e < 4; ++e) iv.v[e] = ix[g * 4 + e];
            *reinterpret_cast<Vec16<int32_t>*>(IDX + gr * N + gc) = iv;
        }
    };
    // Outputs whose row and column could meet in a NaN product: recomputed
    // after the stores with the serial rule (one runtime loop over a mask).
    uint64_t redo = 0;
    if constexpr (!ARGMAX) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t gr = row0 + trow(i);
            const uint32_t ra = clsA[gr < M ? gr : M - 1];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int64_t gc = col0 + tcol(j);
                if (nan_danger<SR>(ra, clsB[gc < N ? gc : N - 1])) redo |= uint64_t(1) << (i * TN + j);
            }
            if (gr >= M) continue;
#pragma unroll
            for (int g = 0; g < TN / 4; ++g) {
                const int64_t gc = col0 + g * 64 + tx * 4;
                if (gc >= N) continue;  // N is a multiple of 4: whole groups only
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    Vec16<T> cv;
                    cv.v[0] = acc[i][g * 4 + 2 * h];
                    cv.v[1] = acc[i][g * 4 + 2 * h + 1];
                    *reinterpret_cast<Vec16<T>*>(C + gr * N + gc + 2 * h) = cv;
                }
            }
        }
#pragma unroll 1
        while (redo) {
            const int o = __builtin_ctzll(redo);
            redo &= redo - 1;
            const int64_t gr = row0 + trow(o / TN), gc = col0 + tcol(o % TN);
            if (gr >= M || gc >= N) continue;
            T v;
            int32_t ix;
            cpu_select<SR, T>(A + gr * K, 1, B + gc, N, K, v, ix);
            C[gr * N + gc] = v;
        }
        return;
    }
    {
        uint32_t ra[TM], cb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int64_t gr = row0 + trow(i);
            ra[i] = clsA[gr < M ? gr : M - 1];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t gc = col0 + tcol(j);
            cb[j] = clsB[gc < N ? gc : N - 1];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                if (nan_danger<SR>(ra[i], cb[j])) {
                    redo |= uint64_t(1) << (i * TN + j);
                    ch[i][j] = -2;
                }
    }

    // Exact first k inside each output's recorded chunk (as tg_gemm_dl): a
    // counting sort by chunk, then one output per thread at a time.
    constexpr uint16_t NONE = 0xFFFF;
    uint32_t* hist = reinterpret_cast<uint32_t*>(dl64_lds + Cfg::HIST_OFF);
    uint16_t* chs = reinterpret_cast<uint16_t*>(dl64_lds + Cfg::CHS_OFF);
    uint16_t* list = reinterpret_cast<uint16_t*>(dl64_lds + Cfg::LIST_OFF);
    int* misc = reinterpret_cast<int*>(dl64_lds + Cfg::MISC_OFF);
    static_assert(Cfg::MISC_OFF + 64 <= Cfg::LDS_BYTES, "epilogue arrays fit the LDS block");
    const int64_t nchunks = nkt;
    int shift = 0;
    while (((nchunks - 1) >> shift) >= Cfg::NB) ++shift;
    const int nb = int(((nchunks - 1) >> shift) + 1);
    __syncthreads();  // every wave is done with the tile buffers
    if (tid < Cfg::NB) hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int lid = trow(i) * BN + tcol(j);
            chs[lid] = ch[i][j] < 0 ? NONE : uint16_t(ch[i][j]);
            if (ch[i][j] >= 0) atomicAdd(&hist[ch[i][j] >> shift], 1u);
        }
    __syncthreads();
    const int cnt = tid < nb ? int(hist[tid]) : 0;
    int total = 0;
    const int start = block_exclusive_scan(cnt, misc, total);
    if (tid < nb) hist[tid] = uint32_t(start);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
            if (ch[i][j] >= 0)
                list[atomicAdd(&hist[ch[i][j] >> shift], 1u)] = uint16_t(trow(i) * BN + tcol(j));
    __syncthreads();

    constexpr int NW = CL / 2;  // 16-byte vectors per window
    for (int e = tid; e < total; e += TG_THREADS) {
        const int lid = int(list[e]);
        const int64_t c = int64_t(chs[lid]);
        const int64_t gr = row0 + lid / BN, gc = col0 + (lid & (BN - 1));
        const T* ap = A + (gr < M ? gr : M - 1) * K + c * CL;
        const T* bp = BT + (gc < N ? gc : N - 1) * K + c * CL;
        T p[CL];
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const Vec16<T> av = *reinterpret_cast<const Vec16<T>*>(ap + 2 * w);
            const Vec16<T> bv = *reinterpret_cast<const Vec16<T>*>(bp + 2 * w);
            p[2 * w] = tmul<SR, T>(av.v[0], bv.v[0]);
            p[2 * w + 1] = tmul<SR, T>(av.v[1], bv.v[1]);
        }
        T mx = tjoin<SR, T>(p[0], p[1]);
#pragma unroll
        for (int kk = 2; kk < CL; kk += 2) mx = tjoin<SR, T>(tjoin<SR, T>(mx, p[kk]), p[kk + 1]);
        uint32_t bits = 0;
#pragma unroll
        for (int kk = 0; kk < CL; ++kk) bits |= (p[kk] == mx) ? (1u << kk) : 0u;
        const int f = bits ? int(__builtin_ctz(bits)) : 0;
        int r = f;
        if (mx == T(0) && __builtin_signbit(p[f])) r |= 32;
        chs[lid] = uint16_t(r);
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < TM; ++i) {
        T v[TN];
        int32_t ix[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if (ch[i][j] == -2) {  // redone below
                v[j] = acc[i][j];
                ix[j] = 0;
            } else if (ch[i][j] < 0) {  // the tropical zero was never beaten
                v[j] = tzero<SR, T>();
                ix[j] = 0;
            } else {
                const int r = chs[trow(i) * BN + tcol(j)];
                ix[j] = ch[i][j] * CL + (r & 31);
                v[j] = acc[i][j];
                if (v[j] == T(0)) v[j] = (r & 32) ? -T(0) : T(0);
            }
        }
        store_row(i, v, ix);
    }
#pragma unroll 1
    while (redo) {
        const int o = __builtin_ctzll(redo);
        redo &= redo - 1;
        const int64_t gr = row0 + trow(o / TN), gc = col0 + tcol(o % TN);
        if (gr >= M || gc >= N) continue;
        T v;
        int32_t ix;
        cpu_select<SR, T>(A + gr * K, 1, BT + gc * K, 1, K, v, ix);
        C[gr * N + gc] = v;
        IDX[gr * N + gc] = ix;
    }
}

}  // namespace tg
