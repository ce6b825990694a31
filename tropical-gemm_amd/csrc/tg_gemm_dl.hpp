// tg_gemm_dl.hpp -- direct-to-LDS tropical GEMM for 32-bit types (gfx950).
//
// Same contract as tg_gemm_tiles (tg_kernels.hpp).  Tiles go from HBM
// straight into LDS with global_load_lds_dwordx4 (no staging registers, no
// LDS-store VALU work), which frees the registers the argmax bookkeeping
// needs.
//
// Layouts (per LDS buffer; two buffers, loads of k-tile t+1 overlap the
// compute of k-tile t):
//   A tile  BM rows x 32 k, row-major (128 B rows).  The 16-byte quad q of
//           row r is stored at quad position q ^ ((r >> 2) & 7), so the four
//           rows a wave reads at one k fall in different banks.
//   B tile  32 k x BN cols, row-major.
// 16 x 16 threads; thread (tx, ty) owns rows (i >> 2) * 64 + ty*4 + (i & 3)
// for i < TM and columns (j >> 2) * 64 + tx*4 + (j & 3) for j < TN.  Per
// pair of k it reads TM ds_read_b64 of A and TN/2 ds_read_b128 of B for
// 2 TM TN products: 4 (TM + TN) / (TM TN) bytes of LDS per product (1.5 for
// 4 x 8, 1 for 8 x 8).
#pragma once

#include <utility>

#include "tg_kernels.hpp"

namespace tg {

// Tile configurations, TM x TN outputs per thread:
//   4 x 8: 64 x 128 tiles; argmax held to 3 waves/SIMD (<= 168 VGPRs),
//          value-only at 2.
//   4 x 4: 64 x 64 tiles, 4 waves/SIMD (<= 128 VGPRs): small problems, split
//          K, partial k-tiles.
//   8 x 8: 128 x 128 tiles, value-only, 2 waves/SIMD: 1 byte of LDS per
//          product (MaxPlus f32 4096^3 value-only: 1.86 ms against 1.99 for
//          4 x 8 and 2.04-2.14 for 4 x 4 on MI355X).
template <int TM_, int TN_>
struct DlCfg {
    static constexpr int TM = TM_, TN = TN_;
    static constexpr int BM = 16 * TM_, BN = 16 * TN_, BK = TG_CHUNK;
    static constexpr int WAVES_ARGMAX = TN_ == 8 ? 3 : 4;
    static constexpr int WAVES_VALUE = TN_ == 8 ? 2 : 4;
    static constexpr int NAI = BM * BK / 1024;      // 1 KB A-tile loads per wave
    static constexpr int NBI = BK * BN / 1024;      // 1 KB B-tile loads per wave
    static constexpr int RPI = 256 / BN;            // B k-rows per 1 KB load
    static constexpr int LPR = BN / 4;              // lanes per B k-row
    static constexpr int A_BYTES = BM * BK * 4;   // one A buffer
    static constexpr int B_BYTES = BK * BN * 4;   // one B buffer
    static constexpr int TILE_BYTES = 2 * (A_BYTES + B_BYTES);
    // Argmax epilogue, reusing the tile buffers: bucket counts (then bucket
    // cursors), per-output chunk (u16; the resolve overwrites it with its
    // result), chunk-sorted output list (u16), a few words of scan scratch.
    static constexpr int OUTS = BM * BN;            // outputs per tile
    static constexpr int NB = 256;                  // chunk buckets
    static constexpr int HIST_OFF = 0;
    static constexpr int CHS_OFF = HIST_OFF + NB * 4;
    static constexpr int LIST_OFF = CHS_OFF + OUTS * 2;
    static constexpr int MISC_OFF = LIST_OFF + OUTS * 2;
    static constexpr int LDS_BYTES = (MISC_OFF + 64 > TILE_BYTES) ? MISC_OFF + 64 : TILE_BYTES;
};

// Exclusive prefix sum over 256 threads (tid 0..255: the workgroup, or one
// 256-thread half of it, each half with its own scratch); returns the
// exclusive prefix of x and sets total.  scratch: 5 ints of LDS.  Every
// thread of the workgroup calls it (it holds two barriers).
__device__ __forceinline__ int block_exclusive_scan(int x, int* scratch, int& total,
                                                    int tid = int(threadIdx.x)) {
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
    }
    if (lane == 63) scratch[wave] = inc;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int t = scratch[w];
        if (w < wave) before += t;
        total += t;
    }
    __syncthreads();
    return before + inc - x;
}

// One 16-byte direct load per lane: global src -> LDS at dst + lane * 16
// (dst must be the same for the whole wave).  A non-template wrapper: the
// builtin with template-dependent pointer types is not accepted by the host
// compilation pass.
__device__ __forceinline__ void lds_load16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// Byte address of a pointer into LDS, as ds_* instructions take it (the low
// 32 bits of the generic address are the offset in the LDS aperture).
__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// A 16-byte LDS read issued without a wait: the caller waits for it with
// lds_wait before it uses r.  The compiler does not track these reads, so
// nothing else may read r in between.
template <int OFF, typename V>
__device__ __forceinline__ void lds_read16_nowait(V& r, uint32_t addr) {
    static_assert(sizeof(V) == 16 && OFF >= 0 && OFF < 65536, "ds_read_b128, 16-bit offset");
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
}

template <int OFF, typename V>
__device__ __forceinline__ void lds_read8_nowait(V& r, uint32_t addr) {
    static_assert(sizeof(V) == 8 && OFF >= 0 && OFF < 65536, "ds_read_b64, 16-bit offset");
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
}

// Waits for every outstanding LDS read of this wave; the values of the
// registers read into (tied here) are only used after it.
// lds_wait<N>: waits until at most N of this wave's LDS reads are
// outstanding (LDS reads complete in order, so the older ones are done; a
// scalar load in flight only makes the wait stricter).
template <int N = 0, typename V>
__device__ __forceinline__ void lds_wait(V& r0, V& r1, V& r2, V& r3) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3) : "i"(N) : "memory");
}
template <int N = 0, typename V, typename W>
__device__ __forceinline__ void lds_wait(V& r0, V& r1, V& r2, V& r3, W& r4, W& r5, W& r6, W& r7) {
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3), "+v"(r4), "+v"(r5), "+v"(r6), "+v"(r7)
                 : "i"(N)
                 : "memory");
}

// An empty asm statement that uses x: the values are computed before it (and
// so before every later asm statement, which keeps its order).
template <typename T>
__device__ __forceinline__ void pin8(const T& x0, const T& x1, const T& x2, const T& x3, const T& x4,
                                     const T& x5, const T& x6, const T& x7) {
    asm volatile("" ::"v"(x0), "v"(x1), "v"(x2), "v"(x3), "v"(x4), "v"(x5), "v"(x6), "v"(x7));
}

// f(std::integral_constant<int, I>{}) for I = 0 .. N-1, in order: the body
// sees I as a constant expression (immediate LDS offsets, unrolled chunks).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// True when tg_gemm_dl<.., CL> can run the problem: K and N multiples of
// 4 and 16-byte aligned operands, outputs and batch strides (tiles load and
// store 16 bytes per lane), and chunk indices that fit the epilogue's 16-bit
// slots.  M, N and K need not fill the tiles: the loads of a partial tile
// clamp their rows, columns and k into the matrix (in-bounds duplicates),
// the k past K of the last k-tile are then overwritten in LDS with operands
// whose product is the tropical zero, and the stores skip rows past M and
// 4-column groups past N.
template <int CL>
inline bool dl_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, int64_t sC,
                    const void* A, const void* B, const void* C, const void* IDX) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return M > 0 && N > 0 && K > 0 && N % 4 == 0 && K % 4 == 0 && (K + CL - 1) / CL < 0xFFFF &&
           K < (int64_t(1) << 26) && N < (int64_t(1) << 28) && sA % 4 == 0 && sB % 4 == 0 && sC % 4 == 0 && a16(A) && a16(B) && a16(C) &&
           (IDX == nullptr || a16(IDX));
}

// True when the pipelined value-only 8 x 8 main loop (PIPE) can run the
// problem: its per-lane load offsets (up to 127 rows of A, 32 k rows of B)
// fit 32 bits.
inline bool pipe_fits(int64_t N, int64_t K) {
    return K < (int64_t(1) << 23) && N < (int64_t(1) << 25);
}

// True when every tile of the problem is full.
template <int TM, int TN>
inline bool dl_full_tiles(int64_t M, int64_t N, int64_t K) {
    return M % DlCfg<TM, TN>::BM == 0 && N % DlCfg<TM, TN>::BN == 0 && K % DlCfg<TM, TN>::BK == 0;
}

// Split K for problems with too few 64 x 64 tiles (partial ones included) to
// fill the chip: the largest power of two S with at most 512 workgroups in
// total (two per CU: longer slices, each resolving its own argmax, beat four
// per CU; MaxPlus f32 1024^3 + argmax on MI355X: S = 2 69 us against 77 us
// for S = 4 and 95 us for S = 8), slices of at least 256 k and slice
// lengths that are multiples of 64.
// N a multiple of 4, as the kernel needs (the merge then reads whole 16-byte
// groups of the dense M x N partials).
inline int dl_splits(int64_t M, int64_t N, int64_t K, int64_t batch) {
    if (M <= 0 || N <= 0 || N % 4 != 0 || K % 64 != 0 || batch <= 0) return 1;
    const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64) * batch;
    int s = 1;
    while (tiles * s * 2 <= 512 && K % (int64_t(64) * s * 2) == 0 && K / (s * 2) >= 256) s *= 2;
    return s;
}

// Combines the S split-K partials of tg_gemm_dl.  Slices are visited in k
// order and a later slice replaces the running result only if strictly
// better, so equal values keep the earlier slice's index and bits: the
// reference's first-k rule across slices.  A slice whose chain met a NaN
// product left NaN in its partial; such an output is recomputed here with
// the reference's serial rule over the whole k range (A row, and B^T row
// with argmax or B column without).  Partials are dense, slice stride
// sY = batch * M * N; outputs use the batch stride sC.  16-byte vectors
// (N, so M * N, is a multiple of 4 here).
template <int SR, typename T, bool ARGMAX>
__global__ __launch_bounds__(256) void tg_merge_splits(const T* __restrict__ PV,
                                                       const int32_t* __restrict__ PI,
                                                       T* __restrict__ C, int32_t* __restrict__ IDX,
                                                       int S, int64_t MN, int64_t batch, int64_t sY,
                                                       int64_t sC, const T* __restrict__ A,
                                                       const T* __restrict__ B,
                                                       const T* __restrict__ BT, int64_t N,
                                                       int64_t K, int64_t sA, int64_t sB) {
    const int64_t nvec = batch * MN / 4;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t v = int64_t(blockIdx.x) * 256 + threadIdx.x; v < nvec; v += stride) {
        const int64_t e = v * 4;
        const int64_t z = e / MN;
        const int64_t r = e - z * MN;
        Vec16<T> best = *reinterpret_cast<const Vec16<T>*>(PV + e);
        Vec16<int32_t> bi{};
        if constexpr (ARGMAX) bi = *reinterpret_cast<const Vec16<int32_t>*>(PI + e);
        bool nan[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) nan[q] = tisnan(best.v[q]);
        for (int y = 1; y < S; ++y) {
            const Vec16<T> pv = *reinterpret_cast<const Vec16<T>*>(PV + y * sY + e);
            Vec16<int32_t> pi{};
            if constexpr (ARGMAX) pi = *reinterpret_cast<const Vec16<int32_t>*>(PI + y * sY + e);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                nan[q] = nan[q] || tisnan(pv.v[q]);
                if (tbetter<SR, T>(pv.v[q], best.v[q])) {
                    best.v[q] = pv.v[q];
                    if constexpr (ARGMAX) bi.v[q] = pi.v[q];
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (nan[q]) {
                const int64_t i = (r + q) / N, j = (r + q) - ((r + q) / N) * N;
                const T* a = A + z * sA + i * K;
                int32_t ix;
                if (ARGMAX && BT != nullptr)
                    cpu_select<SR, T>(a, 1, BT + z * (N * K) + j * K, 1, K, best.v[q], ix);
                else  // value-only, or argmax resolved from B (no B^T staged)
                    cpu_select<SR, T>(a, 1, B + z * sB + j, N, K, best.v[q], ix);
                if constexpr (ARGMAX) bi.v[q] = ix;
            }
        }
        *reinterpret_cast<Vec16<T>*>(C + z * sC + r) = best;
        if constexpr (ARGMAX) *reinterpret_cast<Vec16<int32_t>*>(IDX + z * sC + r) = bi;
    }
}

// Chunk records of four outputs: ch[q] = c where cand[q] strictly beats
// prev[q] (the reference's keep-rule "acc >= p" for max, "acc <= p" for min,
// types/max_plus.rs:66-73, min_plus.rs:66-73).  The four compares write four
// SGPR masks before the four selects read them: compiled per output, each
// compare went to VCC and its select waited two wait states on it (the
// gfx950 VALU-mask hazard), which cost more than the compare itself.
template <int SR, typename T>
__device__ __forceinline__ void record4(int32_t& c0, int32_t& c1, int32_t& c2, int32_t& c3,
                                        T n0, T n1, T n2, T n3, T p0, T p1, T p2, T p3,
                                        int32_t cv) {
    uint64_t m0, m1, m2, m3;
#define TG_RECORD4_ASM(CMP)                                                                    \
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
    if constexpr (std::is_same<T, float>::value) {
        if constexpr (SR == SR_MINPLUS) TG_RECORD4_ASM("v_cmp_lt_f32_e64");
        else TG_RECORD4_ASM("v_cmp_gt_f32_e64");
    } else {
        static_assert(std::is_same<T, int32_t>::value, "32-bit types only");
        if constexpr (SR == SR_MINPLUS) TG_RECORD4_ASM("v_cmp_lt_i32_e64");
        else TG_RECORD4_ASM("v_cmp_gt_i32_e64");
    }
#undef TG_RECORD4_ASM
}

// Waves per SIMD come from the tile configuration (DlCfg): other resident
// waves hide the LDS latency of the main loop.
// TAILK: K is not a multiple of BK (the last k-tile is partial); a separate
// instantiation, so full-K problems run the plain pipeline.
// BDIRECT (argmax): the resolve reads each window's B values down B's column
// (CL loads with stride N) instead of from a staged B^T row, and BT is
// unused; for split-K problems whose B stays in L2 (the host decides), where
// it saves the transpose launch (1024^3: 68 against 71 us per call).
// PIPE (value-only 8 x 8 outputs, whole k-tiles; its value is the waves per
// SIMD the kernel is built for, 2): the fragments of the next k pair are
// read from LDS while the current pair is folded (reads issued ahead and
// waited for explicitly), so a wave does not stall on LDS between pairs
// (MaxPlus f32 4096^3 on MI355X: 1.847 against 1.891 ms).
template <int SR, typename T, bool ARGMAX, int TM_, int TN_, int CL, bool TAILK = false,
          bool BDIRECT = false, int PIPE = 0, int HALVES = 1>
__global__ __launch_bounds__(TG_THREADS * HALVES) __attribute__((amdgpu_waves_per_eu(
    PIPE != 0 ? PIPE : ARGMAX ? DlCfg<TM_, TN_>::WAVES_ARGMAX : DlCfg<TM_, TN_>::WAVES_VALUE))) void tg_gemm_dl(
    const T* __restrict__ A, const T* __restrict__ B, const T* __restrict__ BT,
    T* __restrict__ C, int32_t* __restrict__ IDX, int64_t M, int64_t N, int64_t K, int64_t sA,
    int64_t sB, int64_t sC, int tiles_m, int tiles_n, int64_t KS, int64_t sY) {
    static_assert(sizeof(T) == 4, "direct-to-LDS kernel is for 32-bit types");
    using Cfg = DlCfg<TM_, TN_>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, TM = Cfg::TM, TN = Cfg::TN;
    constexpr int NAI = Cfg::NAI, NBI = Cfg::NBI;
    static_assert(CL == 8 || CL == 16 || CL == 32, "argmax chunk of 8, 16 or 32 k");
    static_assert(!ARGMAX || (BK / CL) % 2 == 0, "argmax: an even number of chunks per k-tile");
    static_assert(!ARGMAX || TM == 4, "argmax tiles have 4 rows per thread");
    static_assert(HALVES == 1 || ((HALVES == 2 || HALVES == 4) && ARGMAX && !TAILK && PIPE == 0),
                  "K slices per workgroup (2 or 4): argmax, whole k-tiles");
    extern __shared__ __align__(16) unsigned char dl_lds_all[];
    // HALVES > 1: the workgroup is HALVES 256-thread parts ("halves" for
    // short), each running the kernel on its own K slice with its own LDS
    // block; they meet only at the barriers (every barrier is reached by
    // all of them) and in the merge before the resolve.
    const int half = HALVES > 1 ? int(__builtin_amdgcn_readfirstlane(threadIdx.x >> 8)) : 0;
    unsigned char* const dl_lds = dl_lds_all + (HALVES > 1 ? half * Cfg::LDS_BYTES : 0);
    T* const As0 = reinterpret_cast<T*>(dl_lds);
    T* const Bs0 = reinterpret_cast<T*>(dl_lds + 2 * Cfg::A_BYTES);

    const int tid = int(threadIdx.x) & (TG_THREADS - 1);
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
    // Split K: slice y covers k in [y*KS, (y+1)*KS) and writes its (value,
    // argmax) partial at C/IDX + y*sY (tg_merge_splits combines them).  An
    // unsplit launch has gridDim.y == 1, KS == K and sY == 0.  With
    // halves, half h is slice h (KS == K / HALVES) and the halves merge in
    // LDS into C/IDX (sY unused).
    const int64_t y = HALVES > 1 ? half : int64_t(blockIdx.y);
    C += z * sC + (HALVES > 1 ? 0 : y * sY);
    if (ARGMAX) {
        IDX += z * sC + (HALVES > 1 ? 0 : y * sY);
        if constexpr (!BDIRECT) BT += z * (N * K);
    }
    // Tile row / column of this thread's output (i, j).
    auto trow = [&](int i) { return (i >> 2) * 64 + ty * 4 + (i & 3); };
    auto tcol = [&](int j) { return (j >> 2) * 64 + tx * 4 + (j & 3); };

    // Direct loads of k-tile t.  A: 8 rows per 1 KB instruction, wave w
    // issues instructions NAI*w .. NAI*w + NAI-1; B: RPI k-rows per
    // instruction, wave w issues NBI*w .. NBI*w + NBI-1.  Each address is a
    // wave-uniform base (SGPRs) plus a 32-bit per-lane byte offset (a VGPR
    // each for A, one for B), so the loads hold few registers through the
    // main loop.  In a partial tile, rows past M read row M-1 and 4-column
    // groups past N read the last group: in-bounds duplicates that only feed
    // outputs that are never stored.  A base row: the first row of the
    // instruction, clamped; the lane's row offset stays in [0, 7], so the
    // offsets fit 32 bits for K < 2^26 (dl_fits).
    uint32_t offA[NAI];
#pragma unroll
    for (int q = 0; q < NAI; ++q) {
        const int64_t rb = row0 + (wave * NAI + q) * 8;
        const int64_t gr = rb + (lane >> 3);
        const int r = int(gr - row0);
        const int qsrc = (lane & 7) ^ ((r >> 2) & 7);
        offA[q] = uint32_t(((gr < M ? gr : M - 1) - (rb < M ? rb : M - 1)) * K * 4 + qsrc * 16);
    }
    auto a_base = [&](int q) {
        const int64_t rb = row0 + (wave * NAI + q) * 8;
        return reinterpret_cast<const unsigned char*>(A + (rb < M ? rb : M - 1) * K);
    };
    const int64_t gcB = col0 + (lane % Cfg::LPR) * 4;
    const uint32_t offB =
        uint32_t((lane / Cfg::LPR) * N * 4 + (gcB < N ? gcB : N - 4) * 4);
    auto b_base = [&](int q, int64_t k0) {
        return reinterpret_cast<const unsigned char*>(B + (k0 + (wave * NBI + q) * Cfg::RPI) * N);
    };
    auto issue_loads = [&](int64_t t, int buf) {
        T* adst = As0 + buf * (BM * BK);
        T* bdst = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int q = 0; q < NAI; ++q)
            lds_load16(a_base(q) + t * BK * 4 + offA[q], adst + (wave * NAI + q) * 256);
#pragma unroll
        for (int q = 0; q < NBI; ++q)
            lds_load16(b_base(q, t * BK) + offB, bdst + (wave * NBI + q) * 256);
    };
    // The last k-tile when K is not a multiple of BK: A quads past K read the
    // row's last quad and B rows past K read row K-1 (in bounds; overwritten
    // in LDS by patch_tail before use).
    auto issue_tail_loads = [&](int64_t t, int buf) {
        T* adst = As0 + buf * (BM * BK);
        T* bdst = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int q = 0; q < NAI; ++q) {
            const int r = (wave * NAI + q) * 8 + (lane >> 3);
            const int qsrc = (lane & 7) ^ ((r >> 2) & 7);
            const int64_t kq = t * BK + qsrc * 4;
            const int64_t kc = kq < K - 4 ? kq : K - 4;
            lds_load16(a_base(q) + kc * 4 + (offA[q] - qsrc * 16), adst + (wave * NAI + q) * 256);
        }
#pragma unroll
        for (int q = 0; q < NBI; ++q) {
            const int kr = (wave * NBI + q) * Cfg::RPI + lane / Cfg::LPR;
            const int64_t kk = t * BK + kr;
            const int64_t kc = kk < K - 1 ? kk : K - 1;
            lds_load16(reinterpret_cast<const unsigned char*>(B + kc * N) +
                           (offB - uint32_t((lane / Cfg::LPR) * N * 4)),
                       bdst + (wave * NBI + q) * 256);
        }
    };
    // k in [kv, BK) of the tile in buffer buf: A gets the tropical zero and B
    // gets 0, so those products are the tropical zero (never an improvement;
    // no infinities meet, and integers do not wrap).
    auto patch_tail = [&](int buf, int kv) {
        T* as = As0 + buf * (BM * BK);
        T* bs = Bs0 + buf * (BK * BN);
        const int na = BM * (BK - kv);
        for (int e = tid; e < na; e += TG_THREADS) {
            const int r = e / (BK - kv), k = kv + e % (BK - kv);
            as[r * BK + (((k >> 2) ^ ((r >> 2) & 7)) << 2) + (k & 3)] = tzero<SR, T>();
        }
        const int nb = (BK - kv) * BN;
        for (int e = tid; e < nb; e += TG_THREADS) bs[kv * BN + e] = T(0);
    };

    // acc / alt: the running value, alternating between the two arrays from
    // chunk to chunk (argmax: the chain of a chunk runs from one into the
    // other, so the value held before the chunk is still there for the
    // record, and no copies are needed).  ch: last chunk that strictly
    // improved the output (-1: the tropical zero was never beaten).
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

    // Fragment reads.  A: row trow(i), k pair (kk, kk+1) at its swizzled quad.
    // The swizzle of a thread's rows is ty & 7 for every i ((trow(i) >> 2) & 7);
    // swz_t is re-declared opaque once per k-tile, so the eight swizzled quad
    // offsets are recomputed per tile (a few VALU ops) instead of being held
    // in registers through the loop.
    int swz_t = ty & 7;
    auto load_frag = [&](int buf, int kk, T (&a)[TM][2], T (&b)[2][TN]) {
        const T* as = As0 + buf * (BM * BK);
        const T* bs = Bs0 + buf * (BK * BN);
        const int q = (((kk >> 2) ^ swz_t) << 2) + (kk & 3);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int off = trow(i) * BK + q;
            a[i][0] = as[off];
            a[i][1] = as[off + 1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < TN; ++j) b[h][j] = bs[(kk + h) * BN + tcol(j)];
    };
    // One argmax chunk: the products of k in [s*CL, (s+1)*CL) of the tile in
    // buffer buf fold into a max3/min3 chain that starts from `from` and ends
    // in `to`; the chunk is recorded where `to` strictly beats `from`.
    // Value-only: the chain runs in place (from and to are the same array).
    auto chunk = [&](int64_t t, int buf, int s, const T (&from)[TM][TN], T (&to)[TM][TN]) {
#pragma unroll
        for (int kk = s * CL; kk < (s + 1) * CL; kk += 2) {
            T a[TM][2], b[2][TN];
            load_frag(buf, kk, a, b);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const T p0 = tmul<SR, T>(a[i][0], b[0][j]);
                    const T p1 = tmul<SR, T>(a[i][1], b[1][j]);
                    const T st = kk == s * CL ? from[i][j] : to[i][j];
                    to[i][j] = tjoin<SR, T>(tjoin<SR, T>(st, p0), p1);
                }
        }
        if constexpr (ARGMAX) {
            int32_t cv;
            asm volatile("v_mov_b32 %0, %1" : "=v"(cv) : "s"(int32_t(t * (BK / CL) + s)));
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; j += 4)
                    record4<SR, T>(ch[i][j], ch[i][j + 1], ch[i][j + 2], ch[i][j + 3], to[i][j],
                                   to[i][j + 1], to[i][j + 2], to[i][j + 3], from[i][j],
                                   from[i][j + 1], from[i][j + 2], from[i][j + 3], cv);
        }
    };

    // k-tiles [t0, t1) of this slice; t (and so every chunk index) is global.
    // Split slices are whole k-tiles; an unsplit K may end in a partial one
    // holding kv valid k.
    const int64_t t0 = y * (KS / BK);
    const int64_t t1 = t0 + (KS + BK - 1) / BK;
    const int kv = TAILK ? int(KS - (t1 - 1 - t0) * BK) : BK;
    if constexpr (PIPE != 0) {
        static_assert(TM == 8 && TN == 8 && !TAILK && !ARGMAX,
                      "pipelined main loop: value-only 8 x 8 outputs, whole k-tiles");
        typedef T V4 __attribute__((ext_vector_type(4)));
        typedef T V2 __attribute__((ext_vector_type(2)));
        // Per-thread LDS byte addresses in buffer 0.  A: row trow(i) at
        // a_thr + 128 (i & 3) + 64 * 128 (i >> 2); its k quad kq at the
        // swizzled position (kq ^ swz) << 4 (row starts are 128-byte
        // aligned, so the XOR touches only the quad bits).  B: k row at
        // +512 k, this thread's column quads at +16 tx and +256 + 16 tx.
        const uint32_t lds0 = lds_byte_addr(dl_lds);
        const uint32_t a_thr = lds0 + uint32_t(ty) * (4 * BK * 4);
        const uint32_t b_thr = lds0 + 2 * Cfg::A_BYTES + uint32_t(tx) * 16;
        const uint32_t sw16 = uint32_t(ty & 7) << 4;
        // Global -> LDS loads of k-tile t: wave-uniform base pointers advanced
        // by a constant per tile, plus per-lane 32-bit byte offsets fixed for
        // the whole loop (the row and column clamps of partial tiles
        // included; they fit 32 bits by pipe_fits).
        uint32_t poffA[NAI], poffB[NBI];
#pragma unroll
        for (int q = 0; q < NAI; ++q) {
            const int r = (wave * NAI + q) * 8 + (lane >> 3);
            const int64_t gr = row0 + r < M ? row0 + r : M - 1;
            const int qsrc = (lane & 7) ^ ((r >> 2) & 7);
            poffA[q] = uint32_t((gr - row0) * K * 4 + qsrc * 16);
        }
#pragma unroll
        for (int q = 0; q < NBI; ++q) {
            const int64_t kr = (wave * NBI + q) * Cfg::RPI + lane / Cfg::LPR;
            const int64_t gc = col0 + (lane % Cfg::LPR) * 4;
            poffB[q] = uint32_t(kr * N * 4 + (gc < N ? gc : N - 4) * 4);
        }
        const unsigned char* const a_row0 = reinterpret_cast<const unsigned char*>(A + row0 * K);
        const unsigned char* const b_col0 = reinterpret_cast<const unsigned char*>(B);
        auto pipe_loads = [&](int64_t t, int buf) __attribute__((always_inline)) {
            T* adst = As0 + buf * (BM * BK);
            T* bdst = Bs0 + buf * (BK * BN);
            const unsigned char* ap = a_row0 + t * (BK * 4);
            const unsigned char* bp = b_col0 + t * (BK * N * 4);
#pragma unroll
            for (int q = 0; q < NAI; ++q) lds_load16(ap + poffA[q], adst + (wave * NAI + q) * 256);
#pragma unroll
            for (int q = 0; q < NBI; ++q) lds_load16(bp + poffB[q], bdst + (wave * NBI + q) * 256);
        };
        // Fragments.  B: two register sets by pair parity, bf[s][h*2 + g] = k
        // row h of the pair, column quad g.  A: one set, af[i] = the pair's
        // two k of row i, refilled half a pair behind the folds.  Pair P runs
        // as: fold rows 0-3; read rows 0-3 and B of P+1; wait for rows 4-7 of
        // P; fold them; read rows 4-7 of P+1; wait for rows 0-3 and B of P+1
        // (8, then 12 reads in flight; the waits count them).
        V4 bf[2][4];
        V2 af[TM];
        auto read_b = [&](auto pc, uint32_t bbuf, int set) __attribute__((always_inline)) {
            constexpr int P = decltype(pc)::value;
            lds_read16_nowait<P * 1024>(bf[set][0], bbuf);
            lds_read16_nowait<P * 1024 + 256>(bf[set][1], bbuf);
            lds_read16_nowait<P * 1024 + 512>(bf[set][2], bbuf);
            lds_read16_nowait<P * 1024 + 768>(bf[set][3], bbuf);
        };
        auto read_a_half = [&](auto pc, auto hc, uint32_t abuf) __attribute__((always_inline)) {
            constexpr int P = decltype(pc)::value, H = decltype(hc)::value;
            const uint32_t addr = (sw16 ^ uint32_t((P / 2) << 4)) + abuf;
            static_for<4>([&](auto ic) __attribute__((always_inline)) {
                constexpr int I = decltype(ic)::value;
                lds_read8_nowait<H * 64 * BK * 4 + I * 128 + (P & 1) * 8>(af[H * 4 + I], addr);
            });
        };
        // Folds rows [I0, I1) of the pair into acc, row by row, each row's
        // results pinned so the fold happens here (the instruction selector
        // would otherwise place it after later asm statements: nothing else
        // ties it) and a row's temporaries die before the next row starts.
        auto fold_rows = [&](auto i0c, auto i1c, int sb) __attribute__((always_inline)) {
            constexpr int I0 = decltype(i0c)::value, I1 = decltype(i1c)::value;
#pragma unroll
            for (int i = I0; i < I1; ++i) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const T p0 = tmul<SR, T>(af[i][0], bf[sb][j >> 2][j & 3]);
                    const T p1 = tmul<SR, T>(af[i][1], bf[sb][2 + (j >> 2)][j & 3]);
                    acc[i][j] = tjoin<SR, T>(tjoin<SR, T>(acc[i][j], p0), p1);
                }
                pin8(acc[i][0], acc[i][1], acc[i][2], acc[i][3], acc[i][4], acc[i][5], acc[i][6],
                     acc[i][7]);
            }
        };
        constexpr int PAIRS = BK / 2;
        // Prologue: tile t0 in LDS (and t0 + 1 on its way), the first pair's
        // fragments read.
        pipe_loads(t0, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // Tile count as a 32-bit scalar (the loop's control stays in SGPRs).
        const int ntiles = __builtin_amdgcn_readfirstlane(int(t1 - t0));
        if (ntiles > 1) pipe_loads(t0 + 1, 1);
        read_a_half(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, a_thr);
        read_b(std::integral_constant<int, 0>{}, b_thr, 0);
        read_a_half(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, a_thr);
        lds_wait(af[0], af[1], af[2], af[3], af[4], af[5], af[6], af[7]);
        lds_wait(bf[0][0], bf[0][1], bf[0][2], bf[0][3]);
        for (int it = 0; it < ntiles; ++it) {
            const int64_t t = t0 + it;
            const int buf = it & 1;
            const uint32_t abuf = a_thr + uint32_t(buf) * Cfg::A_BYTES;
            const uint32_t bbuf = b_thr + uint32_t(buf) * Cfg::B_BYTES;
            const uint32_t abuf_n = a_thr + uint32_t(buf ^ 1) * Cfg::A_BYTES;
            const uint32_t bbuf_n = b_thr + uint32_t(buf ^ 1) * Cfg::B_BYTES;
            const bool more = it + 1 < ntiles;
            static_for<PAIRS>([&](auto pc) __attribute__((always_inline)) {
                constexpr int P = decltype(pc)::value;
                constexpr int NP = P + 1;
                constexpr int SB = P & 1;
                fold_rows(std::integral_constant<int, 0>{}, std::integral_constant<int, 4>{}, SB);
                __builtin_amdgcn_sched_barrier(0);
                bool issued = true;
                if constexpr (NP < PAIRS) {
                    read_a_half(std::integral_constant<int, NP>{}, std::integral_constant<int, 0>{}, abuf);
                    read_b(std::integral_constant<int, NP>{}, bbuf, NP & 1);
                } else if (more) {
                    // Tile t+1 complete in LDS, and every wave done reading
                    // tile t (their reads were waited for): load t+2 into
                    // this buffer, read t+1's first pair.
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                    if (it + 2 < ntiles) pipe_loads(t + 2, buf);
                    read_a_half(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, abuf_n);
                    read_b(std::integral_constant<int, 0>{}, bbuf_n, 0);
                } else {
                    issued = false;
                }
                // Rows 4-7 of pair P: their reads are older than the eight
                // just issued.
                if (issued)
                    lds_wait<8>(af[4], af[5], af[6], af[7]);
                else
                    lds_wait<0>(af[4], af[5], af[6], af[7]);
                __builtin_amdgcn_sched_barrier(0);
                fold_rows(std::integral_constant<int, 4>{}, std::integral_constant<int, 8>{}, SB);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (NP < PAIRS) {
                    read_a_half(std::integral_constant<int, NP>{}, std::integral_constant<int, 1>{}, abuf);
                    lds_wait<4>(af[0], af[1], af[2], af[3], bf[NP & 1][0], bf[NP & 1][1],
                                bf[NP & 1][2], bf[NP & 1][3]);
                } else if (more) {
                    read_a_half(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{}, abuf_n);
                    lds_wait<4>(af[0], af[1], af[2], af[3], bf[0][0], bf[0][1], bf[0][2], bf[0][3]);
                }
            });
        }
    } else {
    if (TAILK && t1 - 1 == t0)
        issue_tail_loads(t0, 0);
    else
        issue_loads(t0, 0);
    for (int64_t t = t0; t < t1; ++t) {
        const int buf = int((t - t0) & 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t + 1 < t1) {
            if (TAILK && t + 2 == t1)
                issue_tail_loads(t + 1, buf ^ 1);
            else
                issue_loads(t + 1, buf ^ 1);
        }
        if (TAILK && t + 1 == t1) {
            patch_tail(buf, kv);
            __syncthreads();
        }
        asm volatile("" : "+v"(swz_t));
        if constexpr (ARGMAX) {
#pragma unroll
            for (int s = 0; s < BK / CL; s += 2) {
                chunk(t, buf, s, acc, alt);
                chunk(t, buf, s + 1, alt, acc);
            }
        } else {
#pragma unroll
            for (int s = 0; s < BK / CL; ++s) chunk(t, buf, s, acc, acc);
        }
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
            Vec16<T> cv;
#pragma unroll
            for (int e = 0; e < 4; ++e) cv.v[e] = v[g * 4 + e];
            *reinterpret_cast<Vec16<T>*>(C + gr * N + gc) = cv;
            if constexpr (ARGMAX) {
                Vec16<int32_t> iv;
#pragma unroll
                for (int e = 0; e < 4; ++e) iv.v[e] = ix[g * 4 + e];
                *reinterpret_cast<Vec16<int32_t>*>(IDX + gr * N + gc) = iv;
            }
        }
    };
    // An output whose chain met a NaN product ends NaN (f32 chains propagate
    // NaN).  Unsplit, it is recomputed after the stores with the reference's
    // serial rule over the whole k range (cpu_select: B read down its column,
    // or B^T along its row) and stored again; a split-K slice leaves NaN in
    // its partial and tg_merge_splits recomputes the output.  Rare: only NaN
    // inputs, or infinities meeting (-inf + inf, 0 * inf), make NaN products.
    // The outputs to redo go through a bit mask and one runtime loop, so the
    // serial code is not unrolled per output and does not press on the main
    // loop's registers.
    const bool split = HALVES > 1 || gridDim.y > 1;
    static_assert(TM * TN <= 64, "one mask bit per output");
    uint64_t redo = 0;
    auto redo_outputs = [&](bool argmax_out) {
#pragma unroll 1
        while (redo) {
            const int o = __builtin_ctzll(redo);
            redo &= redo - 1;
            const int64_t gr = row0 + trow(o / TN), gc = col0 + tcol(o % TN);
            if (split || gr >= M || gc >= N) continue;
            T v;
            int32_t ix;
            if (argmax_out && !BDIRECT)
                cpu_select<SR, T>(A + gr * K, 1, BT + gc * K, 1, K, v, ix);
            else
                cpu_select<SR, T>(A + gr * K, 1, B + gc, N, K, v, ix);
            C[gr * N + gc] = v;
            if (argmax_out) IDX[gr * N + gc] = ix;
        }
    };
    if constexpr (!ARGMAX) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            int32_t none[TN] = {};
#pragma unroll
            for (int j = 0; j < TN; ++j)
                if (tisnan(acc[i][j])) redo |= uint64_t(1) << (i * TN + j);
            store_row(i, acc[i], none);
        }
        if constexpr (std::is_floating_point<T>::value) redo_outputs(false);
    } else {
        // Exact first k inside each output's recorded chunk c.  The window of
        // chunk c holds the final value as its own maximum (no product of an
        // earlier chunk reaches it), so the window alone gives the target and
        // the first k attaining it.  Outputs are resolved in chunk order (LDS
        // counting sort), so workgroups running side by side read the same
        // A-row / B^T-row segments at about the same time and mostly hit in
        // cache.  The resolve returns the offset inside the chunk and, for a
        // zero maximum, the sign of the first zero product (the CPU keeps the
        // first occurrence's bits); it writes them over the output's chunk
        // slot, and the thread that owns the output combines them with its
        // own record.
        constexpr uint16_t NONE = 0xFFFF;
        // Halves: the first half's block holds the one sorted list of the
        // merged outputs; each half keeps its own scan scratch.
        constexpr bool H2 = HALVES > 1;
        unsigned char* const ep_lds = H2 ? dl_lds_all : dl_lds;
        uint32_t* hist = reinterpret_cast<uint32_t*>(ep_lds + Cfg::HIST_OFF);
        uint16_t* chs = reinterpret_cast<uint16_t*>(ep_lds + Cfg::CHS_OFF);
        uint16_t* list = reinterpret_cast<uint16_t*>(ep_lds + Cfg::LIST_OFF);
        int* misc = reinterpret_cast<int*>(dl_lds + Cfg::MISC_OFF);
        int* const shared_total = reinterpret_cast<int*>(ep_lds + Cfg::MISC_OFF) + 8;
        static_assert(Cfg::MISC_OFF + 64 <= Cfg::LDS_BYTES, "epilogue arrays fit the LDS block");
        static_assert(Cfg::NB <= TG_THREADS, "one bucket per thread in the scan");
        // Buckets: chunk >> shift, at most NB of them.
        const int64_t nchunks = (K + CL - 1) / CL;
        int shift = 0;
        while (((nchunks - 1) >> shift) >= Cfg::NB) ++shift;
        const int nb = int(((nchunks - 1) >> shift) + 1);

        // NaN chains: no record is meaningful; -2 keeps them out of the sort.
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                if (tisnan(acc[i][j])) ch[i][j] = -2;
        __syncthreads();  // every wave is done with the tile buffers
        if constexpr (H2) {
            // Merge the halves before the resolve, in k order as
            // tg_merge_splits does: a later slice replaces the running result
            // only if strictly better.  Only the winning slice's chunk is
            // then resolved, by all the workgroup's threads.  An output that
            // met a NaN product in any slice (chunk -2) is recomputed at the
            // end.  Halves 1.. hand over through their own LDS blocks.
            static_assert(2 * TM * TN * TG_THREADS * 4 <= Cfg::LDS_BYTES, "merge buffer fits");
            if (half > 0) {
                T* const mv = reinterpret_cast<T*>(dl_lds);
                int32_t* const mi = reinterpret_cast<int32_t*>(mv + TM * TN * TG_THREADS);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        mv[(i * TN + j) * TG_THREADS + tid] = acc[i][j];
                        mi[(i * TN + j) * TG_THREADS + tid] = ch[i][j];
                    }
            }
            __syncthreads();
            if (half == 0) {
#pragma unroll 1
                for (int h = 1; h < HALVES; ++h) {
                    const T* const mv = reinterpret_cast<const T*>(dl_lds_all + h * Cfg::LDS_BYTES);
                    const int32_t* const mi =
                        reinterpret_cast<const int32_t*>(mv + TM * TN * TG_THREADS);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const T v1 = mv[(i * TN + j) * TG_THREADS + tid];
                            const int32_t c1 = mi[(i * TN + j) * TG_THREADS + tid];
                            if (ch[i][j] == -2 || c1 == -2) {
                                ch[i][j] = -2;
                            } else if (tbetter<SR, T>(v1, acc[i][j])) {
                                acc[i][j] = v1;
                                ch[i][j] = c1;
                            }
                        }
                }
            }
            __syncthreads();  // the merge buffers are free again
        }
        const bool sorter = !H2 || half == 0;
        if (sorter && tid < Cfg::NB) hist[tid] = 0;
        __syncthreads();
        if (sorter) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int lid = trow(i) * BN + tcol(j);
                    chs[lid] = ch[i][j] < 0 ? NONE : uint16_t(ch[i][j]);
                    if (ch[i][j] >= 0) atomicAdd(&hist[ch[i][j] >> shift], 1u);
                }
        }
        __syncthreads();
        // Exclusive scan of the bucket counts; the starts become cursors.
        const int cnt = sorter && tid < nb ? int(hist[tid]) : 0;
        int total = 0;
        const int start = block_exclusive_scan(cnt, misc, total, tid);
        if (sorter && tid < nb) hist[tid] = uint32_t(start);
        if constexpr (H2) {
            if (half == 0 && tid == 0) *shared_total = total;
        }
        __syncthreads();
        if constexpr (H2) total = *shared_total;
        if (sorter) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    if (ch[i][j] >= 0)
                        list[atomicAdd(&hist[ch[i][j] >> shift], 1u)] = uint16_t(trow(i) * BN + tcol(j));
        }
        __syncthreads();

        // Resolve, chunk-sorted, one output per thread at a time, the next
        // output's windows loading while the current one is scanned (loads
        // of a list entry this thread owns, unconditional, so each wait
        // covers only the older pair).
        constexpr int NW = CL / 4;
        struct Window {
            Vec16<T> a[NW], b[NW];
        };
        auto window_ptrs = [&](int e, const T*& ap, const T*& bp) {
            const int lid = int(list[e]);
            const int64_t c = int64_t(chs[lid]);
            // Clamped like the tile loads (outputs past M or N are not
            // stored; their windows just stay in bounds).
            const int64_t gr = row0 + lid / BN, gc = col0 + (lid & (BN - 1));
            ap = A + (gr < M ? gr : M - 1) * K + c * CL;
            // BDIRECT: bp is the window's first element in B's column (stride N).
            bp = BDIRECT ? B + c * CL * N + (gc < N ? gc : N - 1)
                         : BT + (gc < N ? gc : N - 1) * K + c * CL;
            return c;
        };
        auto load_window = [&](int e, Window& wv) {
            const T* ap;
            const T* bp;
            const int64_t c = window_ptrs(e, ap, bp);
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                // Quads of a window past K read the row's last quad:
                // duplicates that come after their originals, so the first
                // match is a k < K.
                const int64_t off = (!TAILK || c * CL + w * 4 <= K - 4) ? w * 4 : K - 4 - c * CL;
                wv.a[w] = *reinterpret_cast<const Vec16<T>*>(ap + off);
                if constexpr (BDIRECT) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) wv.b[w].v[q] = bp[(off + q) * N];
                } else {
                    wv.b[w] = *reinterpret_cast<const Vec16<T>*>(bp + off);
                }
            }
        };
        // One list entry's resolve: first k of its window attaining the
        // window's optimum, and for a zero optimum the sign of that
        // product; written over the entry's chunk slot.
        auto resolve_entry = [&](int e, const Window& cur) __attribute__((always_inline)) {
            T p[CL];
#pragma unroll
            for (int w = 0; w < NW; ++w)
#pragma unroll
                for (int q = 0; q < 4; ++q) p[w * 4 + q] = tmul<SR, T>(cur.a[w].v[q], cur.b[w].v[q]);
            T mx = tjoin<SR, T>(p[0], p[1]);
#pragma unroll
            for (int kk = 2; kk < CL; kk += 2) mx = tjoin<SR, T>(tjoin<SR, T>(mx, p[kk]), p[kk + 1]);
            uint32_t bits = 0;
#pragma unroll
            for (int kk = 0; kk < CL; ++kk) bits |= (p[kk] == mx) ? (1u << kk) : 0u;
            const int f = bits ? int(__builtin_ctz(bits)) : 0;
            int r = f;
            if constexpr (std::is_floating_point<T>::value) {
                if (mx == T(0)) {
                    const T* ap;
                    const T* bp;
                    window_ptrs(e, ap, bp);
                    const T bf = BDIRECT ? bp[int64_t(f) * N] : bp[f];
                    if (__builtin_signbit(tmul<SR, T>(ap[f], bf))) r |= 32;
                }
            }
            chs[int(list[e])] = uint16_t(r);
        };
        // Halves: all the workgroup's threads resolve the merged list.
        constexpr int RT = TG_THREADS * HALVES;
        const int rt = H2 ? int(threadIdx.x) : tid;
        if (rt < total) {
            Window cur;
            load_window(rt, cur);
            for (int e = rt; e < total; e += RT) {
                // The next entry this thread owns, or this one again (its
                // chunk slot is overwritten only below): never another
                // thread's entry, whose slot may already hold an offset.
                const int en = e + RT < total ? e + RT : e;
                Window nxt;
                load_window(en, nxt);
                resolve_entry(e, cur);
                cur = nxt;
            }
        }
        __syncthreads();

        // Each output's (value, first k) of this slice; acc and ch take them.
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                int32_t ix;
                if (ch[i][j] == -2) {  // the chain met a NaN product: redone below
                    ix = 0;
                    redo |= uint64_t(1) << (i * TN + j);
                } else if (ch[i][j] < 0) {  // the tropical zero was never beaten
                    acc[i][j] = tzero<SR, T>();
                    ix = 0;
                } else {
                    const int r = chs[trow(i) * BN + tcol(j)];
                    ix = ch[i][j] * CL + (r & 31);
                    if constexpr (std::is_floating_point<T>::value) {
                        if (acc[i][j] == T(0)) acc[i][j] = (r & 32) ? -T(0) : T(0);
                    }
                }
                ch[i][j] = ix;
            }
        if constexpr (H2) {
            // The first half holds the merged outputs; a NaN in either slice
            // is recomputed with the reference's serial rule over the whole
            // k range (the unsplit kernel's redo, which a split slice skips).
            if (half == 0) {
#pragma unroll
                for (int i = 0; i < TM; ++i) store_row(i, acc[i], ch[i]);
#pragma unroll 1
                while (redo) {
                    const int o = __builtin_ctzll(redo);
                    redo &= redo - 1;
                    const int64_t gr = row0 + trow(o / TN), gc = col0 + tcol(o % TN);
                    if (gr >= M || gc >= N) continue;
                    T v;
                    int32_t ix;
                    if (!BDIRECT)
                        cpu_select<SR, T>(A + gr * K, 1, BT + gc * K, 1, K, v, ix);
                    else
                        cpu_select<SR, T>(A + gr * K, 1, B + gc, N, K, v, ix);
                    C[gr * N + gc] = v;
                    IDX[gr * N + gc] = ix;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < TM; ++i) store_row(i, acc[i], ch[i]);
            if constexpr (std::is_floating_point<T>::value) redo_outputs(true);
        }
    }
}

}  // namespace tg
