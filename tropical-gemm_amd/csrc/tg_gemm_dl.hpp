// tg_gemm_dl.hpp -- direct-to-LDS tropical GEMM for 32-bit types (gfx950).
//
// Same contract as tg_gemm_tiles (tg_kernels.hpp), for problems whose tiles
// are all full: M % 64 == 0, N % 128 == 0, K % 32 == 0, 16-byte aligned A, B
// and batch strides.  Tiles go from HBM straight into LDS with
// global_load_lds_dwordx4 (no staging registers, no LDS-store VALU work),
// which frees the registers the argmax bookkeeping needs and keeps three
// waves per SIMD resident.
//
// Layouts (per LDS buffer; two buffers, loads of chunk t+1 overlap the
// compute of chunk t):
//   A tile  64 rows x 32 k, row-major (128 B rows).  The 16-byte quad q of
//           row r is stored at quad position q ^ ((r >> 2) & 7), so the four
//           rows a wave reads at one k fall in different banks.
//   B tile  32 k x 128 cols, row-major (512 B rows).
// Each thread owns 4 consecutive rows (ty*4 + i) and 8 columns
// (g*64 + tx*4 + e): per pair of k it reads four ds_read_b64 of A and four
// ds_read_b128 of B for 64 products.
#pragma once

#include "tg_kernels.hpp"

namespace tg {

// Tile configurations: 16 x 16 threads, 4 x TN outputs per thread.
//   TN = 8: 64 x 128 tiles; argmax held to 3 waves/SIMD (<= 168 VGPRs),
//           value-only at 2 (its schedule wants ~200 VGPRs).
//   TN = 4: 64 x 64 tiles, 4 waves/SIMD (<= 128 VGPRs): twice the tiles, so
//           4096^2 outputs make exactly 4 rounds of 1024 resident workgroups.
template <int TN_>
struct DlCfg {
    static constexpr int BM = 64, BN = 16 * TN_, BK = TG_CHUNK, TM = 4, TN = TN_;
    static constexpr int WAVES_ARGMAX = TN_ == 8 ? 3 : 4;
    static constexpr int WAVES_VALUE = TN_ == 8 ? 2 : 4;
    static constexpr int NBI = BK * BN / 1024;      // 1 KB B-tile loads per wave
    static constexpr int RPI = 256 / BN;            // B k-rows per 1 KB load
    static constexpr int LPR = BN / 4;              // lanes per B k-row
    static constexpr int A_BYTES = BM * BK * 4;   // one A buffer
    static constexpr int B_BYTES = BK * BN * 4;   // one B buffer
    static constexpr int TILE_BYTES = 2 * (A_BYTES + B_BYTES);
    // Argmax epilogue, reusing the tile buffers: bucket counts, per-output
    // chunk (u16), chunk-sorted output list (u16), per-output result (u8),
    // then a few words of scan scratch past the tile buffers.
    static constexpr int OUTS = BM * BN;            // outputs per tile
    static constexpr int NB_MAX = 2048;             // chunk buckets
    static constexpr int HIST_OFF = 0;
    static constexpr int CHS_OFF = HIST_OFF + NB_MAX * 4;
    static constexpr int LIST_OFF = CHS_OFF + OUTS * 2;
    static constexpr int RES_OFF = LIST_OFF + OUTS * 2;
    static constexpr int MISC_OFF = RES_OFF + OUTS;
    static constexpr int LDS_BYTES = (MISC_OFF + 64 > TILE_BYTES) ? MISC_OFF + 64 : TILE_BYTES;
    static_assert(MISC_OFF <= TILE_BYTES, "epilogue arrays must fit in the tile buffers");
};

// Exclusive prefix sum over the 256 threads of a workgroup; returns the
// exclusive prefix of x and sets total.  scratch: 5 ints of LDS.
__device__ __forceinline__ int block_exclusive_scan(int x, int* scratch, int& total) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
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

// True when tg_gemm_dl<.., TN, CL> can run the problem: K and N multiples of
// 4 and 16-byte aligned operands, outputs and batch strides (tiles load and
// store 16 bytes per lane), and chunk indices that fit the epilogue's 16-bit
// slots.  M, N and K need not fill the tiles: the loads of a partial tile
// clamp their rows, columns and k into the matrix (in-bounds duplicates),
// the k past K of the last k-tile are then overwritten in LDS with operands
// whose product is the tropical zero, and the stores skip rows past M and
// 4-column groups past N.
template <int TN, int CL>
inline bool dl_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, int64_t sC,
                    const void* A, const void* B, const void* C, const void* IDX) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    return M > 0 && N > 0 && K > 0 && N % 4 == 0 && K % 4 == 0 && (K + CL - 1) / CL < 0xFFFF &&
           sA % 4 == 0 && sB % 4 == 0 && sC % 4 == 0 && a16(A) && a16(B) && a16(C) &&
           (IDX == nullptr || a16(IDX));
}

// True when every tile of the problem is full.
template <int TN>
inline bool dl_full_tiles(int64_t M, int64_t N, int64_t K) {
    return M % DlCfg<TN>::BM == 0 && N % DlCfg<TN>::BN == 0 && K % DlCfg<TN>::BK == 0;
}

// Split K for problems with too few 64 x 64 tiles (partial ones included) to
// fill the chip: the largest power of two S with at most 1024 workgroups in
// total, slices of at least 256 k and slice lengths that are multiples of 64.
// N a multiple of 4, as the kernel needs (the merge then reads whole 16-byte
// groups of the dense M x N partials).
inline int dl_splits(int64_t M, int64_t N, int64_t K, int64_t batch) {
    if (M <= 0 || N <= 0 || N % 4 != 0 || K % 64 != 0 || batch <= 0) return 1;
    const int64_t tiles = ((M + 63) / 64) * ((N + 63) / 64) * batch;
    int s = 1;
    while (tiles * s * 2 <= 1024 && K % (int64_t(64) * s * 2) == 0 && K / (s * 2) >= 256) s *= 2;
    return s;
}

// Combines the S split-K partials of tg_gemm_dl.  Slices are visited in k
// order and a later slice replaces the running result only if strictly
// better, so equal values keep the earlier slice's index and bits: the
// reference's first-k rule across slices.  Partials are dense, slice stride
// sY = batch * M * N; outputs use the batch stride sC.  16-byte vectors
// (N, so M * N, is a multiple of 4 here).
template <int SR, typename T, bool ARGMAX>
__global__ __launch_bounds__(256) void tg_merge_splits(const T* __restrict__ PV,
                                                       const int32_t* __restrict__ PI,
                                                       T* __restrict__ C, int32_t* __restrict__ IDX,
                                                       int S, int64_t MN, int64_t batch, int64_t sY,
                                                       int64_t sC) {
    const int64_t nvec = batch * MN / 4;
    const int64_t stride = int64_t(gridDim.x) * 256;
    for (int64_t v = int64_t(blockIdx.x) * 256 + threadIdx.x; v < nvec; v += stride) {
        const int64_t e = v * 4;
        const int64_t z = e / MN;
        const int64_t r = e - z * MN;
        Vec16<T> best = *reinterpret_cast<const Vec16<T>*>(PV + e);
        Vec16<int32_t> bi{};
        if constexpr (ARGMAX) bi = *reinterpret_cast<const Vec16<int32_t>*>(PI + e);
        for (int y = 1; y < S; ++y) {
            const Vec16<T> pv = *reinterpret_cast<const Vec16<T>*>(PV + y * sY + e);
            Vec16<int32_t> pi{};
            if constexpr (ARGMAX) pi = *reinterpret_cast<const Vec16<int32_t>*>(PI + y * sY + e);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (tbetter<SR, T>(pv.v[q], best.v[q])) {
                    best.v[q] = pv.v[q];
                    if constexpr (ARGMAX) bi.v[q] = pi.v[q];
                }
            }
        }
        *reinterpret_cast<Vec16<T>*>(C + z * sC + r) = best;
        if constexpr (ARGMAX) *reinterpret_cast<Vec16<int32_t>*>(IDX + z * sC + r) = bi;
    }
}

// Waves per SIMD come from the tile configuration (DlCfg): other resident
// waves hide the LDS latency of the main loop.
// TAILK: K is not a multiple of BK (the last k-tile is partial); a separate
// instantiation, so full-K problems run the plain pipeline.
template <int SR, typename T, bool ARGMAX, int TN_, int CL, bool TAILK = false>
__global__ __launch_bounds__(TG_THREADS) __attribute__((amdgpu_waves_per_eu(
    ARGMAX ? DlCfg<TN_>::WAVES_ARGMAX : DlCfg<TN_>::WAVES_VALUE))) void tg_gemm_dl(
    const T* __restrict__ A, const T* __restrict__ B, const T* __restrict__ BT,
    T* __restrict__ C, int32_t* __restrict__ IDX, int64_t M, int64_t N, int64_t K, int64_t sA,
    int64_t sB, int64_t sC, int tiles_m, int tiles_n, int64_t KS, int64_t sY) {
    static_assert(sizeof(T) == 4, "direct-to-LDS kernel is for 32-bit types");
    using Cfg = DlCfg<TN_>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, TM = Cfg::TM, TN = Cfg::TN;
    constexpr int NBI = Cfg::NBI;
    static_assert(CL == 8 || CL == 16 || CL == 32, "argmax chunk of 8, 16 or 32 k");
    extern __shared__ __align__(16) unsigned char dl_lds[];
    T* const As0 = reinterpret_cast<T*>(dl_lds);
    T* const Bs0 = reinterpret_cast<T*>(dl_lds + 2 * Cfg::A_BYTES);

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
    // Split K: slice y covers k in [y*KS, (y+1)*KS) and writes its (value,
    // argmax) partial at C/IDX + y*sY (tg_merge_splits combines them).  An
    // unsplit launch has gridDim.y == 1, KS == K and sY == 0.
    const int64_t y = blockIdx.y;
    C += z * sC + y * sY;
    if (ARGMAX) {
        IDX += z * sC + y * sY;
        BT += z * (N * K);
    }

    // Per-lane global sources of this wave's direct loads (chunk 0).  A: 8
    // rows per 1 KB instruction, wave w issues instructions 2w, 2w+1.  B:
    // RPI k-rows per instruction, wave w issues NBI*w .. NBI*w + NBI-1.  In a
    // partial tile, rows past M read row M-1 and 4-column groups past N read
    // the last group: in-bounds duplicates that only feed outputs that are
    // never stored.
    const T* srcA[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = (wave * 2 + q) * 8 + (lane >> 3);
        const int qpos = lane & 7;
        const int qsrc = qpos ^ ((r >> 2) & 7);
        const int64_t gr = row0 + r < M ? row0 + r : M - 1;
        srcA[q] = A + gr * K + qsrc * 4;
    }
    const T* srcB[NBI];
#pragma unroll
    for (int q = 0; q < NBI; ++q) {
        const int kr = (wave * NBI + q) * Cfg::RPI + lane / Cfg::LPR;
        const int64_t gc = col0 + (lane % Cfg::LPR) * 4;
        srcB[q] = B + int64_t(kr) * N + (gc < N ? gc : N - 4);
    }
    auto issue_loads = [&](int64_t t, int buf) {
        T* adst = As0 + buf * (BM * BK);
        T* bdst = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int q = 0; q < 2; ++q)
            lds_load16(srcA[q] + t * BK, adst + (wave * 2 + q) * 256);
#pragma unroll
        for (int q = 0; q < NBI; ++q)
            lds_load16(srcB[q] + t * BK * N, bdst + (wave * NBI + q) * 256);
    };
    // The last k-tile when K is not a multiple of BK: A quads past K read the
    // row's last quad and B rows past K read row K-1 (in bounds; overwritten
    // in LDS by patch_tail before use).
    auto issue_tail_loads = [&](int64_t t, int buf) {
        T* adst = As0 + buf * (BM * BK);
        T* bdst = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int r = (wave * 2 + q) * 8 + (lane >> 3);
            const int qsrc = (lane & 7) ^ ((r >> 2) & 7);
            const int64_t kq = t * BK + qsrc * 4;
            lds_load16(srcA[q] - qsrc * 4 + (kq < K - 4 ? kq : K - 4), adst + (wave * 2 + q) * 256);
        }
#pragma unroll
        for (int q = 0; q < NBI; ++q) {
            const int kr = (wave * NBI + q) * Cfg::RPI + lane / Cfg::LPR;
            const int64_t kk = t * BK + kr;
            lds_load16(srcB[q] - int64_t(kr) * N + (kk < K - 1 ? kk : K - 1) * N,
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

    T acc[TM][TN];
    int32_t ch[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            acc[i][j] = tzero<SR, T>();
            ch[i][j] = -1;
        }

    // Fragment reads.  A: row ty*4+i, k pair (kk, kk+1) at its swizzled quad.
    const int swz = ty & 7;
    auto load_frag = [&](int buf, int kk, T (&a)[TM][2], T (&b)[2][TN]) {
        const T* as = As0 + buf * (BM * BK);
        const T* bs = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int r = ty * 4 + i;
            const int off = r * BK + (((kk >> 2) ^ swz) << 2) + (kk & 3);
            a[i][0] = as[off];
            a[i][1] = as[off + 1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[h][j] = bs[(kk + h) * BN + (j >> 2) * 64 + tx * 4 + (j & 3)];
    };

    // k-tiles [t0, t1) of this slice; t (and so every chunk index) is global.
    // Split slices are whole k-tiles; an unsplit K may end in a partial one
    // holding kv valid k.
    const int64_t t0 = y * (KS / BK);
    const int64_t t1 = t0 + (KS + BK - 1) / BK;
    const int kv = TAILK ? int(KS - (t1 - 1 - t0) * BK) : BK;
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

        // The LDS tile holds BK / CL argmax chunks of CL consecutive k.  Each
        // chunk folds its products into a max3/min3 chain that starts from
        // the running value, so the running value needs no separate update;
        // with argmax the chunk is recorded iff the chain's result beats the
        // value held before the chunk strictly (the reference's "keep acc iff
        // acc >= p").
#pragma unroll
        for (int s = 0; s < BK / CL; ++s) {
            T an[TM][TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) an[i][j] = acc[i][j];
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
                        an[i][j] = tjoin<SR, T>(tjoin<SR, T>(an[i][j], p0), p1);
                    }
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (ARGMAX) {
                        if (tbetter<SR, T>(an[i][j], acc[i][j]))
                            ch[i][j] = int32_t(t * (BK / CL) + s);
                    }
                    acc[i][j] = an[i][j];
                }
        }
    }

    // ---- epilogue ------------------------------------------------------------
    // Output (i, j) of this thread: tile row ty*4+i, tile column (j>>2)*64 +
    // tx*4 + (j&3); its local id is row*BN + column.
    auto store_row = [&](int i, const T (&v)[TN], const int32_t (&ix)[TN]) {
        const int64_t gr = row0 + ty * 4 + i;
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
    if constexpr (!ARGMAX) {
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            int32_t none[TN] = {};
            store_row(i, acc[i], none);
        }
    } else {
        // Exact first k inside each output's recorded chunk c.  The window of
        // chunk c holds the final value as its own maximum (no product of an
        // earlier chunk reaches it), so the window alone gives the target and
        // the first k attaining it.  Outputs are resolved in chunk order
        // (LDS counting sort), so workgroups running side by side read the
        // same A-row / B^T-row segments at about the same time and mostly hit
        // in cache.  The resolve returns the offset inside the chunk and, for
        // a zero maximum, the sign of the first zero product (the CPU keeps
        // the first occurrence's bits).
        constexpr uint16_t NONE = 0xFFFF;
        uint32_t* hist = reinterpret_cast<uint32_t*>(dl_lds + Cfg::HIST_OFF);
        uint16_t* chs = reinterpret_cast<uint16_t*>(dl_lds + Cfg::CHS_OFF);
        uint16_t* list = reinterpret_cast<uint16_t*>(dl_lds + Cfg::LIST_OFF);
        uint8_t* res = dl_lds + Cfg::RES_OFF;
        int* misc = reinterpret_cast<int*>(dl_lds + Cfg::MISC_OFF);
        // Buckets: chunk >> shift, at most NB_MAX of them.
        const int64_t nchunks = (K + CL - 1) / CL;
        int shift = 0;
        while (((nchunks - 1) >> shift) >= Cfg::NB_MAX) ++shift;
        const int nb = int(((nchunks - 1) >> shift) + 1);

        __syncthreads();  // every wave is done with the tile buffers
        for (int b = tid; b < nb; b += TG_THREADS) hist[b] = 0;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int lid = (ty * 4 + i) * BN + (j >> 2) * 64 + tx * 4 + (j & 3);
                chs[lid] = ch[i][j] < 0 ? NONE : uint16_t(ch[i][j]);
            }
        __syncthreads();
        uint16_t rank[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                rank[i][j] = ch[i][j] < 0 ? 0 : uint16_t(atomicAdd(&hist[ch[i][j] >> shift], 1u));
        __syncthreads();
        // Exclusive scan of the bucket counts, 8 buckets per thread.
        constexpr int PER = Cfg::NB_MAX / TG_THREADS;
        int cnt[PER];
        int mine = 0;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int b = tid * PER + q;
            cnt[q] = b < nb ? int(hist[b]) : 0;
            mine += cnt[q];
        }
        int total = 0;
        int run = block_exclusive_scan(mine, misc, total);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int b = tid * PER + q;
            if (b < nb) hist[b] = uint32_t(run);
            run += cnt[q];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if (ch[i][j] >= 0) {
                    const int lid = (ty * 4 + i) * BN + (j >> 2) * 64 + tx * 4 + (j & 3);
                    list[hist[ch[i][j] >> shift] + rank[i][j]] = uint16_t(lid);
                }
            }
        __syncthreads();

        // Resolve, chunk-sorted, one output per thread at a time (two in
        // flight would push the kernel past the 3-waves-per-SIMD register
        // budget of the main loop).
        constexpr int NW = CL / 4;
        constexpr int G = 1;
        for (int e0 = 0; e0 < total; e0 += TG_THREADS * G) {
            int lid[G];
            int64_t c[G];
            bool valid[G];
            Vec16<T> av[G][NW], bv[G][NW];
            const T* ap[G];
            const T* bp[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const int e = e0 + g * TG_THREADS + tid;
                valid[g] = e < total;
                lid[g] = valid[g] ? int(list[e]) : 0;
                c[g] = valid[g] ? int64_t(chs[lid[g]]) : 0;
                // Clamped like the tile loads (outputs past M or N are not
                // stored; their windows just stay in bounds).  Quads of a
                // window past K read the row's last quad: duplicates that
                // come after their originals, so the first match is a k < K.
                const int64_t gr = row0 + lid[g] / BN, gc = col0 + (lid[g] & (BN - 1));
                ap[g] = A + (gr < M ? gr : M - 1) * K + c[g] * CL;
                bp[g] = BT + (gc < N ? gc : N - 1) * K + c[g] * CL;
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    const int64_t off =
                        (!TAILK || c[g] * CL + w * 4 <= K - 4) ? w * 4 : K - 4 - c[g] * CL;
                    av[g][w] = *reinterpret_cast<const Vec16<T>*>(ap[g] + off);
                    bv[g][w] = *reinterpret_cast<const Vec16<T>*>(bp[g] + off);
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                T p[CL];
#pragma unroll
                for (int kk = 0; kk < CL; ++kk)
                    p[kk] = tmul<SR, T>(av[g][kk >> 2].v[kk & 3], bv[g][kk >> 2].v[kk & 3]);
                T mx = tjoin<SR, T>(p[0], p[1]);
#pragma unroll
                for (int kk = 2; kk < CL; kk += 2) mx = tjoin<SR, T>(tjoin<SR, T>(mx, p[kk]), p[kk + 1]);
                // Last match scanning downwards == first match; groups of 8
                // compares keep few lane masks live at once.
                int f = 0;
#pragma unroll
                for (int q = CL / 8 - 1; q >= 0; --q) {
#pragma unroll
                    for (int kk = q * 8 + 7; kk >= q * 8; --kk) f = (p[kk] == mx) ? kk : f;
                    __builtin_amdgcn_sched_barrier(0);
                }
                int r = f;
                if constexpr (std::is_floating_point<T>::value) {
                    if (mx == T(0) && __builtin_signbit(tmul<SR, T>(ap[g][f], bp[g][f]))) r |= 32;
                }
                if (valid[g]) res[lid[g]] = uint8_t(r);
            }
        }
        __syncthreads();

#pragma unroll
        for (int i = 0; i < TM; ++i) {
            T v[TN];
            int32_t ix[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int lid = (ty * 4 + i) * BN + (j >> 2) * 64 + tx * 4 + (j & 3);
                const uint16_t cc = chs[lid];
                if (cc == NONE) {  // the tropical zero was never beaten
                    v[j] = tzero<SR, T>();
                    ix[j] = 0;
                } else {
                    const int r = res[lid];
                    ix[j] = int32_t(cc) * CL + (r & 31);
                    v[j] = acc[i][j];
                    if constexpr (std::is_floating_point<T>::value) {
                        if (v[j] == T(0)) v[j] = (r & 32) ? -T(0) : T(0);
                    }
                }
            }
            store_row(i, v, ix);
        }
    }
}

}  // namespace tg
