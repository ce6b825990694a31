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

struct DlCfg {
    static constexpr int BM = 64, BN = 128, BK = TG_CHUNK, TM = 4, TN = 8;
    static constexpr int A_BYTES = BM * BK * 4;   // one A buffer
    static constexpr int B_BYTES = BK * BN * 4;   // one B buffer
    static constexpr int LDS_BYTES = 2 * (A_BYTES + B_BYTES);
};

// One 16-byte direct load per lane: global src -> LDS at dst + lane * 16
// (dst must be the same for the whole wave).  A non-template wrapper: the
// builtin with template-dependent pointer types is not accepted by the host
// compilation pass.
__device__ __forceinline__ void lds_load16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// True when tg_gemm_dl can run the problem.
inline bool dl_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, const void* A,
                    const void* B) {
    return M > 0 && N > 0 && K > 0 && M % DlCfg::BM == 0 && N % DlCfg::BN == 0 &&
           K % DlCfg::BK == 0 && sA % 4 == 0 && sB % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(A) & 15u) == 0 && (reinterpret_cast<uintptr_t>(B) & 15u) == 0;
}

template <int SR, typename T, bool ARGMAX>
__global__ __launch_bounds__(TG_THREADS) void tg_gemm_dl(
    const T* __restrict__ A, const T* __restrict__ B, const T* __restrict__ BT,
    T* __restrict__ C, int32_t* __restrict__ IDX, int64_t M, int64_t N, int64_t K, int64_t sA,
    int64_t sB, int64_t sC, int tiles_m, int tiles_n) {
    static_assert(sizeof(T) == 4, "direct-to-LDS kernel is for 32-bit types");
    constexpr int BM = DlCfg::BM, BN = DlCfg::BN, BK = DlCfg::BK, TM = DlCfg::TM, TN = DlCfg::TN;
    extern __shared__ __align__(16) unsigned char dl_lds[];
    T* const As0 = reinterpret_cast<T*>(dl_lds);
    T* const Bs0 = reinterpret_cast<T*>(dl_lds + 2 * DlCfg::A_BYTES);

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
    if (ARGMAX) {
        IDX += z * sC;
        BT += z * (N * K);
    }

    // Per-lane global sources of this wave's direct loads (chunk 0).  A: 8
    // rows per 1 KB instruction, wave w issues instructions 2w, 2w+1.  B: 2
    // k-rows per instruction, wave w issues 4w .. 4w+3.
    const T* srcA[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int r = (wave * 2 + q) * 8 + (lane >> 3);
        const int qpos = lane & 7;
        const int qsrc = qpos ^ ((r >> 2) & 7);
        srcA[q] = A + (row0 + r) * K + qsrc * 4;
    }
    const T* srcB[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int kr = (wave * 4 + q) * 2 + (lane >> 5);
        srcB[q] = B + int64_t(kr) * N + col0 + (lane & 31) * 4;
    }
    auto issue_loads = [&](int64_t t, int buf) {
        T* adst = As0 + buf * (BM * BK);
        T* bdst = Bs0 + buf * (BK * BN);
#pragma unroll
        for (int q = 0; q < 2; ++q)
            lds_load16(srcA[q] + t * BK, adst + (wave * 2 + q) * 256);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_load16(srcB[q] + t * BK * N, bdst + (wave * 4 + q) * 256);
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

    const int64_t ntiles = K / BK;
    issue_loads(0, 0);
    for (int64_t t = 0; t < ntiles; ++t) {
        const int buf = int(t & 1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (t + 1 < ntiles) issue_loads(t + 1, buf ^ 1);

        T cm[TM][TN];
        {
            T a[TM][2], b[2][TN];
            load_frag(buf, 0, a, b);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    cm[i][j] = tjoin<SR, T>(tmul<SR, T>(a[i][0], b[0][j]), tmul<SR, T>(a[i][1], b[1][j]));
        }
#pragma unroll
        for (int kk = 2; kk < BK; kk += 2) {
            T a[TM][2], b[2][TN];
            load_frag(buf, kk, a, b);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const T p0 = tmul<SR, T>(a[i][0], b[0][j]);
                    const T p1 = tmul<SR, T>(a[i][1], b[1][j]);
                    cm[i][j] = tjoin<SR, T>(tjoin<SR, T>(cm[i][j], p0), p1);
                }
        }
        // Strict improvement only (the reference's "keep acc iff acc >= p").
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if constexpr (ARGMAX) {
                    if (tbetter<SR, T>(cm[i][j], acc[i][j])) ch[i][j] = int32_t(t);
                }
                acc[i][j] = tjoin<SR, T>(acc[i][j], cm[i][j]);
            }
    }

    // ---- epilogue ------------------------------------------------------------
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int64_t gr = row0 + ty * 4 + i;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t gc = col0 + (j >> 2) * 64 + tx * 4 + (j & 3);
            T val = acc[i][j];
            int32_t idx = 0;
            if constexpr (ARGMAX) {
                // Exact first k inside the recorded chunk (see tg_gemm_tiles).
                constexpr int NW = BK / 4;
                const int64_t c = ch[i][j] < 0 ? 0 : ch[i][j];
                const T* ap = A + gr * K + c * BK;
                const T* bp = BT + gc * K + c * BK;
                Vec16<T> av[NW], bv[NW];
#pragma unroll
                for (int w = 0; w < NW; ++w) {
                    av[w] = reinterpret_cast<const Vec16<T>*>(ap)[w];
                    bv[w] = reinterpret_cast<const Vec16<T>*>(bp)[w];
                }
                int32_t f = 0;
#pragma unroll
                for (int qd = BK / 8 - 1; qd >= 0; --qd) {
#pragma unroll
                    for (int kk = qd * 8 + 7; kk >= qd * 8; --kk) {
                        const T p = tmul<SR, T>(av[kk >> 2].v[kk & 3], bv[kk >> 2].v[kk & 3]);
                        f = (p == val) ? kk : f;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                idx = int32_t(c * BK + f);
                if constexpr (std::is_floating_point<T>::value) {
                    if (val == T(0)) val = tmul<SR, T>(ap[f], bp[f]);
                }
                if (ch[i][j] < 0) {
                    val = tzero<SR, T>();
                    idx = 0;
                }
                IDX[gr * N + gc] = idx;
            }
            C[gr * N + gc] = val;
        }
    }
}

}  // namespace tg
