// tg_gemm_kresw.hpp -- K-resident argmax kernel with wave-private row tiles
// for i32 MaxPlus/MinPlus (gfx950).
//
// Same contract as tg_gemm_kres8 (int32 MaxPlus/MinPlus with argmax, K in
// {64, 96, 128}, N a multiple of 128), for tall-skinny products such as
// Viterbi steps.  One 1024-thread workgroup per CU holds the K x 128 B panel
// of its column tile in LDS as f32 keys; each of its 16 waves then works on
// its own 16-row tiles with no workgroup barrier:
//   A   a wave streams its 16 x K rows through its own two-slot LDS ring,
//       one 32-k tile at a time (prefetched into registers while the
//       previous k-tile computes); only the wave itself writes and reads its
//       slots, and LDS runs a wave's instructions in order, so no barrier is
//       needed between the store of a k-tile and its reads;
//   B   loaded once per batch item (the only barriers of the kernel);
//   out each lane owns rows ty*4 .. ty*4+3 and columns tx*4 .. tx*4+3 and
//       64 + tx*4 .. 64 + tx*4+3 of the 16 x 128 tile; C and argmax leave
//       through non-temporal 16-byte stores.
// Four waves per SIMD (<= 128 VGPRs) cover the LDS and global latency that
// the 4-wave workgroups of tg_gemm_kres8 cover with barriers between them.
//
// Paths:
//   f32 keys  every |x| < 2^15 in the B panel (one vote per batch item) and
//             in the wave's A rows (checked per k-tile before it is
//             stored): a max3/min3 chain on keys (a+b)*256 + (255-k)
//             (MinPlus: + k), exact integers below 2^24 held as f32; the
//             key decodes to the value and the argmax;
//   exact     anything else (the wave drops a tile as soon as one of its
//             k-tiles leaves the range): (value, k) updated on every strict
//             improvement in k order, A and B read from global memory (L2).
#pragma once

#include "tg_gemm_kres8.hpp"

namespace tg {

struct KreswCfg {
    static constexpr int WAVES = 16, ROWS = 16, BK = 32, BN = 128, TM = 4, TN = 8;
    static constexpr int SLOT = ROWS * BK;  // elements per A ring slot
    static constexpr int KT_MIN = 2, KT_MAX = 4;
    static constexpr int MAX_COL_TILES = 16;
};

// Dynamic LDS bytes of tg_gemm_kresw at K = 32 * KT: the B panel, every
// wave's two A slots, one vote word (padded to 16 bytes).
__host__ __device__ constexpr size_t kresw_lds_bytes(int KT) {
    return size_t(KT * KreswCfg::BK * KreswCfg::BN + KreswCfg::WAVES * 2 * KreswCfg::SLOT) * 4 + 16;
}

// True when tg_gemm_kresw can run the problem: 16-row tiles, N a multiple of
// 128 with at most 16 column tiles, K a multiple of 32 from 64 to 128,
// 16-byte aligned operands, outputs and batch strides.  (The caller also
// checks for int32 and an additive semiring.)
inline bool kresw_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, int64_t sC,
                       const void* A, const void* B, const void* C, const void* IDX) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    using Cfg = KreswCfg;
    return M > 0 && N > 0 && M % Cfg::ROWS == 0 && M / Cfg::ROWS < (int64_t(1) << 31) &&
           N % Cfg::BN == 0 && N / Cfg::BN <= Cfg::MAX_COL_TILES && K % Cfg::BK == 0 &&
           K >= int64_t(Cfg::BK) * Cfg::KT_MIN && K <= int64_t(Cfg::BK) * Cfg::KT_MAX &&
           sA % 4 == 0 && sB % 4 == 0 && sC % 4 == 0 && a16(A) && a16(B) && a16(C) && a16(IDX);
}

// grid = (G, 1, 1) with G a multiple of tiles_n (one workgroup per CU),
// block = 1024, dynamic LDS = kresw_lds_bytes(KT).  K = 32 * KT.
template <int SR, int KT>
__global__ __launch_bounds__(1024) void tg_gemm_kresw(const int32_t* __restrict__ A,
                                                      const int32_t* __restrict__ B,
                                                      int32_t* __restrict__ C,
                                                      int32_t* __restrict__ IDX, int64_t M,
                                                      int64_t N, int64_t sA, int64_t sB,
                                                      int64_t sC, int tiles_n, int64_t batch) {
    static_assert(SR == SR_MAXPLUS || SR == SR_MINPLUS, "keys need an additive semiring");
    static_assert(KT >= KreswCfg::KT_MIN && KT <= KreswCfg::KT_MAX, "K-resident tile count");
    using Cfg = KreswCfg;
    constexpr int BK = Cfg::BK, BN = Cfg::BN, TM = Cfg::TM, TN = Cfg::TN, ROWS = Cfg::ROWS;
    constexpr int K = KT * BK;
    extern __shared__ __align__(16) unsigned char kw_lds[];
    float* const Bs = reinterpret_cast<float*>(kw_lds);
    int* const vote = reinterpret_cast<int*>(kw_lds + kresw_lds_bytes(KT) - 16);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tx = lane & 15;
    const int ty = lane >> 4;  // rows ty*4 .. ty*4+3 of the wave's tile
    float* const As = Bs + K * BN + wave * 2 * Cfg::SLOT;

    const int tn = int(blockIdx.x) % tiles_n;
    const int64_t col0 = int64_t(tn) * BN;
    const int64_t groups = int64_t(gridDim.x) / tiles_n;  // workgroups per column tile
    const int64_t first = (int64_t(blockIdx.x) / tiles_n) * Cfg::WAVES + wave;
    const int64_t stride = groups * Cfg::WAVES;
    const int64_t tiles = M / ROWS;

    auto small = [](int32_t x) { return uint32_t(x) + 32768u < 65536u; };  // |x| < 2^15
    // k-tile t of row tile rr: 16 rows x 32 k = 128 quads; lane holds quads
    // lane and lane + 64 (row q >> 3, k quad q & 7).  Wave-uniform bases,
    // 32-bit lane offsets.
    Vec16<int32_t> pa[2];
    const int a_off = (lane >> 3) * K + (lane & 7) * 4;  // quad lane; quad lane + 64 is 8 rows on
    auto load_a = [&](const int32_t* Az, int64_t rr, int t) {
        const int32_t* base = Az + rr * (ROWS * K) + t * BK;
        pa[0] = *reinterpret_cast<const Vec16<int32_t>*>(base + a_off);
        pa[1] = *reinterpret_cast<const Vec16<int32_t>*>(base + a_off + 8 * K);
    };
    auto pa_small = [&]() {
        bool ok = true;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) ok = ok && small(pa[u].v[e]);
        return __all(ok) != 0;
    };
    // A keys a*256 into slot s; quad q of row r at quad position q ^ ((r >> 2) & 7).
    auto store_a = [&](int s) {
        float* as = As + s * Cfg::SLOT;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int q = u * 64 + lane;
            const int row = q >> 3;
            float4 o;
            o.x = float(int32_t(uint32_t(pa[u].v[0]) << 8));
            o.y = float(int32_t(uint32_t(pa[u].v[1]) << 8));
            o.z = float(int32_t(uint32_t(pa[u].v[2]) << 8));
            o.w = float(int32_t(uint32_t(pa[u].v[3]) << 8));
            *reinterpret_cast<float4*>(as + row * BK + (((q & 7) ^ ((row >> 2) & 7)) << 2)) = o;
        }
    };
    typedef int v4i_t __attribute__((ext_vector_type(4)));
    // Row i of the lane's rows in row tile rr.
    auto store_row = [&](int32_t* Cz, int32_t* Iz, int64_t rr, int i, const int32_t (&cv)[TN],
                         const int32_t (&iv)[TN]) {
        v4i_t c0, c1, i0, i1;
#pragma unroll
        for (int j = 0; j < TN / 2; ++j) {
            c0[j] = cv[j];
            c1[j] = cv[j + TN / 2];
            i0[j] = iv[j];
            i1[j] = iv[j + TN / 2];
        }
        // Computed here from an opaque copy of the lane id: hoisted out of
        // the tile loop, the four rows' addresses would stay live (and
        // spill) across the main loop.
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int64_t base = rr * ROWS * N + col0;
        const int off = ((ln >> 4) * 4 + i) * int(N) + (ln & 15) * 4;
        int32_t* cp = Cz + base + off;
        int32_t* ip = Iz + base + off;
        __builtin_nontemporal_store(c0, reinterpret_cast<v4i_t*>(cp));
        __builtin_nontemporal_store(c1, reinterpret_cast<v4i_t*>(cp + BN / 2));
        __builtin_nontemporal_store(i0, reinterpret_cast<v4i_t*>(ip));
        __builtin_nontemporal_store(i1, reinterpret_cast<v4i_t*>(ip + BN / 2));
    };

    for (int64_t z = 0; z < batch; ++z) {
        const int32_t* Az = A + z * sA;
        const int32_t* Bz = B + z * sB + col0;
        int32_t* Cz = C + z * sC;
        int32_t* Iz = IDX + z * sC;
        // B panel as keys (b << 8) + (255 - k) (MinPlus: + k), with a vote on
        // the f32-key range.  The first barrier ends every wave's use of the
        // previous item's panel and vote; the second orders the vote's reset
        // before the threads that clear it.
        __syncthreads();
        if (tid == 0) *vote = 1;
        __syncthreads();
        bool bsmall = true;
        for (int q = tid; q < K * BN / 4; q += 1024) {
            const int k = (q * 4) / BN;
            const Vec16<int32_t> v =
                *reinterpret_cast<const Vec16<int32_t>*>(Bz + int64_t(k) * N + (q * 4) % BN);
            const uint32_t low = SR == SR_MINPLUS ? uint32_t(k) : uint32_t(255 - k);
            float4 o;
            o.x = float(int32_t((uint32_t(v.v[0]) << 8) + low));
            o.y = float(int32_t((uint32_t(v.v[1]) << 8) + low));
            o.z = float(int32_t((uint32_t(v.v[2]) << 8) + low));
            o.w = float(int32_t((uint32_t(v.v[3]) << 8) + low));
            *reinterpret_cast<float4*>(Bs + q * 4) = o;
#pragma unroll
            for (int e = 0; e < 4; ++e) bsmall = bsmall && small(v.v[e]);
        }
        if (!bsmall) *vote = 0;
        __syncthreads();
        const bool bkeys = *vote != 0;

        int64_t r = first;
        if (bkeys && r < tiles) load_a(Az, r, 0);
        for (; r < tiles; r += stride) {
            const bool more = r + stride < tiles;
            bool fast = bkeys;
            if (fast) {
                float key[TM][TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) key[i][j] = tzero<SR, float>();
#pragma unroll 1
                for (int t = 0; t < KT; ++t) {
                    if (!pa_small()) {  // wave-uniform: the tile takes the exact path
                        fast = false;
                        break;
                    }
                    store_a(t & 1);
                    if (t + 1 < KT) load_a(Az, r, t + 1);
                    else if (more) load_a(Az, r + stride, 0);
                    const float* as = As + (t & 1) * Cfg::SLOT;
                    const float* bs = Bs + t * BK * BN;
#pragma unroll
                    for (int kk = 0; kk < BK; kk += 2) {
                        float a[TM][2], b[2][TN];
#pragma unroll
                        for (int i = 0; i < TM; ++i) {
                            const int off = (ty * 4 + i) * BK + (((kk >> 2) ^ ty) << 2) + (kk & 3);
                            a[i][0] = as[off];
                            a[i][1] = as[off + 1];
                        }
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int j = 0; j < TN / 2; ++j) {
                                b[h][j] = bs[(kk + h) * BN + tx * 4 + j];
                                b[h][j + TN / 2] = bs[(kk + h) * BN + BN / 2 + tx * 4 + j];
                            }
#pragma unroll
                        for (int i = 0; i < TM; ++i)
#pragma unroll
                            for (int j = 0; j < TN; ++j)
                                key[i][j] = tjoin<SR, float>(
                                    tjoin<SR, float>(key[i][j], a[i][0] + b[0][j]),
                                    a[i][1] + b[1][j]);
                        // One k pair's fragments at a time: hoisting more would
                        // take the registers of the fourth wave per SIMD.
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                if (fast) {
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        int32_t cv[TN], iv[TN];
#pragma unroll
                        for (int j = 0; j < TN; ++j) {
                            const int32_t ik = int32_t(key[i][j]);  // exact: an integer key
                            cv[j] = ik >> 8;
                            iv[j] = SR == SR_MINPLUS ? (ik & 255) : 255 - (ik & 255);
                        }
                        store_row(Cz, Iz, r, i, cv, iv);
                    }
                    continue;
                }
            }
            // ---- exact path -----------------------------------------------
            // The reference's rule per output: from the tropical zero with
            // index 0, take (p, k) on every strict improvement, k ascending
            // (core/argmax.rs:24-33, core/kernel.rs:119-167).  One half of the
            // lane's columns at a time (registers for a fourth wave per
            // SIMD); four A values of a row per 16-byte load, the half's 4 B
            // values per k as one 16-byte load, both from L2.
            {
                const int32_t* arow = Az + (r * ROWS + ty * 4) * K;
#pragma unroll 1
                for (int h = 0; h < 2; ++h) {
                    int32_t val[TM][4], ix[TM][4];
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            val[i][j] = tzero<SR, int32_t>();
                            ix[i][j] = 0;
                        }
                    const int32_t* bcol = Bz + h * (BN / 2) + tx * 4;
#pragma unroll 1
                    for (int k0 = 0; k0 < K; k0 += 4) {
                        Vec16<int32_t> a4[TM];
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            a4[i] = *reinterpret_cast<const Vec16<int32_t>*>(arow + i * K + k0);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const Vec16<int32_t> b4 =
                                *reinterpret_cast<const Vec16<int32_t>*>(bcol + int64_t(k0 + e) * N);
#pragma unroll
                            for (int i = 0; i < TM; ++i)
#pragma unroll
                                for (int j = 0; j < 4; ++j) {
                                    const int32_t p = tmul<SR, int32_t>(a4[i].v[e], b4.v[j]);
                                    const bool take = tbetter<SR, int32_t>(p, val[i][j]);
                                    val[i][j] = take ? p : val[i][j];
                                    ix[i][j] = take ? k0 + e : ix[i][j];
                                }
                        }
                    }
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        v4i_t cv, iv;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            cv[j] = val[i][j];
                            iv[j] = ix[i][j];
                        }
                        int ln = lane;
                        asm volatile("" : "+v"(ln));
                        const int64_t o = (r * ROWS + (ln >> 4) * 4 + i) * N + col0 + h * (BN / 2) +
                                          (ln & 15) * 4;
                        __builtin_nontemporal_store(cv, reinterpret_cast<v4i_t*>(Cz + o));
                        __builtin_nontemporal_store(iv, reinterpret_cast<v4i_t*>(Iz + o));
                    }
                }
            }
            if (bkeys && more) load_a(Az, r + stride, 0);
        }
    }
}

}  // namespace tg
