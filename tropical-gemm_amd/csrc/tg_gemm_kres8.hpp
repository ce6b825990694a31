// tg_gemm_kres8.hpp -- K-resident argmax kernel with 64 x 128 tiles for i32
// MaxPlus/MinPlus (gfx950).
//
// Same contract as tg_gemm_kres, for int32 MaxPlus/MinPlus with K in
// {64, 96, 128} and N a multiple of 128 (tall-skinny products such as
// Viterbi steps).  Each thread owns 4 rows x 8 columns of a 64 x 128 tile:
// per k a thread reads 4 A and 8 B values for 32 products (tg_gemm_kres: 4
// and 4 for 16), and runs 32 independent chains.
//
// Persistent: the grid holds every resident workgroup slot (two per CU at
// K = 128).  Workgroup w (renumbered per XCD) owns column tile w % tiles_n and
// walks the row tiles of all batch items with a stride of gridDim.x / tiles_n.
//   B panel  K x 128, resident in LDS (64 KB at K = 128), loaded when the
//            batch item changes and rewritten into keys once;
//   A panel  the next row tile's 64 x K panel is prefetched into registers
//            while the current one computes; it reaches LDS one 32-k tile at
//            a time through a two-slot ring (16 KB), so a k-tile is stored
//            while the previous one computes and one barrier per k-tile
//            suffices.
//
// Paths, chosen per row tile from the magnitudes of its A panel and the B
// panel:
//   f32 keys  every |x| < 2^15: value-only chain on keys (a+b)*256 + (255-k)
//             (MinPlus: + k), exact integers below 2^24 held as f32; the key
//             decodes to the value and the argmax (no resolve);
//   chunked   anything else: exact wrapping products, chunks of 8 k with one
//             compare and one select per output per chunk, resolved against
//             the A row (global memory, L2) and the raw B panel (LDS).  The B
//             panel is reloaded raw when a tile needs this path and rewritten
//             into keys again when the next tile does not.
//
// LDS layouts:
//   A slot s  64 rows x 32 k, row-major (128 B rows); the 16-byte quad q of
//             row r sits at quad position q ^ ((r >> 2) & 7), so the four
//             rows a wave reads at one k fall in different banks.
//   B         K rows x 128 columns, row-major (512 B rows).  Thread tx reads
//             columns tx*4 .. tx*4+3 and 64 + tx*4 .. 64 + tx*4+3.
#pragma once

#include "tg_gemm_dl.hpp"

namespace tg {

struct Kres8Cfg {
    static constexpr int BM = 64, BN = 128, BK = 32, TM = 4, TN = 8, CL = 8;
    static constexpr int A_TILE = BM * BK;  // elements per A k-tile slot
    static constexpr int KT_MIN = 2, KT_MAX = 4;
};

// True when tg_gemm_kres8 can run the problem: full 64 x 128 tiles, K a
// multiple of 32 from 64 to 128, 16-byte aligned operands, outputs and batch
// strides.  (The caller also checks for int32 and an additive semiring.)
inline bool kres8_fits(int64_t M, int64_t N, int64_t K, int64_t sA, int64_t sB, int64_t sC,
                       const void* A, const void* B, const void* C, const void* IDX) {
    auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    using Cfg = Kres8Cfg;
    return M > 0 && N > 0 && N < (int64_t(1) << 30) && M % Cfg::BM == 0 && N % Cfg::BN == 0 &&
           K % Cfg::BK == 0 &&
           K >= int64_t(Cfg::BK) * Cfg::KT_MIN && K <= int64_t(Cfg::BK) * Cfg::KT_MAX &&
           sA % 4 == 0 && sB % 4 == 0 && sC % 4 == 0 && a16(A) && a16(B) && a16(C) && a16(IDX);
}

// grid = (G, 1, 1) with G a multiple of tiles_n, block = 256.  K = 32 * KT.
template <int SR, int KT>
__global__ __launch_bounds__(TG_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void
tg_gemm_kres8(const int32_t* __restrict__ A, const int32_t* __restrict__ B,
              int32_t* __restrict__ C, int32_t* __restrict__ IDX, int64_t N, int64_t sA,
              int64_t sB, int64_t sC, int tiles_m, int tiles_n, int64_t batch) {
    static_assert(SR == SR_MAXPLUS || SR == SR_MINPLUS, "keys need an additive semiring");
    static_assert(KT >= Kres8Cfg::KT_MIN && KT <= Kres8Cfg::KT_MAX, "K-resident tile count");
    using Cfg = Kres8Cfg;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, TM = Cfg::TM, TN = Cfg::TN;
    constexpr int CL = Cfg::CL, CPT = BK / CL;
    constexpr int K = KT * BK;
    constexpr int BPW = K / 8;  // 1 KB direct-to-LDS B loads per wave (two k rows each)
    constexpr int BQ = K / 8;   // 16-byte B slots per thread
    constexpr int FORM_ORIG = 0, FORM_F32 = 1;
    __shared__ __align__(16) int32_t As[2 * Cfg::A_TILE];
    __shared__ __align__(16) int32_t Bs[K * BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tx = tid & 15;
    const int ty = tid >> 4;
    const int swz = ty & 7;  // (row >> 2) & 7 for the rows ty*4 .. ty*4+3
    // Consecutive workgroup ids go round-robin over the 8 XCDs; renumber so
    // the workgroups sharing a row tile (one per column tile) sit on one XCD.
    int lb = int(blockIdx.x);
    if ((gridDim.x & 7) == 0 && (int(gridDim.x >> 3) % tiles_n) == 0)
        lb = int(blockIdx.x & 7) * int(gridDim.x >> 3) + int(blockIdx.x >> 3);
    const int tn = lb % tiles_n;
    const int64_t step = int64_t(gridDim.x) / tiles_n;
    const int64_t total = batch * tiles_m;
    const int64_t col0 = int64_t(tn) * BN;
    int64_t r = int64_t(lb) / tiles_n;
    if (r >= total) return;

    // ---- A panel: registers -> LDS ring ---------------------------------
    // K-tile t of a row tile's 64 x K panel is 512 quads of 16 bytes; thread
    // tid holds quads tid and tid + 256 of every k-tile: pre[2t + u].
    Vec16<int32_t> pre[2 * KT];
    auto load_a = [&](int64_t rr) {
        const int64_t z = rr / tiles_m;
        const int64_t tm = rr - z * tiles_m;
        const int32_t* ap = A + z * sA + tm * BM * K;
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int qd = u * TG_THREADS + tid;
                pre[2 * t + u] =
                    *reinterpret_cast<const Vec16<int32_t>*>(ap + (qd >> 3) * K + t * BK + (qd & 7) * 4);
            }
    };
    auto store_tile = [&](auto tc, int form) {
        constexpr int t = decltype(tc)::value;
        int32_t* as = As + (t & 1) * Cfg::A_TILE;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int qd = u * TG_THREADS + tid;
            const int row = qd >> 3;
            Vec16<int32_t> v = pre[2 * t + u];
            if (form == FORM_F32) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v.v[e] = __float_as_int(float(int32_t(uint32_t(v.v[e]) << 8)));
            }
            *reinterpret_cast<Vec16<int32_t>*>(as + row * BK + (((qd & 7) ^ ((row >> 2) & 7)) << 2)) = v;
        }
    };
    // k-tile t of the prefetched panel into ring slot t & 1 (t is uniform).
    auto store_a = [&](int t, int form) {
        switch (t) {
            case 0: store_tile(std::integral_constant<int, 0>{}, form); break;
            case 1: store_tile(std::integral_constant<int, 1>{}, form); break;
            case 2: if constexpr (KT > 2) store_tile(std::integral_constant<int, 2>{}, form); break;
            default: if constexpr (KT > 3) store_tile(std::integral_constant<int, 3>{}, form); break;
        }
    };

    // ---- B panel ----------------------------------------------------------
    // Batch item z's K x 128 panel straight into LDS; each wave load covers
    // two k rows (1 KB).  Ends with a barrier.
    auto load_b = [&](int64_t z) {
        const int32_t* bz = B + z * sB + col0;
        // The lane's offset inside a row pair.  The empty asm keeps the
        // compiler from precomputing all BPW addresses once and holding them
        // (in spilled registers) across the whole kernel.
        int32_t lane_off = (lane >> 5) * int32_t(N) + (lane & 31) * 4;
        asm volatile("" : "+v"(lane_off));
#pragma unroll
        for (int q = 0; q < BPW; ++q) {
            const int p = wave * BPW + q;  // k row pair
            lds_load16(bz + int64_t(2 * p) * N + lane_off, Bs + p * 2 * BN);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    auto below = [](int32_t x, int bits) {
        return uint32_t(x) + (1u << (bits - 1)) < (1u << bits);  // unsigned: no overflow
    };
    // Workgroup-wide AND of pred, voted through four flag words in ring slot
    // 1 (two barriers; the leading one also ends every earlier use of the
    // ring).  Slot 1 is next written after the barrier that follows the
    // first k-tile's store, by which point every wave has read the flags.
    // (__syncthreads_and would add LDS of its own beyond the 80 KB that two
    // workgroups per CU leave at K = 128.)
    auto block_all = [&](int pred) {
        const int w = __all(pred);
        __syncthreads();
        if (lane == 0) As[Cfg::A_TILE + wave] = w;
        __syncthreads();
        return As[Cfg::A_TILE] & As[Cfg::A_TILE + 1] & As[Cfg::A_TILE + 2] & As[Cfg::A_TILE + 3];
    };
    // Rewrites the raw B panel in LDS into f32 keys b*256 + (255 - k)
    // (MinPlus: + k); ends with a barrier.
    auto rewrite_b = [&]() {
#pragma unroll
        for (int q = 0; q < BQ; ++q) {
            const int slot = q * TG_THREADS + tid;
            const int k = (slot * 4) / BN;
            const uint32_t low = SR == SR_MINPLUS ? uint32_t(k) : uint32_t(255 - k);
            Vec16<int32_t>* pv = reinterpret_cast<Vec16<int32_t>*>(Bs) + slot;
            Vec16<int32_t> v = *pv;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                v.v[e] = __float_as_int(float(int32_t((uint32_t(v.v[e]) << 8) + low)));
            *pv = v;
        }
        __syncthreads();
    };

    // Fragments of k pair (kk, kk+1) of k-tile t as element type U: A rows
    // ty*4+i from ring slot t & 1, B columns tx*4 + j and 64 + tx*4 + j.
    auto frag = [&](auto zero, int t, int kk, auto (&a)[TM][2], auto (&b)[2][TN]) {
        using U = decltype(zero);
        const U* as = reinterpret_cast<const U*>(As) + (t & 1) * Cfg::A_TILE;
        const U* bs = reinterpret_cast<const U*>(Bs) + t * BK * BN;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int off = (ty * 4 + i) * BK + (((kk >> 2) ^ swz) << 2) + (kk & 3);
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
    };

    int64_t zb = -1;        // batch item whose B panel is in LDS
    int bform = FORM_ORIG;  // form of the B panel in LDS
    int bok = 0;
    load_a(r);
    for (; r < total; r += step) {
        const int64_t z = r / tiles_m;
        const int64_t tm = r - z * tiles_m;
        if (z != zb) {
            __syncthreads();  // every wave is done with the previous B panel
            load_b(z);
            bform = FORM_ORIG;
            zb = z;
            int ok = 1;
#pragma unroll
            for (int q = 0; q < BQ; ++q) {
                const Vec16<int32_t> v = reinterpret_cast<const Vec16<int32_t>*>(Bs)[q * TG_THREADS + tid];
#pragma unroll
                for (int e = 0; e < 4; ++e) ok &= below(v.v[e], 16);
            }
            bok = block_all(ok);
        }
        int aok = 1;
#pragma unroll
        for (int q = 0; q < 2 * KT; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) aok &= below(pre[q].v[e], 16);
        // Also the barrier after the previous tile's last use of As and Bs.
        const int form = block_all(bok && aok) ? FORM_F32 : FORM_ORIG;
        if (form != bform) {
            if (bform != FORM_ORIG) load_b(z);  // restore the raw B panel
            if (form != FORM_ORIG) rewrite_b();
            bform = form;
        }
        const bool more = r + step < total;
        // K-tile pipeline: slot t & 1 holds k-tile t; k-tile t+1 is stored
        // while t computes; the barrier closing iteration t makes it visible
        // and frees slot t & 1 for k-tile t+2.  The next row tile's panel is
        // requested once its last k-tile is stored.
        store_a(0, form);
        __syncthreads();
        if (KT == 1 && more) load_a(r + step);

        const int64_t row0 = tm * BM + ty * 4;
        int32_t* Ct = C + z * sC + row0 * N + col0 + tx * 4;
        int32_t* It = IDX + z * sC + row0 * N + col0 + tx * 4;
        auto store_row = [&](int i, const int32_t (&cv)[TN], const int32_t (&iv)[TN]) {
            Vec16<int32_t> c0, c1, i0, i1;
#pragma unroll
            for (int j = 0; j < TN / 2; ++j) {
                c0.v[j] = cv[j];
                c1.v[j] = cv[j + TN / 2];
                i0.v[j] = iv[j];
                i1.v[j] = iv[j + TN / 2];
            }
            // Non-temporal (streaming) stores: the outputs are not read
            // again here, and keeping them out of the caches measured 6%
            // faster on the Viterbi shape (262144 x 128 x 128).
            typedef int v4i_t __attribute__((ext_vector_type(4)));
            auto stream16 = [](int32_t* p, const Vec16<int32_t>& v) {
                v4i_t x;
                __builtin_memcpy(&x, &v, 16);
                __builtin_nontemporal_store(x, reinterpret_cast<v4i_t*>(p));
            };
            stream16(Ct + int64_t(i) * N, c0);
            stream16(Ct + int64_t(i) * N + BN / 2, c1);
            stream16(It + int64_t(i) * N, i0);
            stream16(It + int64_t(i) * N + BN / 2, i1);
        };

        if (form == FORM_F32) {
            float key[TM][TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) key[i][j] = tzero<SR, float>();
#pragma unroll 1
            for (int t = 0; t < KT; ++t) {
                if (t + 1 < KT) {
                    store_a(t + 1, FORM_F32);
                    if (t + 2 == KT && more) load_a(r + step);
                }
#pragma unroll
                for (int kk = 0; kk < BK; kk += 2) {
                    float a[TM][2], b[2][TN];
                    frag(0.0f, t, kk, a, b);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            key[i][j] = tjoin<SR, float>(tjoin<SR, float>(key[i][j], a[i][0] + b[0][j]),
                                                         a[i][1] + b[1][j]);
                }
                __syncthreads();
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                int32_t cv[TN], iv[TN];
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int32_t ik = int32_t(key[i][j]);  // exact: an integer key
                    cv[j] = ik >> 8;
                    iv[j] = SR == SR_MINPLUS ? (ik & 255) : 255 - (ik & 255);
                }
                store_row(i, cv, iv);
            }
            continue;
        }

        // ---- chunked path -------------------------------------------------
        // acc: running value; ch: last chunk that strictly improved it (-1: the
        // tropical zero was never beaten).  Each chunk folds its products into
        // a max3/min3 chain that starts from acc, so the chunk improved acc iff
        // the chain's result beats acc strictly.
        int32_t acc[TM][TN], ch[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                acc[i][j] = tzero<SR, int32_t>();
                ch[i][j] = -1;
            }
#pragma unroll 1
        for (int t = 0; t < KT; ++t) {
            if (t + 1 < KT) {
                store_a(t + 1, FORM_ORIG);
                if (t + 2 == KT && more) load_a(r + step);
            }
#pragma unroll
            for (int s = 0; s < CPT; ++s) {
                int32_t an[TM][TN];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) an[i][j] = acc[i][j];
#pragma unroll
                for (int kk = s * CL; kk < (s + 1) * CL; kk += 2) {
                    int32_t a[TM][2], b[2][TN];
                    frag(int32_t(0), t, kk, a, b);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int j = 0; j < TN; ++j)
                            an[i][j] = tjoin<SR, int32_t>(
                                tjoin<SR, int32_t>(an[i][j], tmul<SR, int32_t>(a[i][0], b[0][j])),
                                tmul<SR, int32_t>(a[i][1], b[1][j]));
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        if (tbetter<SR, int32_t>(an[i][j], acc[i][j])) ch[i][j] = t * CPT + s;
                        acc[i][j] = an[i][j];
                    }
            }
            __syncthreads();
        }
        // Resolve each output inside its recorded chunk: the chunk holds the
        // final value as its own extremum and no earlier product reaches it,
        // so the first k in the chunk whose product equals the final value is
        // the argmax.  A comes from global memory (L2), B from the raw panel.
        // Outputs whose zero was never beaten keep it, with argmax 0.
        const int32_t* Az = A + z * sA + row0 * K;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            int32_t cv[TN], iv[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int c = ch[i][j];
                const int k0 = (c < 0 ? 0 : c) * CL;
                const Vec16<int32_t> a0 = *reinterpret_cast<const Vec16<int32_t>*>(Az + i * K + k0);
                const Vec16<int32_t> a1 = *reinterpret_cast<const Vec16<int32_t>*>(Az + i * K + k0 + 4);
                const int col = (j < TN / 2 ? 0 : BN / 2) + tx * 4 + (j % (TN / 2));
                int f = CL - 1;
#pragma unroll
                for (int kk = CL - 2; kk >= 0; --kk) {
                    const int32_t av = kk < 4 ? a0.v[kk] : a1.v[kk - 4];
                    f = tmul<SR, int32_t>(av, Bs[(k0 + kk) * BN + col]) == acc[i][j] ? kk : f;
                }
                cv[j] = c < 0 ? tzero<SR, int32_t>() : acc[i][j];
                iv[j] = c < 0 ? 0 : k0 + f;
                // One output's loads at a time: hoisting all 32 outputs' A
                // windows would take the registers of a second wave per SIMD.
                __builtin_amdgcn_sched_barrier(0);
            }
            store_row(i, cv, iv);
        }
    }
}

}  // namespace tg
