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
// lane, in lane order) is applied to its bins in lane order; blocks run in
// sequence.
//   * Bins in LDS (lds_apply): LDS float atomic adds (ds_add_f32 /
//     ds_add_f64, no return) apply the lanes of one instruction that hit
//     the same address in lane order, each an IEEE add rounded to nearest
//     even with denormals kept, and a wave's LDS instructions execute in
//     order.  Measured on gfx950 against the sequential sum in lane order:
//     bit-equal over random keys (1 to 64 distinct per block), mixed
//     magnitudes, round-to-even ties, denormal values and sums, signed
//     zeros, infinities and NaN positions, within one instruction and across
//     consecutive ones.  So one atomic per contribution keeps the
//     reference's order.  The LDS serves these atomics about one lane per
//     2.6 clocks per CU, about 30x slower than integer adds, so a block first
//     ranks its lanes per hash of the bin (a per-wave table of integer
//     counters, kRowCountSlots for grad_A and kCountSlots for grad_B; an
//     integer add with return, also served in lane order, gives each lane
//     the number of earlier lanes with its hash).
//     The first lane of each hash, which is the first lane of its bin, adds
//     with a plain read and write and clears the counter; the later lanes
//     then take the atomic.  A row (column) keeps a mode from its first
//     block: with more than kSecondPlainAbove later lanes there, the second
//     lane of each hash also adds plainly (after the first), and with more
//     than kAllSharedAbove the row runs on atomics only (the ranking would
//     spare too few).  The mode's branch is taken once per group of blocks,
//     so each mode's blocks are scheduled without per-block branches.
//   * Bins in global memory (K too large for LDS: global_apply): the lanes
//     sharing a bin are found by 64-bit ballots over the bits of the bin
//     index (wave_match_mask), and the lowest lane of each group (its
//     leader) applies the group: bin + g(leader) + g(2nd) + ... in lane
//     order, one read and one write of the bin.  Groups have distinct bins,
//     so they run side by side.  Summing (group_sum): in passes of
//     kStageRanks ranks, each member of rank r0 + u posts its value to slot
//     u of its leader's kStageRanks contiguous slots in a per-wave LDS stage,
//     and each leader whose group reaches rank r0 reads its slots with one
//     vector load: kStageRanks values, the missing ranks +0.0.  Adding +0.0
//     never changes a running sum that starts from +0.0 (such a sum is never
//     -0.0 under round-to-nearest), so the leader adds every slot
//     unconditionally.  It clears its slots behind it, so the stage is all
//     +0.0 between passes; no other lane touches the stage, which keeps the
//     LDS work of a pass proportional to the groups that need it.
//
#pragma once

#include "tg_kernels.hpp"

namespace tg {

// Mask of the active lanes whose key equals this lane's (0 for an inactive
// lane).  nbits: bits that can differ between keys (keys < 2^nbits).
__device__ __forceinline__ uint64_t wave_match_mask(uint32_t key, bool active, int nbits) {
    uint64_t match = __ballot(active);
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1u;
        const uint64_t m = __ballot(active && bit);
        match &= bit ? m : ~m;
    }
    return active ? match : 0;
}

// Bits needed for keys in [0, K).
__host__ __device__ inline int key_bits(int64_t K) {
    int b = 0;
    while (b < 31 && (int64_t(1) << b) < K) ++b;
    return b;
}

// Relaxed LDS accesses for the counters and bins that other lanes of the
// wave update: atomics, so the compiler keeps every access (no
// store-to-load forwarding across another lane's add).
template <typename U>
__device__ __forceinline__ U lds_ld(U* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
template <typename U>
__device__ __forceinline__ void lds_st(U* p, U v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
// LDS float add, no return (ds_add_f32 / ds_add_f64): same-address lanes of
// one instruction are applied in lane order (see the header comment).  The
// instruction is written out, so that no other lowering (a compare-and-swap
// loop would serve the lanes in no set order) can take its place.  Later LDS
// accesses of the wave are served after it; a wait the compiler places for
// them also covers it (LDS operations complete in order).
__device__ __forceinline__ void lds_fadd(float* p, float v) {
    const uint32_t a = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
    asm volatile("ds_add_f32 %0, %1" : : "v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_fadd(double* p, double v) {
    const uint32_t a = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
    asm volatile("ds_add_f64 %0, %1" : : "v"(a), "v"(v) : "memory");
}

// Ranks per stage pass.  A wave's stage: 64 leaders x kStageRanks slots
// (with LDS bins: the block's counters instead).  Passes per wait
// (group_sum, which the global-bin kernels use): measured when the LDS-bin
// kernels summed their groups the same way, 2 took C5-like argmax (MaxPlus
// f32 4096^3) from 129 to 122 us for grad_A and 158 to 148 us for grad_B
// against 1 pass; 4 was slower on uniformly random indices.
constexpr int kStageRanks = 4;
constexpr int kStagePasses = 2;
constexpr int kStageSlots = kStageRanks * 64;
constexpr int kStageElems = kStageSlots;
// grad_A's stage is twice as large: its LDS-bin rows rank on 512 counters
// (fewer hash collisions, so fewer lanes take the atomic), and one row more
// or less per CU changes nothing at K = 4096 (eight instead of nine).
constexpr int kRowStageElems = 2 * kStageSlots;

// The leader's sum before + g(leader) + g(rank 1) + g(rank 2) + ... of its
// group (m: this lane's group mask, 0 when inactive); meaningful on leaders
// only.  stage: this wave's kStageSlots slots, all +0.0 on entry and on
// return.  Wave-uniform: call with the whole wave active.
// Stage: 64 leaders x kStageRanks contiguous slots; 16-byte aligned (the
// kernels put the stages at the start of their LDS).  kStagePasses passes
// reuse the same slots back to back: LDS executes a wave's instructions in
// order, so a pass's stores land after the previous pass's loads and
// clears, and the wave waits once per kStagePasses passes, before the adds.
template <typename T>
__device__ __forceinline__ T group_sum(uint64_t m, T g, T before, bool& leader, T* stage) {
    typedef T Slots __attribute__((ext_vector_type(kStageRanks)));
    const int lane = threadIdx.x & 63;
    const uint32_t rank =
        __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u));
    leader = m != 0 && rank == 0;
    const int size = __popcll(m);
    T acc = before + g;
    if (__ballot(leader && size > 1)) {
        const int lead = m != 0 ? int(__builtin_ctzll(m)) : 0;
        Slots* mine = reinterpret_cast<Slots*>(stage) + lane;
        for (int r0 = 1; __ballot(leader && size > r0); r0 += kStagePasses * kStageRanks) {
            Slots v[kStagePasses];
#pragma unroll
            for (int p = 0; p < kStagePasses; ++p) {
                const int rp = r0 + p * kStageRanks;
                const uint32_t d = rank - uint32_t(rp);
                if (m != 0 && d < uint32_t(kStageRanks)) stage[lead * kStageRanks + int(d)] = g;
                // The members' stores are issued before the leaders' loads;
                // the compiler must not move them across, as it cannot see
                // the other lanes.
                asm volatile("" ::: "memory");
                v[p] = Slots(T(0));
                if (leader && size > rp) {
                    v[p] = *mine;
                    *mine = Slots(T(0));
                }
                asm volatile("" ::: "memory");
            }
#pragma unroll
            for (int p = 0; p < kStagePasses; ++p)
#pragma unroll
                for (int u = 0; u < kStageRanks; ++u) acc = acc + v[p][u];
        }
    }
    return acc;
}

// Zeroes this wave's stage of ELEMS elements (which hold its 32-bit
// counters with LDS bins).
template <int ELEMS, typename T>
__device__ __forceinline__ void stage_clear(T* stage) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < ELEMS / 64; ++u) stage[u * 64 + lane] = T(0);
    asm volatile("" ::: "memory");
}

// Zeroes this wave's n LDS bins, one 16-byte store per lane and step when n
// is a multiple of the vector (the bins then start 16-byte aligned: the
// stages and every wave's bins before them are whole vectors).
template <typename T>
__device__ __forceinline__ void bins_zero(T* bins, int64_t n) {
    constexpr int E = 16 / sizeof(T);
    typedef T V __attribute__((ext_vector_type(E)));
    const int lane = threadIdx.x & 63;
    if (n % E == 0) {
        for (int64_t k = int64_t(lane) * E; k < n; k += 64 * E) *reinterpret_cast<V*>(bins + k) = V(T(0));
    } else {
        for (int64_t k = lane; k < n; k += 64) bins[k] = T(0);
    }
}

// LDS bins: counters per wave (in its stage, zero between blocks), and the
// counts of later lanes (lanes after the first of their hash in the block)
// that set a row's (column's) mode from its first block.
constexpr int kCountSlots = 256;     // grad_B (its stage)
constexpr int kRowCountSlots = 512;  // grad_A (its larger stage)
constexpr int kAllSharedAbove = 48;
constexpr int kSecondPlainAbove = 8;
static_assert(kCountSlots * sizeof(uint32_t) <= kStageElems * sizeof(float) &&
                  kRowCountSlots * sizeof(uint32_t) <= kRowStageElems * sizeof(float),
              "the counters fit a wave's stage");

// bins[key] += g in lane order among equal keys, bins in LDS (see the header
// comment), in one of three modes that a row (column) keeps from its first
// block on.  MODE 0: the first lane of each hash adds plainly, the later
// lanes take the ordered atomic.  MODE 2 (rows whose blocks repeat bins
// often): the second lane of each hash also adds plainly, after the first,
// so fewer lanes take the atomic.  MODE 1 (blocks of few bins): atomics
// only.  Returns the mode that this block's ranks select.  Wave-uniform.
template <int MODE, int SLOTS, typename T>
__device__ __forceinline__ int lds_apply(T* bins, uint32_t* cnt, int32_t key, T g, bool active) {
    if constexpr (MODE == 1) {
        if (active) lds_fadd(bins + key, g);
        return 1;
    } else {
        // Integer adds with return are also served in lane order: r is the
        // number of earlier lanes of the block with this hash.
        const int h = key & (SLOTS - 1);
        const uint32_t r = active ? __hip_atomic_fetch_add(cnt + h, 1u, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_WAVEFRONT)
                                  : 0u;
        if (active && r == 0) {
            const T v = lds_ld(bins + key);
            lds_st(bins + key, v + g);
            lds_st(cnt + h, 0u);
        }
        // Each rank's writes are issued before the next rank's accesses.
        asm volatile("" ::: "memory");
        if constexpr (MODE == 2) {
            if (active && r == 1) {
                const T v = lds_ld(bins + key);
                lds_st(bins + key, v + g);
            }
            asm volatile("" ::: "memory");
        }
        if (active && r >= (MODE == 2 ? 2u : 1u)) lds_fadd(bins + key, g);
        const int later = __popcll(__ballot(active && r > 0));
        return __builtin_amdgcn_readfirstlane(later > kAllSharedAbove      ? 1
                                              : later > kSecondPlainAbove ? 2
                                                                          : 0);
    }
}

// Global bins belong to one wave and only its own lanes read them back, so
// their accesses are workgroup-scope atomics ordered by a workgroup-scope
// fence.  The lanes of a wave go through one CU's vector memory pipeline and
// L1 in order, so the AMDGPU memory model needs no wait or cache action for
// coherence among them (the fence compiles to none outside tgsplit mode).  A
// device-scope fence would also write the XCD's L2 back to memory
// (buffer_wbl2 on gfx950) on every block, for other XCDs these bins never
// reach.
template <typename T>
__device__ __forceinline__ T gbin_ld(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
template <typename T>
__device__ __forceinline__ void gbin_st(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void gbin_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup"); }

// bins[key * es] += g in lane order among equal keys, bins in global memory.
// The next block's leader for a bin may be another lane, so this block's
// writes are fenced before the wave issues its next reads.  Wave-uniform.
template <typename T>
__device__ __forceinline__ void global_apply(T* bins, T* stage, int64_t es, int32_t key, T g,
                                             bool active, int nbits) {
    const uint64_t m = wave_match_mask(uint32_t(key), active, nbits);
    const int lane = threadIdx.x & 63;
    const bool first = m != 0 && int(__builtin_ctzll(m)) == lane;
    T before = T(0);
    if (first) before = gbin_ld(bins + int64_t(key) * es);
    bool leader;
    const T acc = group_sum(m, g, before, leader, stage);
    if (leader) gbin_st(bins + int64_t(key) * es, acc);
    gbin_fence();
}

// ---------------------------------------------------------------------------
// grad_A.  rows = batch * M; row rr is (z = rr / M, i = rr % M).  Each wave
// owns one row at a time; LDS: a stage of kRowStageElems per wave, then K
// bins per wave (not with GLOBAL): waves * (kRowStageElems + K) * sizeof(T).
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
    constexpr int PF = 8;  // blocks of 64 contributions per prefetch chunk
    T* stage = reinterpret_cast<T*>(bwd_lds) + int64_t(wave) * kRowStageElems;
    T* row_bins =
        reinterpret_cast<T*>(bwd_lds) + int64_t(waves) * kRowStageElems + int64_t(wave) * K;
    uint32_t* const cnt = reinterpret_cast<uint32_t*>(stage);
    stage_clear<kRowStageElems>(stage);
    for (int64_t rr = int64_t(blockIdx.x) * waves + wave; rr < rows;
         rr += int64_t(gridDim.x) * waves) {
        const int64_t z = rr / M, i = rr - z * M;
        const T* g_row = G + z * sC + i * N;
        const int32_t* k_row = IDX + z * sC + i * N;
        const T* other = MULT ? OTHER + z * sO : nullptr;
        T* out = GA + z * sA + i * K;
        T* bins = GLOBAL ? out : row_bins;
        if constexpr (GLOBAL) {
            for (int64_t k = lane; k < K; k += 64) gbin_st(bins + k, T(0));
            gbin_fence();  // zeros visible to every lane's first read
        } else {
            bins_zero(bins, K);
        }
        int mode = -1;
        // Contributions in chunks of PF blocks of 64 consecutive j.  The next
        // chunk's loads are issued before the current chunk is applied
        // (unconditional loads of clamped columns, so each wait covers only
        // the older chunk), which hides the global latency behind PF blocks
        // of work; the MaxMul factors of a chunk are gathered at its start.
        auto load_chunk = [&](int64_t j0, int32_t (&kk)[PF], T (&gg)[PF]) {
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                const int64_t j = j0 + 64 * u + lane;
                kk[u] = k_row[j < N ? j : N - 1];
                gg[u] = g_row[j < N ? j : N - 1];
            }
        };
        int32_t kc[PF], kn[PF];
        T gc[PF], gn[PF];
        load_chunk(0, kc, gc);
        for (int64_t j0 = 0; j0 < N; j0 += 64 * PF) {
            load_chunk(j0 + 64 * PF, kn, gn);
            bool act[PF];
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                act[u] = j0 + 64 * u + lane < N && kc[u] >= 0 && int64_t(kc[u]) < K;
                if (MULT && act[u]) gc[u] = gc[u] * other[int64_t(kc[u]) * N + j0 + 64 * u + lane];
            }
            if constexpr (GLOBAL) {
#pragma unroll
                for (int u = 0; u < PF; ++u) {
                    if (j0 + 64 * u >= N) break;
                    global_apply<T>(bins, stage, 1, kc[u], gc[u], act[u], nbits);
                }
            } else {
                // The row's first block sets its mode; the mode's branch is
                // taken once per chunk, so each mode's blocks are scheduled
                // together.
                int u0 = 0;
                if (mode < 0) {
                    mode = lds_apply<0, kRowCountSlots, T>(bins, cnt, kc[0], gc[0], act[0]);
                    u0 = 1;
                }
                auto blocks = [&](auto mc) __attribute__((always_inline)) {
                    constexpr int MODE = decltype(mc)::value;
#pragma unroll
                    for (int u = 0; u < PF; ++u) {
                        if (j0 + 64 * u >= N) break;
                        if (u >= u0)
                            lds_apply<MODE, kRowCountSlots, T>(bins, cnt, kc[u], gc[u], act[u]);
                    }
                };
                if (mode == 0)
                    blocks(std::integral_constant<int, 0>{});
                else if (mode == 2)
                    blocks(std::integral_constant<int, 2>{});
                else
                    blocks(std::integral_constant<int, 1>{});
            }
#pragma unroll
            for (int u = 0; u < PF; ++u) {
                kc[u] = kn[u];
                gc[u] = gn[u];
            }
        }
        if constexpr (!GLOBAL) {
            // The row leaves as one contiguous run: non-temporal stores took
            // 1-3 us off grad_A at 4096^3 on every index pattern tried, and
            // 16-byte ones (with the 16-byte zeroing above) another 5-6 us.
            constexpr int E = 16 / sizeof(T);
            typedef T V __attribute__((ext_vector_type(E)));
            if (K % E == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
                for (int64_t k = int64_t(lane) * E; k < K; k += 64 * E)
                    __builtin_nontemporal_store(*reinterpret_cast<const V*>(bins + k),
                                                reinterpret_cast<V*>(out + k));
            } else {
                for (int64_t k = lane; k < K; k += 64) __builtin_nontemporal_store(bins[k], out + k);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// grad_B.  Column groups: batch * ceil(N / W) groups of W adjacent columns,
// W = waves per workgroup; group gg is (z = gg / groups_n, columns
// c0 = (gg % groups_n) * W ...).  Wave w owns column c0 + w and its K bins
// (LDS, or the grad_B column itself with GLOBAL).  The workgroup stages
// argmax and dC for its W columns in tiles of kBwdTileRows rows through LDS
// (row stride W + 1: the column reads of 64 lanes hit distinct banks); each
// wave then applies its column's tile in blocks of 64 rows, in row order.
// Every thread stages kBwdTileRows / 64 elements per tile and loads the next
// tile's into registers before the current tile is applied (unconditional
// loads of a clamped row and column), so the global latency hides behind a
// tile of bin updates and the waves meet at a barrier once per tile.
// Workgroups on one XCD (launch order b, b + 8, b + 16, ...) take adjacent
// column groups, so the W-column segments that share a cache line are read
// and written through one L2.
//   MULT: MaxMul rule, g *= A[z][i][k] (OTHER = A, row-major M x K).
// GLOBAL: the bins are the grad_B column itself, which the host zero-fills
// before the launch (one coalesced pass: zeroing a column here would take
// K stores of 4 or 8 bytes, N elements apart).
// KP: keys per pass.  Long columns (K >> M) whose bins do not fit the LDS
// eight at a time take their keys in passes of KP (a multiple of 4), which
// keeps 8 columns per group, so rows leave in 8-column pieces; each pass
// reads the group's M rows again.  Every bin still has one owner that adds
// in row order.  KP = K with GLOBAL.
// LDS: a stage of kStageElems per wave, W * KP bins (not with GLOBAL), then
// the tile, kBwdTileRows (W + 1) (4 + sizeof(T)) bytes.
// grid: any size (grid-stride over column groups), block = 64 * W, W <= 8.
// ---------------------------------------------------------------------------
constexpr int kBwdTileRows = 256;

template <typename T, bool MULT, bool GLOBAL>
__global__ __launch_bounds__(512) void tg_bwd_cols(const T* __restrict__ G,
                                                   const int32_t* __restrict__ IDX,
                                                   const T* __restrict__ OTHER, T* GB, int64_t M,
                                                   int64_t N, int64_t K, int64_t sC, int64_t sO,
                                                   int64_t sB, int64_t groups_n, int64_t groups,
                                                   int64_t KP) {
    extern __shared__ __align__(16) unsigned char bwd_lds[];
    constexpr int TB = kBwdTileRows / 64;  // blocks of 64 rows per tile
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int W = blockDim.x >> 6;
    const int stride = W + 1;
    const int nbits = key_bits(K);
    T* stage = reinterpret_cast<T*>(bwd_lds) + wave * kStageElems;
    uint32_t* const cnt = reinterpret_cast<uint32_t*>(stage);
    unsigned char* const after_stage = bwd_lds + size_t(W) * kStageElems * sizeof(T);
    T* bins_all = reinterpret_cast<T*>(after_stage);
    const int64_t bins_bytes = GLOBAL ? 0 : int64_t(W) * KP * int64_t(sizeof(T));
    T* tile_g = reinterpret_cast<T*>(after_stage + bins_bytes);
    int32_t* tile_k =
        reinterpret_cast<int32_t*>(after_stage + bins_bytes + kBwdTileRows * stride * sizeof(T));
    stage_clear<kStageElems>(stage);
    // This thread's staging slots: rows sr + 64 t (t < TB), column sq.
    const int sr = tid / W, sq = tid - (tid / W) * W;
    // XCD-aware order: with a grid that is a multiple of 8, launch slot b
    // (on XCD b % 8) takes rank (b % 8) * (grid / 8) + b / 8.
    const int64_t grid = gridDim.x;
    const int64_t b = blockIdx.x;
    const int64_t first = (grid % 8 == 0) ? (b % 8) * (grid / 8) + b / 8 : b;
    for (int64_t gg = first; gg < groups; gg += grid) {
        const int64_t z = gg / groups_n;
        const int64_t c0 = (gg - z * groups_n) * W;
        const int64_t c = c0 + wave;
        const T* gz = G + z * sC;
        const int32_t* kz = IDX + z * sC;
        const T* other = MULT ? OTHER + z * sO : nullptr;
        T* outz = GB + z * sB;
        // Keys in passes of KP (one pass when the W columns' bins fit the LDS):
        // each pass restages the group's rows and applies the keys of
        // [lo, hi) to bins lo.. of this wave's column.
        for (int64_t lo = 0; lo < K; lo += KP) {
            const int64_t hi = K - lo < KP ? K : lo + KP;
            // Bin of key k: bins[(k - lo) * es].
            T* bins = GLOBAL ? outz + c : bins_all + int64_t(wave) * KP;
            const int64_t es = GLOBAL ? N : 1;
            if (!GLOBAL && c < N) bins_zero(bins, hi - lo);
            int mode = -1;
            const int64_t cc = c0 + sq;
            const int64_t ccl = cc < N ? cc : N - 1;
            int32_t kr[TB];
            T gr[TB];
            auto stage_load = [&](int64_t i0) {
#pragma unroll
                for (int t = 0; t < TB; ++t) {
                    const int64_t i = i0 + 64 * t + sr;
                    const int64_t il = i < M ? i : M - 1;
                    const bool ok = i < M && cc < N;
                    const int32_t kl = kz[il * N + ccl];
                    const T gl = gz[il * N + ccl];
                    kr[t] = ok ? kl : -1;
                    gr[t] = ok ? gl : T(0);
                }
            };
            stage_load(0);
            for (int64_t i0 = 0; i0 < M; i0 += kBwdTileRows) {
                __syncthreads();  // the previous tile's readers are done
#pragma unroll
                for (int t = 0; t < TB; ++t) {
                    tile_k[(64 * t + sr) * stride + sq] = kr[t];
                    tile_g[(64 * t + sr) * stride + sq] = gr[t];
                }
                __syncthreads();
                stage_load(i0 + kBwdTileRows);
                if (c < N) {
                    // This column's blocks of the tile, in row order.
                    auto block = [&](int t, int32_t& key, T& g, bool& active) __attribute__((always_inline)) {
                        const int64_t it = i0 + 64 * t;
                        key = tile_k[(64 * t + lane) * stride + wave];
                        g = tile_g[(64 * t + lane) * stride + wave];
                        active = it < M && int64_t(key) >= lo && int64_t(key) < hi;
                        if (MULT && active) g = g * other[(it + lane) * K + key];
                        key -= int32_t(lo);
                    };
                    if constexpr (GLOBAL) {
#pragma unroll
                        for (int t = 0; t < TB; ++t) {
                            if (i0 + 64 * t >= M) break;
                            int32_t key; T g; bool active;
                            block(t, key, g, active);
                            global_apply<T>(bins, stage, es, key, g, active, nbits);
                        }
                    } else {
                        int t0 = 0;
                        if (mode < 0) {
                            int32_t key; T g; bool active;
                            block(0, key, g, active);
                            mode = lds_apply<0, kCountSlots, T>(bins, cnt, key, g, active);
                            t0 = 1;
                        }
                        auto blocks = [&](auto mc) __attribute__((always_inline)) {
                            constexpr int MODE = decltype(mc)::value;
#pragma unroll
                            for (int t = 0; t < TB; ++t) {
                                if (i0 + 64 * t >= M) break;
                                if (t >= t0) {
                                    int32_t key; T g; bool active;
                                    block(t, key, g, active);
                                    lds_apply<MODE, kCountSlots, T>(bins, cnt, key, g, active);
                                }
                            }
                        };
                        if (mode == 0)
                            blocks(std::integral_constant<int, 0>{});
                        else if (mode == 2)
                            blocks(std::integral_constant<int, 2>{});
                        else
                            blocks(std::integral_constant<int, 1>{});
                    }
                }
            }
            if constexpr (!GLOBAL) {
                __syncthreads();  // every wave's bins are complete
                // The W columns leave together: row k of the group is W
                // consecutive elements of grad_B.  A whole group of 8 columns
                // whose rows start 16-byte aligned leaves in 16-byte stores, 8 / E
                // threads per row, each gathering E columns from their bins;
                // otherwise blockDim = 64 W, and thread tid writes column
                // q = tid % W of rows tid / W, + 64, + 128, ...
                constexpr int E = 16 / sizeof(T);
                typedef T V __attribute__((ext_vector_type(E)));
                const bool vec = W == 8 && c0 + W <= N && N % E == 0 &&
                                 (reinterpret_cast<uintptr_t>(outz) & 15) == 0;
                if (vec) {
                    constexpr int TPR = 8 / E;
                    const int q0 = (tid % TPR) * E;
                    for (int64_t k = lo + tid / TPR; k < hi; k += 512 / TPR) {
                        V v;
#pragma unroll
                        for (int e = 0; e < E; ++e) v[e] = bins_all[int64_t(q0 + e) * KP + (k - lo)];
                        *reinterpret_cast<V*>(outz + k * N + c0 + q0) = v;
                    }
                } else if (c0 + sq < N) {
                    const T* src = bins_all + int64_t(sq) * KP;
                    T* dst = outz + c0 + sq;
                    for (int64_t k = lo + sr; k < hi; k += 64) dst[k * N] = src[k - lo];
                }
            }
            if (lo + KP < K) __syncthreads();  // the next pass zeroes the bins and restages
        }
        __syncthreads();  // the next group zeroes the bins and restages
    }
}

}  // namespace tg
