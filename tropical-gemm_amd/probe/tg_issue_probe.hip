// tg_issue_probe.hip -- register-only issue-rate probe for the tropical
// inner loop on gfx950 (no memory traffic in the timed loop).
//
// Each lane runs 8 x 4 independent accumulator chains; per iteration every
// chain takes two products, acc = max(max(acc, a[r] + b[j]), a2[r] + b2[j]),
// plus 8 operand updates.  The measured rate bounds what a tiled kernel can
// reach with the same instruction mix:
//   f32, A in VGPRs:  v_add_f32 x2 + v_max3_f32 (or v_maximum3_f32) per 2
//                     products (the mix of tg_gemm_dl's main loop)
//   f32, A in SGPRs:  the same with one operand wave-uniform (scalar loads)
//   f64:              v_add_f64 x2 + v_max_f64 x2 per 2 products (no
//                     three-input f64 max on gfx950)
//   f32, DPP operand: the VGPR mix with the second add's B operand read
//                     from the partner lane (lane ^ 1) through DPP, the
//                     operand feed that would let lane pairs share B
//                     fragments instead of each reading them from LDS
// Grid: 256 workgroups x waves_per_simd of 256 threads (4 waves, one per
// SIMD), so waves/SIMD = 1, 2, 4 or 8 across the sweep.
//
// A second probe times LDS reads alone (ds_read_b128, eight independent
// reads per iteration, 32 KB of LDS per workgroup): every lane reading its
// own 16 bytes (1 KB per instruction), and the fragment pattern of the
// tiled kernels' B reads, where the 64 lanes of a wave read 16 distinct
// 16-byte vectors (256 B per instruction, each delivered to 4 lanes).
// Build: make -C tropical-gemm_amd probe; run: tropical-gemm_amd/probe/tg_issue_probe
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CK(x)                                                                        \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                            \
        }                                                                            \
    } while (0)

enum Mix { F32_VGPR = 0, F32_SGPR = 1, F32_IEEE = 2, F64_VGPR = 3, F32_DPP = 4 };

// d = bsrc(lane ^ 1) + a: v_add_f32 with a DPP quad permutation on its first
// operand.  bsrc must not be written by a VALU instruction in the two
// instructions before (the DPP read hazard): the probe never writes it in
// the loop.
__device__ __forceinline__ float add_partner(float bsrc, float a) {
    float d;
    asm volatile("v_add_f32_dpp %0, %1, %2 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf"
                 : "=v"(d)
                 : "v"(bsrc), "v"(a));
    return d;
}

template <typename T, int MIX>
__global__ __launch_bounds__(256) void chains(const T* __restrict__ a_in, const T* __restrict__ b_in,
                                              T* __restrict__ out, int iters) {
    T a[8], a2[8];
    for (int r = 0; r < 8; ++r) {
        if constexpr (MIX == F32_SGPR) {  // wave-uniform: kept in SGPRs
            a[r] = a_in[r];
            a2[r] = a_in[r + 8];
        } else {  // per-lane: kept in VGPRs
            const T d = T(threadIdx.x >> 10);
            a[r] = a_in[r] + d;
            a2[r] = a_in[r + 8] + d;
        }
    }
    T b[4], b2[4];
    for (int j = 0; j < 4; ++j) {
        b[j] = b_in[threadIdx.x * 8 + j];
        b2[j] = b_in[threadIdx.x * 8 + 4 + j];
    }
    T acc[8][4];
    for (int r = 0; r < 8; ++r)
        for (int j = 0; j < 4; ++j) acc[r][j] = T(-1e30);
    if constexpr (MIX == F32_DPP) asm volatile("s_nop 4" ::: "memory");  // b2 settled for DPP
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (MIX == F32_DPP)
                    acc[r][j] = __builtin_fmax(__builtin_fmax(acc[r][j], a[r] + b[j]),
                                               add_partner(b2[j], a2[r]));
                else if constexpr (MIX == F32_IEEE)
                    acc[r][j] = __builtin_elementwise_maximum(
                        __builtin_elementwise_maximum(acc[r][j], a[r] + b[j]), a2[r] + b2[j]);
                else
                    acc[r][j] = __builtin_fmax(__builtin_fmax(acc[r][j], a[r] + b[j]), a2[r] + b2[j]);
            }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            b[j] = b[j] + T(0.5);
            if constexpr (MIX != F32_DPP) b2[j] = b2[j] - T(0.25);  // DPP: b2 stays put
        }
    }
    T s = 0;
    for (int r = 0; r < 8; ++r)
        for (int j = 0; j < 4; ++j) s += acc[r][j];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

// LDS read throughput: lane l of a wave reads vector (l % DISTINCT) of its
// wave's window; the window moves every iteration.
template <int DISTINCT>
__global__ __launch_bounds__(256) void lds_reads(unsigned* __restrict__ out, int iters) {
    __shared__ __align__(16) uint4 buf[2048];  // 32 KB
    const int tid = threadIdx.x;
    for (int i = tid; i < 2048; i += 256) buf[i] = make_uint4(i, 3 * i, 5 * i, 7 * i);
    __syncthreads();
    const int wave = tid >> 6, lane = tid & 63;
    int base = wave * 64 + lane % DISTINCT;
    uint4 keep = make_uint4(0, 0, 0, 0);
    for (int it = 0; it < iters; ++it) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = buf[(base + u * 256) & 2047];
#pragma unroll
        for (int u = 0; u < 8; ++u) asm volatile("" ::"v"(v[u].x), "v"(v[u].y), "v"(v[u].z), "v"(v[u].w));
        keep.x ^= v[0].x;
        base += 17;
    }
    out[blockIdx.x * 256 + tid] = keep.x;
}

template <int DISTINCT>
void run_lds(const char* name, int wgs_per_cu, int iters) {
    unsigned* o;
    const int blocks = 256 * wgs_per_cu;
    CK(hipMalloc(&o, size_t(blocks) * 256 * sizeof(unsigned)));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int w = 0; w < 3; ++w) hipLaunchKernelGGL((lds_reads<DISTINCT>), dim3(blocks), dim3(256), 0, 0, o, iters);
    CK(hipGetLastError());
    CK(hipEventRecord(e0));
    const int reps = 5;
    for (int w = 0; w < reps; ++w) hipLaunchKernelGGL((lds_reads<DISTINCT>), dim3(blocks), dim3(256), 0, 0, o, iters);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    ms /= reps;
    const double instr = double(blocks) * 4 * iters * 8;  // wave instructions
    std::printf("%-28s wgs/CU=%d  %.3f ms  %5.3f wave-reads/ns per CU  %6.1f B/ns per CU delivered  %6.1f B/ns per CU distinct\n",
                name, wgs_per_cu, ms, instr / ms / 1e6 / 256, instr * 1024 / ms / 1e6 / 256,
                instr * 16 * DISTINCT / ms / 1e6 / 256);
    std::fflush(stdout);
    CK(hipFree(o));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
}

template <typename T, int MIX>
void run(const char* name, int wps, int iters, int instr_per_iter) {
    T *a, *b, *o;
    const int blocks = 256 * wps;
    CK(hipMalloc(&a, 64 * sizeof(T)));
    CK(hipMalloc(&b, 256 * 8 * sizeof(T)));
    CK(hipMalloc(&o, size_t(blocks) * 256 * sizeof(T)));
    CK(hipMemset(a, 0, 64 * sizeof(T)));
    CK(hipMemset(b, 0, 256 * 8 * sizeof(T)));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int w = 0; w < 3; ++w) hipLaunchKernelGGL((chains<T, MIX>), dim3(blocks), dim3(256), 0, 0, a, b, o, iters);
    CK(hipGetLastError());
    CK(hipEventRecord(e0));
    const int reps = 5;
    for (int w = 0; w < reps; ++w) hipLaunchKernelGGL((chains<T, MIX>), dim3(blocks), dim3(256), 0, 0, a, b, o, iters);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    ms /= reps;
    const double lanes = double(blocks) * 256;
    const double instrs = lanes * iters * instr_per_iter;
    const double trop = lanes * iters * 64 * 2;  // 64 products per iteration, 2 ops each
    std::printf("%-28s waves/SIMD=%d  %.3f ms  %6.1f T lane-instr/s  %6.1f T tropical ops/s\n", name, wps, ms,
                instrs / ms / 1e9, trop / ms / 1e9);
    std::fflush(stdout);
    CK(hipFree(a));
    CK(hipFree(b));
    CK(hipFree(o));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
}

int main() {
    const int iters = 4096;
    for (int wps = 1; wps <= 8; wps *= 2) {
        // per iteration: 64 adds + 32 three-input maxes + 8 operand updates (f32),
        // 64 adds + 64 maxes + 8 operand updates (f64)
        run<float, F32_VGPR>("f32 add+max3, A in VGPR", wps, iters, 64 + 32 + 8);
        run<float, F32_IEEE>("f32 add+maximum3, A in VGPR", wps, iters, 64 + 32 + 8);
        run<float, F32_SGPR>("f32 add+max3, A in SGPR", wps, iters, 64 + 32 + 8);
        run<double, F64_VGPR>("f64 add+max, A in VGPR", wps, iters, 64 + 64 + 8);
        run<float, F32_DPP>("f32 add+max3, B2 via DPP", wps, iters, 64 + 32 + 4);
    }
    for (int w = 1; w <= 4; ++w) {
        run_lds<64>("LDS b128, 64 distinct/wave", w, 4000);
        run_lds<16>("LDS b128, 16 distinct/wave", w, 4000);
    }
    return 0;
}
