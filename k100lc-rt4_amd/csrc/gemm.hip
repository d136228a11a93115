// gemm.hip -- RT4 W4A8 prefill GEMM on gfx950 int8 matrix cores.
//
//   C[m][n] = Σ_g sa[g][m] * sb[g][n] * I[m][n][g],
//   I[m][n][g] = Σ_{k in group g} q8[m][k] * code[n][k]        (exact int32)
//
// with q8 the prefill activation codes (quant_rows_a8_k semantics, src/k_new.hip:
// 268-301: q8 = 16h + l), sa their per-(group, row) scale (`sc`), code the RT4 int4
// weights and sb the fp32 group-major weight scales (src/model.cpp:190-202).
//
// The reference computes this as two int4 x int4 passes over the digit planes h
// and l plus an add (k_gemm_i4_a8, src/k_gemm.hip:22-34; kernel gemm_w4a4,
// kernels/gemm_core.h:59-206).  Per group its integer content is
// 16*I_h + I_l = I exactly, so here the digits are recombined into int8 once
// and a single int8 contraction runs on v_mfma_i32_32x32x32_i8.
//
// Tiling.  Workgroup tile 128 activation rows x 256 weight rows, 8 waves, each
// wave a 64 x 64 block = 2 x 2 MFMA tiles of 32 x 32; one 128-wide K group is
// four MFMA k-steps.  The int32 accumulators restart at every group (srcC = 0)
// and are folded into fp32 with one fma per output:
//     facc += f32(acc) * (sa * sb),   acc = 16*I exactly (x16 nibble unpack),
// and the result is scaled by 1/16 once at the end (a power of two, so the bits
// equal those of scaling every term).
//
// Data movement.  Per group the workgroup moves 16 KB of int8 activations, 16 KB
// of packed weights and the two scale vectors from global memory straight into
// LDS with global_load_lds_dwordx4 (no VGPR round trip), four stages deep, XOR-
// swizzled so the MFMA fragment reads are bank-conflict free; the weights stay
// packed in LDS and are unpacked after the ds_read.  The LDS DMA is issued from
// inline asm so the compiler does not serialise every LDS read behind all
// outstanding DMA; the kernel waits for the stage it reads (s_waitcnt vmcnt +
// barrier) itself.
//
// Scheduling ("stream-K").  With 128 x 256 tiles the 27B shapes give 544 or 160
// tiles for 256 CUs, so a plain one-tile-per-workgroup grid would leave up to
// 30-40% of the machine idle in the last round.  Instead one persistent
// workgroup per CU takes an equal, contiguous share of the (tile, group) units.
// A tile split between workgroups is combined deterministically: every
// contributor except the last writes its fp32 partial to a workspace slot
// (agent-coherent stores), bumps the tile's counter, and the contributor that
// arrives last sums all partials in workgroup order and writes C; it also resets
// the counter for the next call.  No workgroup ever waits for another.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int BM = 128;           // activation rows per tile
constexpr int BN = 256;           // weight rows (output columns) per tile
constexpr int NT = 512;           // 8 waves
constexpr int A_ST = BM * 128;    // int8 activation tile per stage
constexpr int B_ST = BN * 64;     // packed weight tile per stage
constexpr int S_ST = 2048;        // sa (512 B) + sb (1024 B) + 512 B of the idle waves' loads
constexpr int STAGE = A_ST + B_ST + S_ST;
constexpr int DMA_PER_UNIT = 5;   // DMA instructions per wave per (tile, group) unit
constexpr int PART_FLOATS = NT * 64;   // one partial tile: 64 outputs per thread, [k][thread]

__device__ __forceinline__ uint32_t lds_addr(const unsigned char* l) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(lds_void*)l);
}
// global -> LDS, 16 (resp. 4) bytes per lane; lane i lands at m0 + 16*i (4*i).
__device__ __forceinline__ void dma16(const void* g, unsigned char* l) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr(l)) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, unsigned char* l) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr(l)) : "memory");
}
// Device-scope (sc1) 16-byte stores / loads of split-tile partials, the cache
// policy of agent-scope atomics: the stores write through the per-XCD L2 and
// are in memory once the writer's s_waitcnt has retired them, and the loads
// read the coherent copy.
typedef float v4f __attribute__((ext_vector_type(4)));
// Eight device-scope 16-byte stores (one every NT*4 floats) and the wait for
// them in one asm statement: store data VGPRs must not be overwritten before the
// stores have read them, which the compiler cannot know for asm stores.
__device__ __forceinline__ void store8_dev16(float* p, const v4f* v) {
    constexpr size_t S = (size_t)NT * 4;
    asm volatile(
        "global_store_dwordx4 %0, %8, off sc1\n\t"
        "global_store_dwordx4 %1, %9, off sc1\n\t"
        "global_store_dwordx4 %2, %10, off sc1\n\t"
        "global_store_dwordx4 %3, %11, off sc1\n\t"
        "global_store_dwordx4 %4, %12, off sc1\n\t"
        "global_store_dwordx4 %5, %13, off sc1\n\t"
        "global_store_dwordx4 %6, %14, off sc1\n\t"
        "global_store_dwordx4 %7, %15, off sc1\n\t"
        "s_waitcnt vmcnt(0) expcnt(0)"
        :
        : "v"(p), "v"(p + S), "v"(p + 2 * S), "v"(p + 3 * S), "v"(p + 4 * S), "v"(p + 5 * S), "v"(p + 6 * S),
          "v"(p + 7 * S), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "v"(v[4]), "v"(v[5]), "v"(v[6]), "v"(v[7])
        : "memory");
}
// Eight such loads (one every NT*4 floats) and the wait for them in a single asm
// statement, so the destination registers are not touched before they are valid.
__device__ __forceinline__ void load8_dev16(v4f* v, const float* p) {
    constexpr size_t S = (size_t)NT * 4;
    asm volatile(
        "global_load_dwordx4 %0, %8, off sc1\n\t"
        "global_load_dwordx4 %1, %9, off sc1\n\t"
        "global_load_dwordx4 %2, %10, off sc1\n\t"
        "global_load_dwordx4 %3, %11, off sc1\n\t"
        "global_load_dwordx4 %4, %12, off sc1\n\t"
        "global_load_dwordx4 %5, %13, off sc1\n\t"
        "global_load_dwordx4 %6, %14, off sc1\n\t"
        "global_load_dwordx4 %7, %15, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
        : "v"(p), "v"(p + S), "v"(p + 2 * S), "v"(p + 3 * S), "v"(p + 4 * S), "v"(p + 5 * S), "v"(p + 6 * S),
          "v"(p + 7 * S)
        : "memory");
}

struct Unit {
    int t, g, tm, tn;
    __device__ __forceinline__ int bm() const { return tm * BM; }
    __device__ __forceinline__ int bn() const { return tn * BN; }
    __device__ __forceinline__ void next(int NG, int ntm) {
        if (++g == NG) {
            g = 0;
            ++t;
            if (++tm == ntm) {
                tm = 0;
                ++tn;
            }
        }
    }
};

__device__ __forceinline__ Unit unit_of(int u, int NG, int ntm) {
    Unit x;
    x.t = u / NG;
    x.g = u - x.t * NG;
    x.tn = x.t / ntm;                 // consecutive tiles share their weight rows
    x.tm = x.t - x.tn * ntm;
    return x;
}

// The DMA of one unit: per wave 2 A instructions (8 rows x 128 B each), 2 B
// instructions (16 rows x 64 B each) and 1 scale instruction.  LDS layouts:
//   A  [128 rows][8 x 16 B], 16-byte chunk c of row r stored at c ^ (r & 7)
//   B  [256 rows][4 x 16 B] packed, chunk c of row r stored at c ^ ((r >> 1) & 3)
//   S  sa[128] f32, sb[256] f32
__device__ __forceinline__ void issue(unsigned char* st, const int8_t* __restrict__ A,
                                      const uint32_t* __restrict__ W, const float* __restrict__ sa,
                                      const float* __restrict__ sb, int M, int N, int K, const Unit& x,
                                      int w, int lane) {
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int i = 2 * w + t;
        const int r = 8 * i + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7);
        int gr = x.bm() + r;
        gr = gr < M ? gr : M - 1;
        dma16(A + (size_t)gr * K + (size_t)x.g * 128 + c * 16, st + i * 1024);
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int i = 2 * w + t;
        const int r = 16 * i + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 1) & 3);
        int gr = x.bn() + r;
        gr = gr < N ? gr : N - 1;
        dma16(reinterpret_cast<const unsigned char*>(W) + (size_t)gr * (K >> 1) + (size_t)x.g * 64 + c * 16,
              st + A_ST + i * 1024);
    }
    unsigned char* sdst = st + A_ST + B_ST;
    if (w < 2) {
        int r = x.bm() + w * 64 + lane;
        r = r < M ? r : M - 1;
        dma4(sa + (size_t)x.g * M + r, sdst + w * 256);
    } else {
        const int ww = (w - 2) & 3;   // waves 6, 7 repeat waves 2, 3 into the slack area
        int r = x.bn() + ww * 64 + lane;
        r = r < N ? r : N - 1;
        dma4(sb + (size_t)x.g * N + r, sdst + 512 + (w < 6 ? 0 : 1024) + ww * 256);
    }
}

// Which workgroup's share contains unit u (shares are [T*b/P, T*(b+1)/P)).
__device__ __forceinline__ int owner_of(long long u, long long T, int P) {
    return (int)(((u + 1) * P - 1) / T);
}

template <bool GSUM>
__global__ __launch_bounds__(NT, 1) void gemm_w4a8_k(const int8_t* __restrict__ A,
                                                     const uint32_t* __restrict__ W,
                                                     const float* __restrict__ sa,
                                                     const float* __restrict__ sb,
                                                     float* __restrict__ C,
                                                     int32_t* __restrict__ gsum,
                                                     float* __restrict__ part,
                                                     int* __restrict__ cnt, int M, int N, int K,
                                                     int ntm, long long T) {
    __shared__ __align__(16) unsigned char st0[STAGE];
    __shared__ __align__(16) unsigned char st1[STAGE];
    __shared__ __align__(16) unsigned char st2[STAGE];
    __shared__ __align__(16) unsigned char st3[STAGE];
    __shared__ int s_flag;
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6);
    const int wm = w & 1, wn = w >> 1;
    const int lr = lane & 31, lh = lane >> 5;
    const int NG = K >> 7;
    // Workgroups are dispatched to the 8 XCDs round-robin; renumber them so each
    // XCD owns one contiguous eighth of the units (its tiles share weight rows in
    // its own L2).  All share bookkeeping below uses this logical index.
    const int P = gridDim.x;
    const int b = (P % 8 == 0) ? (int)(blockIdx.x % 8) * (P / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const long long u0 = T * b / P, u1 = T * (b + 1) / P;
    const int n = (int)(u1 - u0);
    const int first_tile = (int)(u0 / NG);

    v16i facc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) facc[i][j][r] = 0;  // bits of +0.0f

    // two cursors: `cu` = unit being computed, `iu` = unit being loaded (3 ahead,
    // clamped to the last unit, whose loads are then simply repeated)
    Unit cu = unit_of((int)u0, NG, ntm);
    Unit iu = cu;
    issue(st0, A, W, sa, sb, M, N, K, iu, w, lane);
    if (1 < n) iu.next(NG, ntm);
    issue(st1, A, W, sa, sb, M, N, K, iu, w, lane);
    if (2 < n) iu.next(NG, ntm);
    issue(st2, A, W, sa, sb, M, N, K, iu, w, lane);
    const v16i zero16 = {};

    for (int i4 = 0; i4 < n; i4 += 4) {
#pragma unroll
        for (int sub = 0; sub < 4; sub++) {
            const int i = i4 + sub;
            if (i >= n) break;
            // the DMA of unit i has landed once at most the 3 younger units' loads are pending
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_UNIT) : "memory");
            __syncthreads();
            if (i + 3 < n) iu.next(NG, ntm);
            issue(sub == 0 ? st3 : sub == 1 ? st0 : sub == 2 ? st1 : st2, A, W, sa, sb, M, N, K, iu, w, lane);
            const unsigned char* cur = sub == 0 ? st0 : sub == 1 ? st1 : sub == 2 ? st2 : st3;
            const Unit x = cu;
            cu.next(NG, ntm);

            // --- group dot products: k-step ks = 2s+t, lane half lh covers codes
            //     [64s + 32lh + 16t, +16) of the group; one b128 of packed B per s
            v16i acc[2][2];
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                uint4 bp[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int r = 64 * wn + 32 * j + lr;
                    const int c = (2 * s2 + lh) ^ ((r >> 1) & 3);
                    bp[j] = *reinterpret_cast<const uint4*>(cur + A_ST + r * 64 + c * 16);
                }
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int ks = 2 * s2 + t;
                    v4i a[2], bb[2];
#pragma unroll
                    for (int ii = 0; ii < 2; ii++) {
                        const int r = 64 * wm + 32 * ii + lr;
                        const int c = (4 * s2 + 2 * lh + t) ^ (r & 7);
                        a[ii] = *reinterpret_cast<const v4i*>(cur + r * 128 + c * 16);
                    }
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const uint32_t x0 = t ? bp[j].z : bp[j].x, x1 = t ? bp[j].w : bp[j].y;
                        bb[j] = v4i{(int)even_x16(x0), (int)odd_x16(x0), (int)even_x16(x1), (int)odd_x16(x1)};
                    }
#pragma unroll
                    for (int ii = 0; ii < 2; ii++)
#pragma unroll
                        for (int j = 0; j < 2; j++)
                            acc[ii][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ii], bb[j],
                                                                               ks == 0 ? zero16 : acc[ii][j], 0, 0, 0);
                }
            }

            // --- fold: lane holds column 32j + lr, rows 8q + 4lh + e of tile (ii, j)
            const float* ls = reinterpret_cast<const float*>(cur + A_ST + B_ST);
            float sbv[2];
#pragma unroll
            for (int j = 0; j < 2; j++) sbv[j] = ls[128 + 64 * wn + 32 * j + lr];
#pragma unroll
            for (int ii = 0; ii < 2; ii++) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 v = *reinterpret_cast<const float4*>(ls + 64 * wm + 32 * ii + 8 * q + 4 * lh);
                    const float sv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int j = 0; j < 2; j++)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const int r = 4 * q + e;
                            const float f = __int_as_float(facc[ii][j][r]);
                            facc[ii][j][r] = __float_as_int(fmaf((float)acc[ii][j][r], sv[e] * sbv[j], f));
                        }
                }
            }
            if (GSUM) {
#pragma unroll
                for (int ii = 0; ii < 2; ii++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int nn = x.bn() + 64 * wn + 32 * j + lr;
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int m = x.bm() + 64 * wm + 32 * ii + 8 * (r >> 2) + 4 * lh + (r & 3);
                            if (m < M && nn < N) gsum[((size_t)m * N + nn) * NG + x.g] = acc[ii][j][r] >> 4;
                        }
                    }
            }

            // --- end of this workgroup's segment of tile x.t: publish it
            if (x.g == NG - 1 || i == n - 1) {
                const long long tb = (long long)x.t * NG, te = tb + NG;
                bool write_c = true;
                if (!(u0 <= tb && u1 >= te)) {
                    // split tile: partial -> workspace slot, last contributor combines
                    const int slot = (x.t == first_tile) ? 0 : 1;
                    // layout [slot][k/4][thread][4]: each store instruction writes 8 KB contiguous
                    float* my = part + ((size_t)b * 2 + slot) * PART_FLOATS + (size_t)threadIdx.x * 4;
                    v4f pv[16];
#pragma unroll
                    for (int ii = 0; ii < 2; ii++)
#pragma unroll
                        for (int j = 0; j < 2; j++)
#pragma unroll
                            for (int r4 = 0; r4 < 4; r4++)
                                pv[(ii * 2 + j) * 4 + r4] = v4f{
                                    __int_as_float(facc[ii][j][4 * r4]), __int_as_float(facc[ii][j][4 * r4 + 1]),
                                    __int_as_float(facc[ii][j][4 * r4 + 2]), __int_as_float(facc[ii][j][4 * r4 + 3])};
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // DMA still in flight counts too
                    store8_dev16(my, pv);
                    store8_dev16(my + (size_t)8 * NT * 4, pv + 8);
                    __syncthreads();
                    const int wf = owner_of(tb, T, P), wl = owner_of(te - 1, T, P);
                    if (threadIdx.x == 0)
                        s_flag = __hip_atomic_fetch_add(cnt + x.t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                                 wl - wf;
                    __syncthreads();
                    write_c = s_flag;
                    if (write_c) {
                        // sum the contributors' partials in workgroup order (deterministic)
#pragma unroll
                        for (int ii = 0; ii < 2; ii++)
#pragma unroll
                            for (int j = 0; j < 2; j++)
#pragma unroll
                                for (int r = 0; r < 16; r++) facc[ii][j][r] = 0;
                        for (int v = wf; v <= wl; v++) {
                            const int ft = (int)((T * v / P) / NG);
                            const float* pp = part + ((size_t)v * 2 + (ft == x.t ? 0 : 1)) * PART_FLOATS +
                                              (size_t)threadIdx.x * 4;
                            v4f pv[16];
                            load8_dev16(pv, pp);
                            load8_dev16(pv + 8, pp + (size_t)8 * NT * 4);
#pragma unroll
                            for (int ii = 0; ii < 2; ii++)
#pragma unroll
                                for (int j = 0; j < 2; j++)
#pragma unroll
                                    for (int r = 0; r < 16; r++) {
                                        const float f = __int_as_float(facc[ii][j][r]);
                                        facc[ii][j][r] = __float_as_int(f + pv[(ii * 2 + j) * 4 + (r >> 2)][r & 3]);
                                    }
                        }
                        if (threadIdx.x == 0)
                            __hip_atomic_store(cnt + x.t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
                if (write_c) {
#pragma unroll
                    for (int ii = 0; ii < 2; ii++)
#pragma unroll
                        for (int j = 0; j < 2; j++) {
                            const int nn = x.bn() + 64 * wn + 32 * j + lr;
                            if (nn < N)
#pragma unroll
                                for (int r = 0; r < 16; r++) {
                                    const int m = x.bm() + 64 * wm + 32 * ii + 8 * (r >> 2) + 4 * lh + (r & 3);
                                    if (m < M) C[(size_t)m * N + nn] = __int_as_float(facc[ii][j][r]) * 0.0625f;
                                }
                        }
                }
#pragma unroll
                for (int ii = 0; ii < 2; ii++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++) facc[ii][j][r] = 0;
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // drain the clamped tail DMA before exit
}

}  // namespace

GemmPlan gemm_plan(int M, int N, int K, int cus) {
    GemmPlan p;
    p.ntm = (M + BM - 1) / BM;
    p.ntn = (N + BN - 1) / BN;
    p.ntiles = p.ntm * p.ntn;
    p.T = (long long)p.ntiles * (K / kGroup);
    p.P = cus > 0 ? cus : 256;
    if (p.T < p.P) p.P = (int)p.T;
    p.part_bytes = (size_t)p.P * 2 * PART_FLOATS * sizeof(float);
    p.cnt_bytes = (size_t)p.ntiles * sizeof(int);
    return p;
}

hipError_t launch_gemm_w4a8(float* C, int32_t* gsum, const int8_t* A, const uint32_t* W,
                            const float* sa, const float* sb, int M, int N, int K, const GemmPlan& p,
                            float* part, int* cnt, hipStream_t st) {
    if (gsum)
        hipLaunchKernelGGL(gemm_w4a8_k<true>, dim3(p.P), dim3(NT), 0, st, A, W, sa, sb, C, gsum, part, cnt, M, N,
                           K, p.ntm, p.T);
    else
        hipLaunchKernelGGL(gemm_w4a8_k<false>, dim3(p.P), dim3(NT), 0, st, A, W, sa, sb, C, gsum, part, cnt, M,
                           N, K, p.ntm, p.T);
    return hipGetLastError();
}

// Zero the split-tile counters once, when their workspace is (re)allocated.
__global__ void zero_i32_k(int* p, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

hipError_t launch_zero_i32(int* p, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(zero_i32_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
    return hipGetLastError();
}

}  // namespace rt4
