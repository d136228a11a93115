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
// LDS with global_load_lds_dwordx4 (no VGPR round trip): four A+B stages and a
// ring of five scale slots, so unit i+4 is loading while unit i computes.  The
// LDS layouts are XOR-swizzled for gfx950's 64-bank LDS, which serves 16 lanes
// of a ds_read_b128 per cycle: any 16 consecutive fragment rows hit 16 distinct
// 16-byte bank groups.  The weights stay packed in LDS and are unpacked after
// the ds_read.  The DMA is issued from inline asm with a per-lane 32-bit offset
// (fixed while the tile is unchanged) and a scalar 64-bit base (advanced per
// group), so it costs no vector ALU work; the compiler does not see it, so it
// does not serialise LDS reads behind it -- the kernel waits itself (s_waitcnt
// vmcnt + barrier).
//
// Per unit each wave: unpacks the weight fragments of the unit (read during the
// previous unit), reads its second activation fragment, runs tiles (0,0) and
// (0,1), folds (0,0), passes the one barrier of the unit (DMA of unit i+1 landed,
// stage i free), issues the DMA of unit i+4 into stage i, reads the fragments of
// unit i+1, and runs tiles (1,0), (1,1) with the remaining folds in between.
// The fold (cvt + mul + fma per output per group) is most of the vector ALU
// work, and on gfx950 vector ALU and MFMA issue overlap only a little, so the
// kernel is bound by VALU + MFMA issue rather than by memory.
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
constexpr int AB_ST = A_ST + B_ST;    // one A+B stage
constexpr int NSC = 5;                // scale slots (a ring: unit i+4 is loaded while unit i folds)
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
//   A  [128 rows][8 x 16 B], 16-byte chunk c of row r stored at c ^ ((r >> 1) & 7)
//   B  [256 rows][4 x 16 B] packed, chunk c of row r stored at c ^ ((r >> 2) & 3)
//   S  sa[128] f32, sb[256] f32
// Per-lane byte offsets of this wave's DMA sources within one (tile, group) unit,
// relative to the unit's scalar bases; they change only when the tile changes.
struct DmaOff {
    uint32_t a[2], b[2], s;
};
__device__ __forceinline__ DmaOff dma_offsets(const Unit& x, int M, int N, int K, int w, int lane) {
    DmaOff o;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int i = 2 * w + t;
        const int r = 8 * i + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        int gr = x.bm() + r;
        gr = gr < M ? gr : M - 1;
        o.a[t] = (uint32_t)gr * (uint32_t)K + c * 16;
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int i = 2 * w + t;
        const int r = 16 * i + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        int gr = x.bn() + r;
        gr = gr < N ? gr : N - 1;
        o.b[t] = (uint32_t)gr * (uint32_t)(K >> 1) + c * 16;
    }
    if (w < 2) {
        int r = x.bm() + w * 64 + lane;
        o.s = (uint32_t)(r < M ? r : M - 1) * 4u;
    } else {
        int r = x.bn() + ((w - 2) & 3) * 64 + lane;
        o.s = (uint32_t)(r < N ? r : N - 1) * 4u;
    }
    return o;
}
__device__ __forceinline__ void dma16s(uint32_t voff, const void* base, unsigned char* l) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds_addr(l)) : "memory");
}
__device__ __forceinline__ void dma4s(uint32_t voff, const void* base, unsigned char* l) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds_addr(l)) : "memory");
}
__device__ __forceinline__ void issue(unsigned char* st, unsigned char* sdst, const int8_t* __restrict__ A,
                                      const uint32_t* __restrict__ W, const float* __restrict__ sa,
                                      const float* __restrict__ sb, int M, int N, int K, const Unit& x,
                                      const DmaOff& o, int w) {
    const int8_t* ab = A + (size_t)x.g * 128;
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(W) + (size_t)x.g * 64;
    dma16s(o.a[0], ab, st + (2 * w) * 1024);
    dma16s(o.a[1], ab, st + (2 * w + 1) * 1024);
    dma16s(o.b[0], wb, st + A_ST + (2 * w) * 1024);
    dma16s(o.b[1], wb, st + A_ST + (2 * w + 1) * 1024);
    if (w < 2)
        dma4s(o.s, sa + (size_t)x.g * M, sdst + w * 256);
    else
        dma4s(o.s, sb + (size_t)x.g * N, sdst + 512 + (w < 6 ? 0 : 1024) + ((w - 2) & 3) * 256);
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
    __shared__ __align__(16) unsigned char sab[4 * AB_ST];
    __shared__ __align__(16) unsigned char ssc[NSC * S_ST];
    __shared__ int s_flag;
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6);
    const int wm = w & 1, wn = w >> 1;
    const int lr = lane & 31, lh = lane >> 5;
    const int NG = K >> 7;
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
            for (int r = 0; r < 16; r++) facc[i][j][r] = 0;

    auto stage = [&](int i) { return sab + (i & 3) * AB_ST; };
    auto slot = [&](int i) { return ssc + (i % NSC) * S_ST; };
    auto read_a = [&](v4i (&dst)[4], const unsigned char* stg, int ii) {
        const int r = 64 * wm + 32 * ii + lr;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int c = (4 * (ks >> 1) + 2 * lh + (ks & 1)) ^ ((r >> 1) & 7);
            dst[ks] = *reinterpret_cast<const v4i*>(stg + r * 128 + c * 16);
        }
    };
    auto read_b = [&](uint4 (&dst)[2][2], const unsigned char* stg) {
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                const int r = 64 * wn + 32 * j + lr;
                const int c = (2 * s2 + lh) ^ ((r >> 2) & 3);
                dst[j][s2] = *reinterpret_cast<const uint4*>(stg + A_ST + r * 64 + c * 16);
            }
    };
    const v16i zero16 = {};
    auto mma = [&](v16i& acc, const v4i (&a)[4], const v4i (&bb)[4]) {
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0], bb[0], zero16, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[1], bb[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[2], bb[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[3], bb[3], acc, 0, 0, 0);
    };
    // fold of tile (ii, j): lane holds column 32j + lr, rows 8q + 4lh + e
    auto fold = [&](v16i& fa, const v16i& acc, const float* ls, int ii, int j, const Unit& x) {
        const float sbv = ls[128 + 64 * wn + 32 * j + lr];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 v = *reinterpret_cast<const float4*>(ls + 64 * wm + 32 * ii + 8 * q + 4 * lh);
            const float sv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int r = 4 * q + e;
                fa[r] = __float_as_int(fmaf((float)acc[r], sv[e] * sbv, __int_as_float(fa[r])));
            }
        }
        if (GSUM) {
            const int nn = x.bn() + 64 * wn + 32 * j + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = x.bm() + 64 * wm + 32 * ii + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M && nn < N) gsum[((size_t)m * N + nn) * NG + x.g] = acc[r] >> 4;
            }
        }
    };

    // prologue: DMA of units 0..3 (clamped to the last unit), then fragments of unit 0
    Unit cu = unit_of((int)u0, NG, ntm);
    Unit iu = cu;
    DmaOff off = dma_offsets(iu, M, N, K, w, lane);
    auto advance = [&]() {
        iu.next(NG, ntm);
        if (iu.g == 0) off = dma_offsets(iu, M, N, K, w, lane);
    };
#pragma unroll
    for (int s = 0; s < 4; s++) {
        if (s > 0 && s < n) advance();
        issue(stage(s), slot(s), A, W, sa, sb, M, N, K, iu, off, w);
    }
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * DMA_PER_UNIT) : "memory");
    __syncthreads();
    v4i a0[4], a1[4];
    uint4 bp[2][2];
    read_a(a0, stage(0), 0);
    read_b(bp, stage(0));

    bool flushed = false;
    for (int i = 0; i < n; i++) {
        const Unit x = cu;
        cu.next(NG, ntm);
        const float* ls = reinterpret_cast<const float*>(slot(i));
        v4i bu[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const uint4 p = bp[j][ks >> 1];
                const uint32_t x0 = (ks & 1) ? p.z : p.x, x1 = (ks & 1) ? p.w : p.y;
                bu[j][ks] = v4i{(int)even_x16(x0), (int)odd_x16(x0), (int)even_x16(x1), (int)odd_x16(x1)};
            }
        read_a(a1, stage(i), 1);
        v16i accA, accB;
        mma(accA, a0, bu[0]);                       // tile (0,0)
        mma(accB, a0, bu[1]);                       // tile (0,1)
        fold(facc[0][0], accA, ls, 0, 0, x);
        // the DMA of unit i+1 has landed once at most the 2 younger units' loads are pending;
        // every wave has finished reading stage i (its LDS reads retire before the barrier).
        // After a flush the C stores of the previous tile are younger than that DMA and
        // their number depends on how many rows and columns of the tile exist (stores to
        // absent ones are never issued), so no count bound is safe: drain everything.
        if (flushed) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_UNIT) : "memory");
        flushed = false;
        __syncthreads();
        if (i + 4 < n) advance();
        issue(stage(i), slot(i + 4), A, W, sa, sb, M, N, K, iu, off, w);
        read_a(a0, stage(i + 1), 0);
        read_b(bp, stage(i + 1));
        mma(accA, a1, bu[0]);                       // tile (1,0)
        fold(facc[0][1], accB, ls, 0, 1, x);
        mma(accB, a1, bu[1]);                       // tile (1,1)
        fold(facc[1][0], accA, ls, 1, 0, x);
        fold(facc[1][1], accB, ls, 1, 1, x);

        // --- end of this workgroup's segment of tile x.t: publish it
        if (x.g == NG - 1 || i == n - 1) {
            flushed = true;
            const long long tb = (long long)x.t * NG, te = tb + NG;
            bool write_c = true;
            if (!(u0 <= tb && u1 >= te)) {
                const int slt = (x.t == first_tile) ? 0 : 1;
                float* my = part + ((size_t)b * 2 + slt) * PART_FLOATS + (size_t)threadIdx.x * 4;
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
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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
                        v4f pv2[16];
                        load8_dev16(pv2, pp);
                        load8_dev16(pv2 + 8, pp + (size_t)8 * NT * 4);
#pragma unroll
                        for (int ii = 0; ii < 2; ii++)
#pragma unroll
                            for (int j = 0; j < 2; j++)
#pragma unroll
                                for (int r = 0; r < 16; r++) {
                                    const float f = __int_as_float(facc[ii][j][r]);
                                    facc[ii][j][r] = __float_as_int(f + pv2[(ii * 2 + j) * 4 + (r >> 2)][r & 3]);
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
