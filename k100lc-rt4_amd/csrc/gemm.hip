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
// Tiling.  Workgroup tile 128 activation rows x 256 weight rows, 8 waves; wave w
// owns weight rows (output columns) 32w..32w+31 and all 128 activation rows, i.e.
// four 32 x 32 row tiles sharing one weight fragment, so each wave unpacks only
// its own 32 weight rows.  One 128-wide K group ("unit" = one tile x one group)
// is four MFMA k-steps per row tile.  The int32 accumulators restart at every
// group and are folded into fp32:
//     facc += f32(acc) * S,   S = sa * sb,   acc = 16*I exactly (x16 nibble unpack),
// and the result is scaled by 1/16 once at the end (a power of two, so the bits
// equal those of scaling every term).  S is formed on the matrix core: one
// two-block fp32 outer product (v_mfma_f32_32x32x1_2b_f32) per pair of row tiles
// gives sa (x) sb for both in the accumulator layout of the int8 tiles (block b:
// the activation scales of row tile 2p + b from lanes 32b..32b+31, the weight
// scale of the lane's column in both halves).  Every element is one fp32
// product, so S is sa * sb correctly rounded, as the reference forms it
// (kernels/gemm_core.h:183).  Against four bf16 MFMAs on exact 3-part splits of
// both scales (the earlier form, within a few ulp) it drops the split work of
// every wave and one LDS pass per unit: C2 gate/up 143 -> 139 us, measured.
//
// What bounds this kernel on gfx950 is instruction issue: measured, a SIMD with
// two such waves issues about one instruction per 4 cycles whatever its kind
// (scalar, vector, LDS; an int8 MFMA takes about 16), with little overlap
// between the two waves, and the fold alone is two vector instructions per
// output per group (128 per wave per unit against 16 MFMAs).  So the
// loop is built for few instructions: every LDS read address is a per-lane
// register (moved on by one stage per unit, one add per register) plus the row
// tile as an immediate offset (a body unrolled over the four stages, which would
// make the stage an immediate too, spilled around the flush); the DMA
// sources are the kernel's scalar base pointers plus per-lane 32-bit offsets,
// moved on by one group per unit (advancing the scalar bases instead measured
// the same); tile bookkeeping is a few scalar counters.  The MFMAs of a row tile are interleaved one by one with the
// fold of the previous row tile (and with the unpack of the next k-step), in an
// order the compiler may not change (sched_barrier; every folded value also
// passes through an empty asm statement where it is formed, without which the
// compiler sinks three of the four folds of a unit past the barrier into one
// block and spills), so the matrix core and the vector ALU work at the same
// time and no fold waits for the MFMA just issued.
//
// Data movement.  Per unit the workgroup moves 16 KB of int8 activations, 16 KB
// of packed weights and the two scale vectors from global memory straight into
// LDS with global_load_lds_dwordx4 (no VGPR round trip), four stages deep (the
// unit three ahead is loading while a unit computes).  Each wave loads exactly
// the weight rows it reads; the activation tile is shared by all waves (one
// barrier per unit).  LDS layouts are XOR-swizzled for gfx950's 64-bank LDS: any
// 16 consecutive fragment rows of a ds_read_b128 hit 16 distinct 16-byte bank
// groups.
//
// Scheduling ("stream-K").  One persistent workgroup per CU takes an equal,
// contiguous share of the (tile, group) units, numbered so each XCD owns a
// contiguous slice.  A tile split between workgroups is combined
// deterministically: every contributor except the last writes its fp32 partial
// to a workspace slot (agent-coherent stores), bumps the tile's counter, and the
// contributor that arrives last sums all partials in workgroup order and writes
// C; it also resets the counter for the next call.  No workgroup ever waits for
// another.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {
namespace {

typedef __attribute__((address_space(3))) void lds_void;
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int BM = 128;           // activation rows per tile
constexpr int BN = 256;           // weight rows (output columns) per tile
constexpr int NT = 512;           // 8 waves
constexpr int NS = 4;             // LDS stages
constexpr int A_ST = BM * 128;    // int8 activation tile per stage
constexpr int B_ST = BN * 64;     // packed weight tile per stage
constexpr int S_ST = 2048;        // sa (512 B) + sb (1024 B) + 512 B written by the two idle waves
constexpr int LDS_B = 0;                       // weight stages
constexpr int LDS_A = LDS_B + NS * B_ST;       // activation stages
constexpr int LDS_S = LDS_A + NS * A_ST;       // scale stages
constexpr int LDS_FLAG = LDS_S + NS * S_ST;
constexpr int LDS_META = LDS_FLAG + 16;            // split-tile metadata (10 ints)
constexpr int LDS_BYTES = LDS_META + 48;
constexpr int DMA_PER_UNIT = 5;   // DMA instructions per wave per unit
constexpr int PART_FLOATS = NT * 64;   // one partial tile: 64 outputs per thread, [k][thread]

// Device-scope (sc1) 16-byte stores / loads of split-tile partials, the cache
// policy of agent-scope atomics: the stores write through the per-XCD L2 and
// are in memory once the writer's s_waitcnt has retired them, and the loads
// read the coherent copy.  Four at a time (one row tile's 16 values per lane,
// at a stride of NT*4 floats), each with its wait in the same asm statement:
// store data registers must not be overwritten before the stores have read them,
// and loaded registers must not be touched before they are valid, neither of
// which the compiler can know for asm memory operations.
__device__ __forceinline__ void store4_dev16(float* p, const v16i& f) {
    constexpr size_t S = (size_t)NT * 4;
    const v4i v0 = __builtin_shufflevector(f, f, 0, 1, 2, 3), v1 = __builtin_shufflevector(f, f, 4, 5, 6, 7);
    const v4i v2 = __builtin_shufflevector(f, f, 8, 9, 10, 11), v3 = __builtin_shufflevector(f, f, 12, 13, 14, 15);
    asm volatile(
        "global_store_dwordx4 %0, %4, off sc1\n\t"
        "global_store_dwordx4 %1, %5, off sc1\n\t"
        "global_store_dwordx4 %2, %6, off sc1\n\t"
        "global_store_dwordx4 %3, %7, off sc1\n\t"
        "s_waitcnt vmcnt(0) expcnt(0)"
        :
        : "v"(p), "v"(p + S), "v"(p + 2 * S), "v"(p + 3 * S), "v"(v0), "v"(v1), "v"(v2), "v"(v3)
        : "memory");
}
__device__ __forceinline__ void add4_dev16(v16i& f, const float* p) {
    constexpr size_t S = (size_t)NT * 4;
    v4f v0, v1, v2, v3;
    asm volatile(
        "global_load_dwordx4 %0, %4, off sc1\n\t"
        "global_load_dwordx4 %1, %5, off sc1\n\t"
        "global_load_dwordx4 %2, %6, off sc1\n\t"
        "global_load_dwordx4 %3, %7, off sc1\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&v"(v0), "=&v"(v1), "=&v"(v2), "=&v"(v3)
        : "v"(p), "v"(p + S), "v"(p + 2 * S), "v"(p + 3 * S)
        : "memory");
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = __float_as_int(__int_as_float(f[e]) + v0[e]);
        f[4 + e] = __float_as_int(__int_as_float(f[4 + e]) + v1[e]);
        f[8 + e] = __float_as_int(__int_as_float(f[8 + e]) + v2[e]);
        f[12 + e] = __float_as_int(__int_as_float(f[12 + e]) + v3[e]);
    }
}

// Per-lane byte offsets of this wave's DMA sources for one tile (relative to the
// unit's scalar bases), unchanged while the tile is.  LDS layouts:
//   A  [128 rows][8 x 16 B], 16-byte chunk c of row r stored at c ^ ((r >> 1) & 7);
//      wave w loads rows 16w..16w+15 (two instructions of 8 rows x 128 B)
//   B  [256 rows][4 x 16 B] packed, chunk c of row r stored at c ^ ((r >> 2) & 3);
//      wave w loads rows 32w..32w+31, the ones it reads
//   S  sa[128] f32 (waves 0, 1), sb[256] f32 (waves 2..5); waves 6, 7 repeat an sb
//      load into the spare 512 B so that every wave issues the same count.
struct DmaOff {
    uint32_t a[2], b[2], s;
};
__device__ __forceinline__ DmaOff dma_offsets(int bm, int bn, int M, int N, int K, int w, int lane) {
    DmaOff o;
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int r = 16 * w + 8 * t + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int gr = min(bm + r, M - 1);
        o.a[t] = (uint32_t)gr * (uint32_t)K + c * 16;
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int r = 32 * w + 16 * t + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        const int gr = min(bn + r, N - 1);
        o.b[t] = (uint32_t)gr * (uint32_t)(K >> 1) + c * 16;
    }
    if (w < 2)
        o.s = (uint32_t)min(bm + 64 * w + lane, M - 1) * 4u;
    else
        o.s = (uint32_t)min(bn + 64 * ((w - 2) & 3) + lane, N - 1) * 4u;
    return o;
}

// Which workgroup's share contains unit u (shares are [T*b/P, T*(b+1)/P)).
__device__ __forceinline__ int owner_of(long long u, long long T, int P) {
    return (int)(((u + 1) * P - 1) / T);
}

// Tile coordinates of a unit, as the flush and the group-sum stores need them.
struct TileRef {
    int t, bm, bn, g;
};

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
    __shared__ __align__(16) unsigned char lds[LDS_BYTES];
    int* s_flag = reinterpret_cast<int*>(lds + LDS_FLAG);
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6);
    const int lr = lane & 31, lh = lane >> 5;
    const int NG = K >> 7;
    const int P = gridDim.x;
    const int b = (P % 8 == 0) ? (int)(blockIdx.x % 8) * (P / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const long long u0 = T * b / P, u1 = T * (b + 1) / P;
    const int n = (int)(u1 - u0);
    const int first_tile = (int)(u0 / NG);

    // per-lane LDS read offsets into the current stage (next_stage moves them on);
    // the row tile is an immediate
    int ra[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) ra[ks] = LDS_A + lr * 128 + (((4 * (ks >> 1) + 2 * lh + (ks & 1)) ^ ((lr >> 1) & 7)) * 16);
    int rb[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
        const int r = 32 * w + lr;
        rb[s2] = LDS_B + r * 64 + (((2 * s2 + lh) ^ ((r >> 2) & 3)) * 16);
    }
    // sa of row 64p + lane (row tile 2p in lanes 0..31, 2p + 1 in lanes 32..63) at
    // rsa + 256p; sb of this lane's column at rsb
    int rsa = LDS_S + lane * 4, rsb = LDS_S + 512 + (32 * w + lr) * 4;
    // per-wave LDS destinations of the DMA (m0 = base + stage immediate)
    const uint32_t L = lds_addr(lds);
    const uint32_t dstA = L + LDS_A + 2 * w * 1024, dstB = L + LDS_B + 2 * w * 1024;
    const uint32_t dstS = L + LDS_S + (w < 2 ? w * 256 : w < 6 ? 512 + (w - 2) * 256 : 1536);

    // facc[ii]: row tile ii (rows 32 ii..32 ii+31) x this wave's 32 columns; lane (lr, lh)
    // holds column 32w + lr, rows 32 ii + 8q + 4lh + e in register 4q + e.
    v16i facc[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) facc[i][r] = 0;

    const v16i zero16 = {};
    const v32f zero32f = {};
    auto unpack_ks = [&](v4i (&bu_)[4], const uint4 (&bp_)[2], int ks) {
        const uint4 p = bp_[ks >> 1];
        const uint32_t x0 = (ks & 1) ? p.z : p.x, x1 = (ks & 1) ? p.w : p.y;
        bu_[ks] = v4i{(int)even_x16(x0), (int)odd_x16(x0), (int)even_x16(x1), (int)odd_x16(x1)};
    };
    // Scale products of row tiles 2p and 2p + 1: the two-block outer product
    // (v_mfma_f32_32x32x1_2b_f32; block b takes its rows from lanes 32b..32b+31 and
    // its columns from the same lanes) of sa[64p + lane] and sb[this lane's column]
    // puts sa[row of register r] * sb[column] of tile 2p + b in register 16b + r,
    // the accumulator layout of the int8 tiles.
    auto scales2 = [&](float sa_pair, float sb_col) __attribute__((always_inline)) -> v32f {
        return __builtin_amdgcn_mfma_f32_32x32x1f32(sa_pair, sb_col, zero32f, 0, 0, 0);
    };
    auto slo = [](const v32f& v) __attribute__((always_inline)) -> v16f {
        return __builtin_shufflevector(v, v, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
    };
    auto shi = [](const v32f& v) __attribute__((always_inline)) -> v16f {
        return __builtin_shufflevector(v, v, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31);
    };
    // quarter q of the fold of row tile ii (registers 4q..4q+3)
    auto fold_q = [&](v16i& fa, const v16i& acc, const v16f& S, int ii, int q, const TileRef& x) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 4 * q; r < 4 * q + 4; r++) {
            int v = __float_as_int(fmaf((float)acc[r], S[r], __int_as_float(fa[r])));
            asm volatile("" : "+v"(v));   // formed here, not sunk past the next MFMAs
            fa[r] = v;
        }
        if (GSUM && x.g >= 0) {
            const int nn = x.bn + 32 * w + lr;
#pragma unroll
            for (int r = 4 * q; r < 4 * q + 4; r++) {
                const int m = x.bm + 32 * ii + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (m < M && nn < N) gsum[((size_t)m * N + nn) * NG + x.g] = acc[r] >> 4;
            }
        }
    };

    // End of this workgroup's segment of tile x.t: publish it (see the file comment).
    // Split-tile metadata of this workgroup's first and last tile (only these can be
    // shared with other workgroups), formed once here so that the flush, which runs
    // amid the pipeline's live registers, needs no 64-bit arithmetic:
    //   [0] first tile, [1] whole, [2] owner of its first unit, [3] owner of its last
    //   unit, [4] partial slot of that first owner; [5..9] the same for the last tile.
    // A contributor v writes its partial of tile t to slot 2v (t is v's first tile) or
    // 2v + 1 (its last tile).  Every contributor after the first owner starts its
    // share inside t, so t is its first tile; the first owner's slot is 0 only if its
    // share starts exactly at the tile's first unit.
    int* meta = reinterpret_cast<int*>(lds + LDS_META);
    if (threadIdx.x == 0) {
        const long long tl = (u1 - 1) / NG;
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const long long t = e ? tl : (long long)first_tile;
            const long long tb = t * NG, te = tb + NG;
            const int wf = owner_of(tb, T, P), wl = owner_of(te - 1, T, P);
            meta[5 * e + 0] = (int)t;
            meta[5 * e + 1] = (u0 <= tb && u1 >= te);
            meta[5 * e + 2] = wf;
            meta[5 * e + 3] = wl;
            meta[5 * e + 4] = (T * wf / P == tb) ? 0 : 1;
        }
    }

    // End of this workgroup's segment of tile x.t: publish it (see the file comment).
    auto flush = [&](const TileRef& x) __attribute__((always_inline)) {
        // only the first and the last tile of a share can be split; tiles between are whole
        const int tf = uniform(meta[0]), tl = uniform(meta[5]);
        const int e = x.t == tf ? 0 : 5;
        const bool whole = (x.t != tf && x.t != tl) || uniform(meta[e + 1]);
        bool write_c = true;
        if (!whole) {
            const int wf = uniform(meta[e + 2]), wl = uniform(meta[e + 3]), slot_f = uniform(meta[e + 4]);
            float* my = part + ((size_t)b * 2 + (e ? 1 : 0)) * PART_FLOATS + (size_t)threadIdx.x * 4;
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
            for (int ii = 0; ii < 4; ii++) store4_dev16(my + (size_t)ii * 4 * NT * 4, facc[ii]);
            __syncthreads();
            if (threadIdx.x == 0)
                *s_flag = __hip_atomic_fetch_add(cnt + x.t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == wl - wf;
            __syncthreads();
            write_c = *s_flag;
            if (write_c) {
#pragma unroll
                for (int ii = 0; ii < 4; ii++)
#pragma unroll
                    for (int r = 0; r < 16; r++) facc[ii][r] = 0;
                for (int v = wf; v <= wl; v++) {
                    const int slot = 2 * v + (v == wf ? slot_f : 0);
                    const float* pp = part + (size_t)slot * PART_FLOATS + (size_t)threadIdx.x * 4;
#pragma unroll
                    for (int ii = 0; ii < 4; ii++) add4_dev16(facc[ii], pp + (size_t)ii * 4 * NT * 4);
                }
                if (threadIdx.x == 0) __hip_atomic_store(cnt + x.t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (write_c) {
            // N passes through an empty asm: the row offsets below are then formed here,
            // in this rare path, instead of being hoisted out of the loops into registers
            // held for the whole kernel.
            int Nv = N;
            asm volatile("" : "+s"(Nv));
            const uint32_t nn = (uint32_t)(x.bn + 32 * w + lr);
            float* cb = C + (size_t)x.bm * Nv + nn;
            const int mrows = M - x.bm;
            if (nn < (uint32_t)N) {
                if (mrows >= BM) {
#pragma unroll
                    for (int ii = 0; ii < 4; ii++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int ml = 32 * ii + 8 * (r >> 2) + 4 * lh + (r & 3);
                            cb[(size_t)ml * Nv] = __int_as_float(facc[ii][r]) * 0.0625f;
                            __builtin_amdgcn_sched_barrier(0);   // one address at a time
                        }
                } else {
#pragma unroll
                    for (int ii = 0; ii < 4; ii++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int ml = 32 * ii + 8 * (r >> 2) + 4 * lh + (r & 3);
                            if (ml < mrows) cb[(size_t)ml * Nv] = __int_as_float(facc[ii][r]) * 0.0625f;
                            __builtin_amdgcn_sched_barrier(0);
                        }
                }
            }
        }
#pragma unroll
        for (int ii = 0; ii < 4; ii++)
#pragma unroll
            for (int r = 0; r < 16; r++) facc[ii][r] = 0;
    };

    // ---- DMA side: the unit being loaded.  Its sources are the kernel arguments
    // (scalar bases) plus per-lane 32-bit offsets that hold the row, the chunk and
    // the group: each unit adds one group to them, a new tile recomputes them.
    int dleft, dtm, dtn, dg0;
    {
        const int t0 = (int)(u0 / NG);
        dg0 = (int)(u0 - (long long)t0 * NG);
        dleft = NG - dg0;
        dtn = t0 / ntm;
        dtm = t0 - dtn * ntm;
    }
    const void* sbase = (w < 2 ? (const void*)sa : (const void*)sb);
    const uint32_t s_step = (w < 2 ? (uint32_t)M : (uint32_t)N) * 4u;
    DmaOff off = dma_offsets(dtm * BM, dtn * BN, M, N, K, w, lane);
    // the group moves the (scalar) source bases; the per-lane offsets change per tile
    const char* bA = reinterpret_cast<const char*>(A) + (size_t)dg0 * 128;
    const char* bW = reinterpret_cast<const char*>(W) + (size_t)dg0 * 64;
    const char* bS = reinterpret_cast<const char*>(sbase) + (size_t)dg0 * s_step;
    // DMA of the unit at the DMA side's position into stage st
    auto issue = [&](int st) __attribute__((always_inline)) {
        const uint32_t da = dstA + st * A_ST, db = dstB + st * B_ST, ds = dstS + st * S_ST;
        dma16<0>(off.a[0], bA, da);
        dma16<1024>(off.a[1], bA, da);
        dma16<0>(off.b[0], bW, db);
        dma16<1024>(off.b[1], bW, db);
        dma4<0>(off.s, bS, ds);
    };
    auto advance_dma = [&]() __attribute__((always_inline)) {
        if (--dleft == 0) {
            dleft = NG;
            if (++dtm == ntm) {
                dtm = 0;
                ++dtn;
            }
            off = dma_offsets(dtm * BM, dtn * BN, M, N, K, w, lane);
            bA = reinterpret_cast<const char*>(A);
            bW = reinterpret_cast<const char*>(W);
            bS = reinterpret_cast<const char*>(sbase);
        } else {
            bA += 128;
            bW += 64;
            bS += s_step;
        }
    };

    // ---- compute side: the tile of the current segment of units
    TileRef cur;
    {
        const int t0 = (int)(u0 / NG);
        cur.t = t0;
        cur.g = (int)(u0 - (long long)t0 * NG);
        const int tn = t0 / ntm;
        cur.bm = (t0 - tn * ntm) * BM;
        cur.bn = tn * BN;
    }

    // prologue: DMA of units 0..3, then the fragments of unit 0
    issue(0);
    if (n > 1) { advance_dma(); issue(1); }
    if (n > 2) { advance_dma(); issue(2); }
    if (n > 3) { advance_dma(); issue(3); }
    if (n > 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * DMA_PER_UNIT) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    v4i a_cur[4], a_nxt[4], bu[4];
    uint4 bp[2];
    // fragment reads: per-lane offsets into the current stage (moved on by one stage
    // per unit: one add per register) plus the row tile (an immediate).  The adds
    // are asm with the register tied in place: written in C, the compiler kept the
    // old and the new offsets alive together and spent 17 adds and 4 moves per
    // unit on the 8 updates (C2 gate/up 139 -> 138 us with them in place).
    auto next_stage = [&](int st_next) __attribute__((always_inline)) {
        const int da = st_next ? A_ST : -(NS - 1) * A_ST, db = st_next ? B_ST : -(NS - 1) * B_ST;
        const int ds = st_next ? S_ST : -(NS - 1) * S_ST;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) asm volatile("v_add_u32 %0, %1, %0" : "+v"(ra[ks]) : "s"(da));
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) asm volatile("v_add_u32 %0, %1, %0" : "+v"(rb[s2]) : "s"(db));
        asm volatile("v_add_u32 %0, %1, %0" : "+v"(rsa) : "s"(ds));
        asm volatile("v_add_u32 %0, %1, %0" : "+v"(rsb) : "s"(ds));
    };
    auto read_a = [&](v4i (&dst)[4], int ii) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) dst[ks] = *reinterpret_cast<const v4i*>(lds + ra[ks] + ii * 4096);
    };
    auto read_b = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++) bp[s2] = *reinterpret_cast<const uint4*>(lds + rb[s2]);
    };
    // the scale operands of a unit, read once its stage is valid (right after the
    // unit's barrier): sb of this wave's column and sa of the two row-tile pairs
    float sa2[2];
    float sbr;
    auto read_s = [&]() __attribute__((always_inline)) {
        sbr = *reinterpret_cast<const float*>(lds + rsb);
        sa2[0] = *reinterpret_cast<const float*>(lds + rsa);
        sa2[1] = *reinterpret_cast<const float*>(lds + rsa + 256);
    };
    read_a(a_cur, 0);
    read_b();
    read_s();

    // Software pipeline over row tiles: the MFMAs of row tile t run while tile t-1
    // is folded.  The last tile of a unit is folded during the first tile of the
    // next unit of the same segment; at the end of a segment it is folded there and
    // the segment is published.
    // Accumulators with fixed roles: row tiles 0 and 2 of a unit go to accA, tiles
    // 1 and 3 to accB, and a fold reads the one the MFMAs are not writing (no copies).
    v16i accA, accB;
    // Scale products: one buffer of two row tiles, (0, 1) from after row tile 0's
    // MFMAs (until then it holds tiles 2 and 3 of the previous unit, the last of which
    // is folded during row tile 0), (2, 3) from before the unit's barrier.
    v32f S2;
    // One row-tile step: the four MFMAs of tile (a, bu) into acc, each followed by a
    // quarter of the fold of the previous tile (prev into facc[fi], with its scale
    // products S, formed one row tile earlier) and, with UNPACK, by the unpack of
    // the next k-step's weights.
    auto step = [&](const v4i (&a)[4], v16i& acc, const v16i& prev, v16i& fa, int fi, const TileRef& fx,
                    bool do_unpack, const v16f& S) __attribute__((always_inline)) {
        if (do_unpack) unpack_ks(bu, bp, 0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[ks], bu[ks], ks ? acc : zero16, 0, 0, 0);
            if (do_unpack && ks < 3) unpack_ks(bu, bp, ks + 1);
            fold_q(fa, prev, S, fi, ks, fx);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // One unit (one group of the current tile) from stage st; `first`: no earlier
    // unit of this segment, so there is no row tile 3 awaiting its fold.
    int i = 0;
    auto unit = [&](bool first) __attribute__((always_inline)) {
        const int st = i & (NS - 1);
        TileRef x = cur;
        TileRef xprev = cur;
        if (GSUM) xprev.g = first ? -1 : cur.g - 1;   // -1: nothing to store
        // row tile 0, with the unpack of this unit's weights and the fold of the
        // previous unit's last tile
        read_a(a_nxt, 1);
        // (for the first unit of a segment accB and S2 are zero: the fold adds exact zeros)
        step(a_cur, accA, accB, facc[3], 3, xprev, true, shi(S2));
        S2 = scales2(sa2[0], sbr);
        // row tile 1, fold of tile 0
        read_a(a_cur, 2);
        step(a_nxt, accB, accA, facc[0], 0, x, false, slo(S2));
        // row tile 2, fold of tile 1
        read_a(a_nxt, 3);
        step(a_cur, accA, accB, facc[1], 1, x, false, shi(S2));
        S2 = scales2(sa2[1], sbr);   // before the barrier: sa2, sbr are refilled with the next unit's after it
        // row tile 3.  The DMA of unit i+1 has landed once at most the two younger
        // units' loads are pending (three units in flight), and every wave has issued
        // its last read of this stage (the barrier waits for LDS reads).  Near the
        // end of the share fewer units are in flight; the first unit of a segment
        // follows a flush, whose C stores are younger than that DMA and whose number
        // depends on how many rows and columns of the tile exist; the group-sum
        // variant stores as it goes.  In those cases no count bound is safe: drain.
        if (GSUM || first || i + 3 >= n) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_UNIT) : "memory");
        __syncthreads();
        if (i + 4 < n) {
            advance_dma();
            issue(st);
        }
        next_stage((st + 1) & (NS - 1));
        read_b();
        read_a(a_cur, 0);
        read_s();
        step(a_nxt, accB, accA, facc[2], 2, x, false, slo(S2));
        ++i;
        if (GSUM) ++cur.g;
    };
    // segments: the units of one tile within this workgroup's share
    while (i < n) {
        const int g0 = (int)((u0 + i) % NG);
        const int len = min(NG - g0, n - i);
        if (GSUM) cur.g = g0;
        accB = zero16;
        S2 = zero32f;
        for (int k = 0; k < len; k++) unit(k == 0);
        // the segment's last row tile 3, then publish the segment
        TileRef xl = cur;
        if (GSUM) xl.g = cur.g - 1;
#pragma unroll
        for (int q = 0; q < 4; q++) fold_q(facc[3], accB, shi(S2), 3, q, xl);
        flush(cur);
        // the next unit's fragments, read again from its stage (still intact): the
        // copies read during the last unit are then dead across the flush, which
        // leaves the flush the registers it needs
        read_b();
        read_a(a_cur, 0);
        read_s();
        // next tile
        ++cur.t;
        cur.bm += BM;
        if (cur.bm >= ntm * BM) {
            cur.bm = 0;
            cur.bn += BN;
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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
