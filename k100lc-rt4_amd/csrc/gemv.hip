// gemv.hip -- RT4 W4A8 decode GEMV for M = 1..4 rows on gfx950 matrix cores.
//
//   y[m][n] = Σ_g f16(ws[n][g]) * sa[m][g] * I[m][n][g],
//   I[m][n][g] = Σ_{k in group g} code[n][k] * xq[m][k]      (exact int32)
//
// Restates gemv_w4a8 (kernels/gemv_w4a8_core.h:76-209) as called by k_gemv_w4a8
// (src/k_gemv.hip:53-106), redesigned for CDNA4.  The kernel is a weight stream:
// 44.5 MB per 27B MLP matrix against a few KB of activations, so its layout is
// chosen for the memory system first.
//
// * Work split: a workgroup owns one tile of RB x 16 weight rows; its W waves
//   split the K groups of that tile, GPW groups (an even number) each.  Every
//   wave issues all of its loads up front.  With RB = 2 a wave multiplies one
//   activation operand into two 16-row blocks, which halves the activation
//   reloads per weight byte; it pays where the tile count is many times the CU
//   count (the LM head), and loses where the grid would be only a few tiles per
//   CU (load imbalance in the last round).
// * Weight loads: one dwordx4 load instruction covers 8 rows x 128 B, i.e. 8
//   whole cache lines (two 128-element groups of 8 rows).  A 16-row MFMA tile
//   would otherwise read 16 half lines per instruction, which measured ~25%
//   slower on gfx950.  Two such loads (rows 0-7 and 8-15 of a group pair) are
//   arranged so that the MFMA operand of the first group is a per-lane select of
//   the two and that of the second group is the other select rotated by 8 lanes
//   (DPP row_ror:8) -- no LDS round trip.
// * Group dot products: v_mfma_i32_16x16x64_i8 with B = 16 weight rows and A =
//   the activation rows (rows M..15 of A are don't-care; their outputs are
//   dropped).  Two MFMAs per group; the int32 accumulator holds 16*I exactly
//   (the x16 nibble unpack, rt4_dev.h).
// * Activations: 16/M groups per register set (lane j holds row j%M of group
//   j/M), rotated into lanes 0..M-1 for the group being multiplied with DPP
//   row_ror.  With AL (one 16-row block per tile, pre-quantized activations) a
//   wave's chunk of activations (M rows x GPW groups x 128 B) arrives in whole
//   cache lines, 16 consecutive bytes per lane, and is redistributed into that
//   register layout through a wave-private LDS slice (XOR-swizzled so the 16
//   lanes of a quarter wave hit 16 distinct bank groups); the per-lane form
//   touches 16 half-used lines per instruction and measured ~5% slower.  The
//   loads sit in a block of their own so that the compiler keeps them ahead of
//   the weight stream (sunk behind it, the first MFMA would wait for every
//   weight load as well).
// * Weight scales: each wave loads its 16 rows x GPW fp16 scales as dwords into
//   a private LDS slice.  Scales and activations are issued before the weight
//   stream: vmcnt retires in order, so the first group can start as soon as its
//   weights land.  With 2 groups per wave, 3-8 chunks per wave and at most 4
//   waves (HS), each lane instead loads the scale dwords of two of its wave's
//   chunks once, before the chunk loop, and each chunk takes its dword from the
//   right lane with one ds_bpermute.
// * fp32 fold once per group: fp32(16I) * (f16(ws)/16 * sa) equals the
//   reference's (ws*sa)*I term bit for bit (power-of-two scaling is exact); only
//   the order of the sum over groups differs from the reference.  The W partial
//   sums of a tile are reduced through LDS.
// * Fused activation quantization (QIN): the whole decode linear of the
//   reference is two launches, quant_act then the GEMV (src/k_gemv.hip:70,
//   96-103).  Here the waves can read the fp32 activations themselves: each lane
//   loads the 32 values of its (row, group, quarter), the four quarter lanes of a
//   group agree on amax with two cross-row swaps, and the lane quantizes its
//   values into the interleaved int8 operand in registers.  The dependent
//   activation latency then hides under the weight stream instead of costing a
//   launch of its own.  Codes and scales are bit-identical to quant_act_a8_k.
//
// Two further forms of the pre-quantized launch, chosen by the default plan:
// * Row-transposed loads (gemv_w4a8_tl_k, 2-4 rows, K a multiple of 512): the
//   4-group configuration with each load instruction covering 4 rows x 256 B,
//   transposed to the operand layout through LDS; bit-identical to gemv_w4a8_k
//   on that configuration.
// * Dot products (gemv_w4a8_dot_k, one row, K a multiple of 256 up to 8192): each
//   wave streams two whole weight rows 1 KB per instruction and folds per group
//   with v_dot4_i32_i8 on the vector ALU.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// Lane j of each 16-lane row receives the value of lane (j + R) mod 16 (row_ror by 16-R).
template <int R>
__device__ __forceinline__ uint4 pull_u4(uint4 v) {
    if constexpr ((R & 15) == 0) {
        return v;
    } else {
        constexpr int C = 0x120 + ((16 - R) & 15);
        return make_uint4(dpp<C>(v.x), dpp<C>(v.y), dpp<C>(v.z), dpp<C>(v.w));
    }
}

// Quantize the 32 activations of one lane -- elements q*32..q*32+31 of a
// 128-group, quarter q held by lanes j, j+16, j+32, j+48 -- as quant_act_a8_k
// does: s = amax > 0 ? amax/127 : 1, c = clamp(rint(v/s), -128, 127).  Outputs the
// interleaved bytes (per 8 elements [c0 c2 c4 c6 c1 c3 c5 c7]) as two dwordx4 and
// the scale.  v/s uses rt4_dev.h's div_by_recip (a correctly rounded reciprocal
// and one fused correction step; equal to the IEEE quotient on every targeted
// input checked, see there).  Scales outside [2^-96, 2^100] (tiny or non-finite
// groups, where the residual could underflow) take the IEEE division instead.
__device__ __forceinline__ uint32_t pack4(int c0, int c1, int c2, int c3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)c1, (uint32_t)c0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)c3, (uint32_t)c2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

__device__ __forceinline__ void quant_lane(const float4 (&x)[8], uint4& a0, uint4& a1, float& scale) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++)
        amax = fmaxf(fmaxf(amax, fmaxf(fabsf(x[i].x), fabsf(x[i].y))), fmaxf(fabsf(x[i].z), fabsf(x[i].w)));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float s = amax > 0.f ? amax / 127.f : 1.f;
    scale = s;
    const bool fast = __all(s >= 0x1p-96f && s <= 0x1p+100f);
    const float y = 1.f / s;
    uint32_t d[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {  // 8 elements -> 2 dwords at a time (short live ranges)
        const float v[8] = {x[2 * k].x, x[2 * k].y, x[2 * k].z, x[2 * k].w,
                            x[2 * k + 1].x, x[2 * k + 1].y, x[2 * k + 1].z, x[2 * k + 1].w};
        int c[8];
        if (fast) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float t = v[e] * y;
                const float r = fmaf(-t, s, v[e]);
                c[e] = clampi((int)lrintf(fmaf(r, y, t)), -128, 127);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) c[e] = clampi((int)lrintf(v[e] / s), -128, 127);
        }
        d[2 * k] = pack4(c[0], c[2], c[4], c[6]);
        d[2 * k + 1] = pack4(c[1], c[3], c[5], c[7]);
    }
    a0 = make_uint4(d[0], d[1], d[2], d[3]);
    a1 = make_uint4(d[4], d[5], d[6], d[7]);
}

// LDS bytes of one wave's activation slice (AL).
template <int M, int GPW>
constexpr int gemv_al_bytes() { return M * GPW * 8 * 16; }

// The end of a tile, shared by the GEMV kernels: the W waves' partial sums are
// reduced through LDS (`red`: W x RB*M*16 floats), in wave order, and written out;
// a K range of a split tile instead publishes its partial (agent-coherent store),
// counts itself in, and the last piece to arrive sums all pieces in order
// (deterministic) and resets the counter for the next call.  No workgroup waits
// for another.  Outputs of the tile: o = (rb*M + r)*16 + l is row r, column
// n0 + 16 rb + l.
template <int M, int RB>
__device__ __forceinline__ void tile_finish(const float (&yacc)[RB][M], float* red, float* __restrict__ y, int N,
                                            int n0, int W, int w, int lane, bool piece, int b, int rem,
                                            const GemvSplit& sp) {
    constexpr int NOUT = RB * M * 16;
    if (W == 1 && !piece) {
        if (lane < 16)
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int r = 0; r < M; r++)
                    if (n0 + 16 * rb + lane < N) y[(size_t)r * N + n0 + 16 * rb + lane] = yacc[rb][r];
        return;
    }
    if (lane < 16)
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int r = 0; r < M; r++) red[(w * NOUT) + (rb * M + r) * 16 + lane] = yacc[rb][r];
    __syncthreads();
    // each thread sums the waves' partials of outputs o = threadIdx.x + i*blockDim.x
    constexpr int OPT = (NOUT + 63) / 64;    // outputs per thread at one wave (upper bound)
    float tot[OPT];
#pragma unroll
    for (int i = 0; i < OPT; i++) {
        const int o = threadIdx.x + i * blockDim.x;
        tot[i] = 0.f;
        if (o < NOUT)
            for (int v = 0; v < W; v++) tot[i] += red[v * NOUT + o];
    }
    if (!piece) {
#pragma unroll
        for (int i = 0; i < OPT; i++) {
            const int o = threadIdx.x + i * blockDim.x;
            const int n = n0 + 16 * (o / (M * 16)) + (o & 15), r = (o >> 4) % M;
            if (o < NOUT && n < N) y[(size_t)r * N + n] = tot[i];
        }
        return;
    }
    __shared__ int s_last;
#pragma unroll
    for (int i = 0; i < OPT; i++) {
        const int o = threadIdx.x + i * blockDim.x;
        if (o < NOUT) store_dev(sp.part + (size_t)b * NOUT + o, tot[i]);
    }
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(sp.cnt + rem, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == sp.S - 1;
    __syncthreads();
    if (!s_last) return;
#pragma unroll
    for (int i = 0; i < OPT; i++) {
        const int o = threadIdx.x + i * blockDim.x;
        if (o < NOUT) {
            float sum = 0.f;
            for (int v = 0; v < sp.S; v++) sum += load_dev(sp.part + (size_t)(rem * sp.S + v) * NOUT + o);
            const int n = n0 + 16 * (o / (M * 16)) + (o & 15), r = (o >> 4) % M;
            if (n < N) y[(size_t)r * N + n] = sum;
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(sp.cnt + rem, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int M, int GPW, int RB, bool AL, bool GSUM, bool QIN, bool HS>
__global__ __launch_bounds__(1024) void gemv_w4a8_k(const uint32_t* __restrict__ wq,
                                                    const uint16_t* __restrict__ ws,
                                                    const int8_t* __restrict__ xq,
                                                    const float* __restrict__ sa,
                                                    const float* __restrict__ xf,
                                                    float* __restrict__ y,
                                                    int32_t* __restrict__ gsum, int N, int K,
                                                    GemvSplit sp) {
    constexpr int GPS = 16 / M;                  // groups per activation register set
    constexpr int NSET = (GPW + GPS - 1) / GPS;
    constexpr int NP = GPW / 2;                  // group pairs per wave
    constexpr int ACH = M * GPW * 8;             // AL: 16-byte chunks of a wave's activations
    constexpr int AIN = (ACH + 63) / 64;         // AL: load instructions for them
    static_assert(!AL || (RB == 1 && !QIN), "line-wise activation loads: one row block, int8 input");
    static_assert(!HS || (AL && GPW == 2), "hoisted scales: line-wise loads, one group pair per wave");
    extern __shared__ __align__(16) unsigned char smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int NG = K >> 7, RS = K >> 1;          // groups and bytes per weight row
    const int NC = (NG + GPW - 1) / GPW;         // group chunks per tile
    // Workgroups [0, npieces) each take one K range of a remainder tile; the rest
    // take whole tiles (see launch_gemv_w4a8).
    const int b = blockIdx.x, npieces = sp.nrem * sp.S;
    const bool piece = b < npieces;
    const int rem = piece ? b / sp.S : 0, pc = piece ? b % sp.S : 0;
    const int tile = piece ? sp.full + rem : b - npieces;
    const int c_lo = piece ? pc * NC / sp.S : 0, c_hi = piece ? (pc + 1) * NC / sp.S : NC;
    const int n0 = tile * 16 * RB;
    // scale slice of this wave: [RB][16 rows][GPW/2] dwords (fp16 pairs); AL: the
    // activation slice [ACH] x 16 B; then the reduction area [W][RB][M][16]
    uint32_t* wsl = reinterpret_cast<uint32_t*>(smem) + (size_t)w * 8 * GPW * RB;
    uint4* axl = reinterpret_cast<uint4*>(smem + (size_t)W * 16 * GPW * 2 * RB) + (size_t)w * ACH;
    float* red = reinterpret_cast<float*>(smem + (size_t)W * 16 * GPW * 2 * RB +
                                          (AL ? (size_t)W * gemv_al_bytes<M, GPW>() : 0));

    // Load mapping of a group pair (rows n0..n0+15, 128 B each):
    //   instruction 1 covers rows 0-7, instruction 2 rows 8-15, 8 lanes per row;
    //   lane (j<8, q):  inst1 = (row j,    chunk q),   inst2 = (row j+8, chunk 4+q)
    //   lane (j>=8, q): inst1 = (row j-8,  chunk 4+q), inst2 = (row j,   chunk q)
    // so the first group of the pair is sel(j<8 ? inst1 : inst2) and the second
    // is ror8(sel(j<8 ? inst2 : inst1)).  Row block rb covers rows n0 + 16 rb ...
    const bool lo = j < 8;
    const unsigned char* p1[RB];
    const unsigned char* p2[RB];
    int rj[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int nb = n0 + 16 * rb;
        int r1 = nb + (lo ? j : j - 8), r2 = nb + (lo ? j + 8 : j);
        r1 = r1 < N ? r1 : N - 1;                // tail rows read a valid row; dropped
        r2 = r2 < N ? r2 : N - 1;
        p1[rb] = reinterpret_cast<const unsigned char*>(wq) + (size_t)r1 * RS + (lo ? q : 4 + q) * 16;
        p2[rb] = reinterpret_cast<const unsigned char*>(wq) + (size_t)r2 * RS + (lo ? 4 + q : q) * 16;
        rj[rb] = nb + j < N ? nb + j : N - 1;
    }
    const int jr = j % M, jg = j / M;
    const v4i zero = {0, 0, 0, 0};
    // HS (even NG, at most 8 chunks per wave): the scale dword (groups 2c, 2c+1) of
    // row n0 + j at this wave's iterations q and q + 4, loaded once before the loop;
    // iteration it takes it from lane j + 16 (it % 4).  Iterations past the wave's
    // last read chunk c_lo again (in bounds, unused).
    uint32_t hsc[2] = {0u, 0u};
    if constexpr (HS) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int c = c_lo + w + (q + 4 * i) * W;
            c = c < c_hi ? c : c_lo;
            hsc[i] = *reinterpret_cast<const uint32_t*>(ws + (size_t)rj[0] * NG + 2 * c);
        }
    }

    float yacc[RB][M];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int r = 0; r < M; r++) yacc[rb][r] = 0.f;

    int it = 0;
    for (int c = c_lo + w; c < c_hi; c += W, it++) {
        const int g0 = uniform(c * GPW);
        // (1) this wave's scales: RB x 16 rows x GPW fp16, as dwords (even NG:
        //     every row starts 4-byte aligned) or as halves (odd NG)
        uint32_t sw[RB][(GPW / 2 + 3) / 4];
#pragma unroll
        for (int rb = 0; rb < (HS ? 0 : RB); rb++)
#pragma unroll
            for (int d = 0; d < (GPW / 2 + 3) / 4; d++) {
                const int dw = q + 4 * d;
                const int g = g0 + 2 * dw;
                const uint16_t* sp = ws + (size_t)rj[rb] * NG;
                uint32_t v = 0;
                if (dw < GPW / 2 && g < NG) {
                    if (!(NG & 1))
                        v = *reinterpret_cast<const uint32_t*>(sp + g);
                    else
                        v = (uint32_t)sp[g] | (g + 1 < NG ? (uint32_t)sp[g + 1] << 16 : 0u);
                }
                sw[rb][d] = v;
            }
        // (2) activations: set s, lane j holds row j%M of group g0 + s*GPS + j/M
        //     (QIN: its fp32 values, quantized after the weight loads are issued)
        uint4 ax0[NSET], ax1[NSET];
        float asc[NSET];
        float4 xv[QIN ? NSET : 1][8];
        uint4 araw[AL ? AIN : 1];
        if constexpr (AL) {
            // chunk e = 64i + lane: row e/(8 GPW), group (e/8)%GPW, 16 bytes at 16(e%8)
#pragma unroll
            for (int i = 0; i < AIN; i++) araw[i] = make_uint4(0, 0, 0, 0);
            if (NG > 0) {   // always true: a block of its own keeps these loads first
#pragma unroll
                for (int i = 0; i < AIN; i++) {
                    int e = i * 64 + lane;
                    e = e < ACH ? e : ACH - 1;
                    const int row = e / (GPW * 8), grp = (e / 8) % GPW, cc = e % 8;
                    int g = g0 + grp;
                    g = g < NG ? g : NG - 1;
                    araw[i] = *reinterpret_cast<const uint4*>(xq + (size_t)row * K + (size_t)g * 128 + cc * 16);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < NSET; s++) {
            int g = g0 + s * GPS + jg;
            g = g < NG ? g : NG - 1;
            if constexpr (AL) {
                (void)g;
            } else if constexpr (QIN) {
                const float4* xp = reinterpret_cast<const float4*>(xf + (size_t)jr * K + (size_t)g * 128 + q * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) xv[s][i] = xp[i];
            } else {
                const uint4* ap = reinterpret_cast<const uint4*>(xq + (size_t)jr * K + (size_t)g * 128 + q * 32);
                ax0[s] = ap[0];
                ax1[s] = ap[1];
            }
        }
        // (3) the weight stream.  A pair starting at the last group of an odd NG
        //     has no second group: its lanes read the first group again (in bounds)
        //     and that result is never used.
        v4u a[RB][NP], b[RB][NP];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            int gp = g0 + 2 * p;
            if (gp >= NG) gp = NG >= 2 ? NG - 2 : 0;
            const int tail = (gp + 1 >= NG) ? 64 : 0;
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                a[rb][p] = __builtin_nontemporal_load(
                    reinterpret_cast<const v4u*>(p1[rb] + (size_t)gp * 64 - (lo ? 0 : tail)));
                b[rb][p] = __builtin_nontemporal_load(
                    reinterpret_cast<const v4u*>(p2[rb] + (size_t)gp * 64 - (lo ? tail : 0)));
            }
        }
#pragma unroll
        for (int rb = 0; rb < (HS ? 0 : RB); rb++)
#pragma unroll
            for (int d = 0; d < (GPW / 2 + 3) / 4; d++) {
                const int dw = q + 4 * d;
                if (dw < GPW / 2) wsl[(rb * 16 + j) * (GPW / 2) + dw] = sw[rb][d];
            }
        if constexpr (QIN) {
#pragma unroll
            for (int s = 0; s < NSET; s++) quant_lane(xv[s], ax0[s], ax1[s], asc[s]);
        }
        if constexpr (AL) {
            // into the wave's slice, then out in the register layout: lane (j, q) of set
            // s takes chunks 2q, 2q+1 of (row j%M, group s*GPS + j/M).  Slot of chunk cc
            // of (row, grp): ((row*GPW + grp)*8 + (cc ^ h)), h = (row*8/Mp + grp/2) % 8
            // with Mp = 1, 2, 4, 4 for M = 1..4.  LDS operations of one wave complete in
            // order, so no barrier is needed; the fences only keep the compiler's order.
            constexpr int RSH = M == 1 ? 3 : M == 2 ? 2 : 1;    // log2(8/Mp)
#pragma unroll
            for (int i = 0; i < AIN; i++) {
                const int e = i * 64 + lane;
                if (e < ACH) {
                    const int row = e / (GPW * 8), grp = (e / 8) % GPW, cc = e % 8;
                    const int h = ((row << RSH) + (grp >> 1)) & 7;
                    axl[(row * GPW + grp) * 8 + (cc ^ h)] = araw[i];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int s = 0; s < NSET; s++) {
                int grp = s * GPS + jg;
                grp = grp < GPW ? grp : GPW - 1;          // lanes past the chunk: unused
                const int h = ((jr << RSH) + (grp >> 1)) & 7;
                ax0[s] = axl[(jr * GPW + grp) * 8 + ((2 * q) ^ h)];
                ax1[s] = axl[(jr * GPW + grp) * 8 + ((2 * q + 1) ^ h)];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }

#pragma unroll
        for (int p = 0; p < NP; p++) {
            v4u t0[RB], t1[RB];
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                v4u x;
                t0[rb].x = lo ? a[rb][p].x : b[rb][p].x;
                t0[rb].y = lo ? a[rb][p].y : b[rb][p].y;
                t0[rb].z = lo ? a[rb][p].z : b[rb][p].z;
                t0[rb].w = lo ? a[rb][p].w : b[rb][p].w;
                x.x = lo ? b[rb][p].x : a[rb][p].x;
                x.y = lo ? b[rb][p].y : a[rb][p].y;
                x.z = lo ? b[rb][p].z : a[rb][p].z;
                x.w = lo ? b[rb][p].w : a[rb][p].w;
                t1[rb].x = dpp<0x128>(x.x);
                t1[rb].y = dpp<0x128>(x.y);
                t1[rb].z = dpp<0x128>(x.z);
                t1[rb].w = dpp<0x128>(x.w);
            }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int u = 2 * p + h, g = g0 + u;
                uint4 xa, xb;
                switch (u % GPS) {
#define RT4_PULL(I)                                      \
    case I:                                              \
        xa = pull_u4<((I) * M) & 15>(ax0[u / GPS]);      \
        xb = pull_u4<((I) * M) & 15>(ax1[u / GPS]);      \
        break;
                    RT4_PULL(0) RT4_PULL(1) RT4_PULL(2) RT4_PULL(3) RT4_PULL(4) RT4_PULL(5) RT4_PULL(6)
                    RT4_PULL(7) RT4_PULL(8) RT4_PULL(9) RT4_PULL(10) RT4_PULL(11) RT4_PULL(12)
                    RT4_PULL(13) RT4_PULL(14) RT4_PULL(15)
#undef RT4_PULL
                }
                const v4i A0 = {(int)xa.x, (int)xa.y, (int)xa.z, (int)xa.w};
                const v4i A1 = {(int)xb.x, (int)xb.y, (int)xb.z, (int)xb.w};
                float a_s[M];
                if (g < NG) {
#pragma unroll
                    for (int r = 0; r < M; r++) {
                        if constexpr (QIN)  // the scale of (row r, group g) sits in lane (u % GPS) * M + r
                            a_s[r] = __int_as_float(
                                __builtin_amdgcn_readlane(__float_as_int(asc[u / GPS]), (u % GPS) * M + r));
                        else
                            a_s[r] = sa[(size_t)r * NG + g];
                    }
                }
#pragma unroll
                for (int rb = 0; rb < RB; rb++) {
                    const v4u qv = h ? t1[rb] : t0[rb];
                    const v4i b0 = {(int)even_x16(qv.x), (int)odd_x16(qv.x), (int)even_x16(qv.y), (int)odd_x16(qv.y)};
                    const v4i b1 = {(int)even_x16(qv.z), (int)odd_x16(qv.z), (int)even_x16(qv.w), (int)odd_x16(qv.w)};
                    v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, zero, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, acc, 0, 0, 0);
                    // lane l < 16 now holds 16*I[m=r][n0+16rb+l] in acc[r]
                    if (g < NG) {
                        const int nl = n0 + 16 * rb + lane;
                        if (GSUM && lane < 16 && nl < N)
#pragma unroll
                            for (int r = 0; r < M; r++) gsum[((size_t)r * N + nl) * NG + g] = acc[r] >> 4;
                        const uint32_t pair =
                            HS ? (uint32_t)__builtin_amdgcn_ds_bpermute((j + 16 * (it & 3)) * 4,
                                                                        (int)((it & 4) ? hsc[1] : hsc[0]))
                               : wsl[(rb * 16 + j) * (GPW / 2) + p];
                        const float s16 = f16_bits_to_f32((uint16_t)(h ? pair >> 16 : pair & 0xFFFFu)) * 0.0625f;
#pragma unroll
                        for (int r = 0; r < M; r++) yacc[rb][r] = fmaf((float)acc[r], s16 * a_s[r], yacc[rb][r]);
                    }
                }
            }
        }
    }

    tile_finish<M, RB>(yacc, red, y, N, n0, W, w, lane, piece, b, rem, sp);
}

// ---- Row-transposed loads (TL): the configuration of gemv_w4a8_k with 4 groups
// per wave, one 16-row block, line-wise activations and pre-quantized input, for
// K a multiple of 512 and at most 8 waves.  Same chunk-to-wave assignment, same
// group order within a wave and the same fold, so its outputs are bit-identical
// to gemv_w4a8_k's on that configuration; only the weight stream differs.
//
// * A chunk (4 groups of 16 rows, 16 x 256 B) is read by four dwordx4 load
//   instructions of 4 rows x 256 B each: instruction k, lane l reads row
//   4k + l/16, 16-byte piece (l%16) ^ (4k + l/16) of the row's 256 B.  Longer runs
//   per row than gemv_w4a8_k's 8 rows x 128 B measured ~8% faster for the load
//   stream alone at the 27B shapes.
// * A wave holds one chunk at a time: its scales, activations and weights are
//   issued together (64 B of weights per lane, twice gemv_w4a8_k's two-group
//   chunk), then used.  About 70 VGPRs, so ~7 waves per SIMD stay resident and
//   other waves' loads cover a wave's arithmetic.  Holding 2 or 4 chunks per wave
//   (all issued before the first is used) measured 5-15% slower: the extra
//   registers cost more residency than the deeper queue gains.
// * The MFMA operand needs row j in lanes j, j+16, j+32, j+48, so each chunk goes
//   through a wave-private 4 KB LDS slice: written lane-linearly (conflict-free),
//   read back as lane (j, q) <- row j, piece 4u + q for group u; the XOR of the
//   piece index with the row keeps the 16 lanes of each read quarter on distinct
//   banks.
template <int M, bool GSUM>
__device__ __forceinline__ void tl_chunk(const unsigned char* const (&pk)[4], const uint16_t* wsr,
                                          const int8_t* __restrict__ xq, const float* __restrict__ sa,
                                          int32_t* __restrict__ gsum, uint4* tl, uint4* axl, int c, int NG,
                                          int K, int N, int n0, int lane, float (&yacc)[1][M]) {
    constexpr int GPW = 4, GPS = 16 / M, NSET = (GPW + GPS - 1) / GPS;
    constexpr int ACH = M * GPW * 8, AIN = (ACH + 63) / 64;
    constexpr int RSH = M == 1 ? 3 : M == 2 ? 2 : 1;    // activation slice swizzle, as gemv_w4a8_k
    const int j = lane & 15, q = lane >> 4;
    const int jr = j % M, jg = j / M;
    const v4i zero = {0, 0, 0, 0};
    const int g0 = uniform(c * GPW);
    // the chunk's scales, activations and weights, all issued before any wait (the
    // scheduler would otherwise sink the later loads behind the first wait); the
    // activations go first, so the LDS staging can start while weights arrive
    uint32_t sw[2];
    v4u araw[AIN], wv[4];
    sw[0] = *reinterpret_cast<const uint32_t*>(wsr + g0);
    sw[1] = *reinterpret_cast<const uint32_t*>(wsr + g0 + 2);
#pragma unroll
    for (int t = 0; t < AIN; t++) {
        int e = t * 64 + lane;
        e = e < ACH ? e : ACH - 1;
        const int row = e / (GPW * 8), grp = (e / 8) % GPW, cc = e % 8;
        araw[t] = *reinterpret_cast<const v4u*>(xq + (size_t)row * K + (size_t)(g0 + grp) * 128 + cc * 16);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) wv[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(pk[k] + (size_t)g0 * 64));
    __builtin_amdgcn_sched_barrier(0);
    {
#pragma unroll
        for (int k = 0; k < 4; k++) tl[k * 64 + lane] = make_uint4(wv[k].x, wv[k].y, wv[k].z, wv[k].w);
#pragma unroll
        for (int t = 0; t < AIN; t++) {
            const int e = t * 64 + lane;
            if (e < ACH) {
                const int row = e / (GPW * 8), grp = (e / 8) % GPW, cc = e % 8;
                const int h = ((row << RSH) + (grp >> 1)) & 7;
                axl[(row * GPW + grp) * 8 + (cc ^ h)] = make_uint4(araw[t].x, araw[t].y, araw[t].z, araw[t].w);
            }
        }
        // LDS operations of one wave complete in order, so no barrier is needed; the
        // fences only keep the compiler's order
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint4 wt[4];
#pragma unroll
        for (int u = 0; u < 4; u++) wt[u] = tl[j * 16 + ((4 * u + q) ^ j)];
        uint4 ax0[NSET], ax1[NSET];
#pragma unroll
        for (int s = 0; s < NSET; s++) {
            int grp = s * GPS + jg;
            grp = grp < GPW ? grp : GPW - 1;          // lanes past the chunk: unused
            const int h = ((jr << RSH) + (grp >> 1)) & 7;
            ax0[s] = axl[(jr * GPW + grp) * 8 + ((2 * q) ^ h)];
            ax1[s] = axl[(jr * GPW + grp) * 8 + ((2 * q + 1) ^ h)];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int g = g0 + u;
            uint4 xa, xb;
            switch (u % GPS) {
#define RT4_PULL(I)                                      \
    case I:                                              \
        xa = pull_u4<((I) * M) & 15>(ax0[u / GPS]);      \
        xb = pull_u4<((I) * M) & 15>(ax1[u / GPS]);      \
        break;
                RT4_PULL(0) RT4_PULL(1) RT4_PULL(2) RT4_PULL(3)
#undef RT4_PULL
            }
            const v4i A0 = {(int)xa.x, (int)xa.y, (int)xa.z, (int)xa.w};
            const v4i A1 = {(int)xb.x, (int)xb.y, (int)xb.z, (int)xb.w};
            float a_s[M];
#pragma unroll
            for (int r = 0; r < M; r++) a_s[r] = sa[(size_t)r * NG + g];
            const uint4 qv = wt[u];
            const v4i b0 = {(int)even_x16(qv.x), (int)odd_x16(qv.x), (int)even_x16(qv.y), (int)odd_x16(qv.y)};
            const v4i b1 = {(int)even_x16(qv.z), (int)odd_x16(qv.z), (int)even_x16(qv.w), (int)odd_x16(qv.w)};
            v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, zero, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, acc, 0, 0, 0);
            // lane l < 16 now holds 16*I[m=r][n0+l] in acc[r]
            const int nl = n0 + lane;
            if (GSUM && lane < 16 && nl < N)
#pragma unroll
                for (int r = 0; r < M; r++) gsum[((size_t)r * N + nl) * NG + g] = acc[r] >> 4;
            const uint32_t pair = sw[u >> 1];
            const float s16 = f16_bits_to_f32((uint16_t)((u & 1) ? pair >> 16 : pair & 0xFFFFu)) * 0.0625f;
#pragma unroll
            for (int r = 0; r < M; r++) yacc[0][r] = fmaf((float)acc[r], s16 * a_s[r], yacc[0][r]);
        }
    }
}

// LDS bytes of a TL workgroup of W waves: transposition slices, activation slices,
// reduction area.
template <int M>
constexpr size_t gemv_tl_lds(int W) {
    return (size_t)W * 4096 + (size_t)W * gemv_al_bytes<M, 4>() + (size_t)W * M * 16 * sizeof(float);
}

template <int M, bool GSUM>
__global__ __launch_bounds__(512) void gemv_w4a8_tl_k(const uint32_t* __restrict__ wq,
                                                      const uint16_t* __restrict__ ws,
                                                      const int8_t* __restrict__ xq,
                                                      const float* __restrict__ sa,
                                                      float* __restrict__ y,
                                                      int32_t* __restrict__ gsum, int N, int K, GemvSplit sp) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
    const int j = lane & 15;
    const int NG = K >> 7, RS = K >> 1, NC = NG >> 2;
    const int b = blockIdx.x, npieces = sp.nrem * sp.S;
    const bool piece = b < npieces;
    const int rem = piece ? b / sp.S : 0, pc = piece ? b % sp.S : 0;
    const int tile = piece ? sp.full + rem : b - npieces;
    const int c_lo = piece ? pc * NC / sp.S : 0, c_hi = piece ? (pc + 1) * NC / sp.S : NC;
    const int n0 = tile * 16;
    uint4* tl = reinterpret_cast<uint4*>(smem) + (size_t)w * 256;
    uint4* axl = reinterpret_cast<uint4*>(smem + (size_t)W * 4096) + (size_t)w * (M * 4 * 8);
    float* red = reinterpret_cast<float*>(smem + (size_t)W * 4096 + (size_t)W * gemv_al_bytes<M, 4>());
    const unsigned char* pk[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int rho = 4 * k + (lane >> 4);
        int r = n0 + rho;
        r = r < N ? r : N - 1;                   // tail rows read a valid row; dropped
        pk[k] = reinterpret_cast<const unsigned char*>(wq) + (size_t)r * RS + (((lane & 15) ^ rho) * 16);
    }
    const uint16_t* wsr = ws + (size_t)(n0 + j < N ? n0 + j : N - 1) * NG;
    float yacc[1][M];
#pragma unroll
    for (int r = 0; r < M; r++) yacc[0][r] = 0.f;
    for (int c = c_lo + w; c < c_hi; c += W)
        tl_chunk<M, GSUM>(pk, wsr, xq, sa, gsum, tl, axl, c, NG, K, N, n0, lane, yacc);
    tile_finish<M, 1>(yacc, red, y, N, n0, W, w, lane, piece, b, rem, sp);
}

// ---- One activation row, row-contiguous dot products (DOT).  At M = 1 a 16-row
// MFMA tile uses one of its 16 activation rows; here the vector ALU does the
// arithmetic instead and the weight stream is laid out for the memory system
// alone.  Each wave owns RPW consecutive weight rows, i.e. one contiguous span of
// RPW*K/2 bytes, read 1 KB per load instruction (lane l of instruction i takes
// bytes 16(64i + l) of the span), every instruction of a batch issued before the
// first is used.  Rows are multiples of 64 B, so the four lanes of a quad always
// hold the four 16-byte quarters of one 128-element group of one row:
//   * lane: the 32 codes times the matching 32 activation codes (read from global
//     memory, interleaved as quant_act_a8_k writes them: per 8 elements
//     [c0 c2 c4 c6 c1 c3 c5 c7], the order of the even and odd nibbles), 8
//     v_dot4_i32_i8 on the x16 nibble unpack -> 16 * its partial, exact;
//   * quad: two DPP adds -> 16 * I[n][g] in all four lanes, exact;
//   * quad leader: fp32(16 I) * (f16(ws)/16 * sa), the fold of gemv_w4a8_k, added
//     to its row's fp32 partial; the wave then sums its 16 leaders per row.
// No LDS, no cross-wave reduction and no K split; only the order of the fp32 sum
// over groups differs from the MFMA forms.
template <int RPW, int NI, bool GSUM>
__global__ __launch_bounds__(256) void gemv_w4a8_dot_k(const uint32_t* __restrict__ wq,
                                                       const uint16_t* __restrict__ ws,
                                                       const int8_t* __restrict__ xq,
                                                       const float* __restrict__ sa,
                                                       float* __restrict__ y,
                                                       int32_t* __restrict__ gsum, int N, int K) {
    static_assert(RPW == 1 || RPW == 2, "one or two rows per wave");
    const int lane = threadIdx.x & 63;
    const int wv = uniform((int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
    const int NG = K >> 7, RS = K >> 1;
    const int n0 = wv * RPW;
    if (n0 >= N) return;                              // whole wave: no barrier follows
    const int nrows = min(RPW, N - n0);
    const int span = nrows * RS;                      // bytes, a multiple of 64; NI = ceil(RPW*RS/1024)
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(wq) + (size_t)n0 * RS;
    const bool leader = (lane & 3) == 3;
    // the wave's weight scales (nrows*NG fp16, contiguous) and the activation
    // scales (NG floats), one dword per lane (RPW*NG <= 128), handed to the pieces
    // with ds_bpermute; then every weight and activation load of the wave, in one
    // straight-line block (a piece past the span -- the tail of the last
    // instruction, or a short last wave -- reads the span's last piece again and is
    // dropped)
    const int nsw = (nrows * NG + 1) >> 1;
    const uint32_t wsd = lane < nsw ? reinterpret_cast<const uint32_t*>(ws + (size_t)n0 * NG)[lane] : 0u;
    const float sad = lane < NG ? sa[lane] : 0.f;
    v4u w4[NI], x0[NI], x1[NI];
    int rsv[NI], gv[NI];
    bool okv[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int ou = (i * 64 + lane) * 16;
        okv[i] = ou < span;
        const int o = okv[i] ? ou : span - 16;
        rsv[i] = RPW == 2 && o >= RS ? 1 : 0;
        const int br = o - rsv[i] * RS;               // byte in the row
        gv[i] = br >> 6;
        w4[i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wb + o));
        const v4u* xp = reinterpret_cast<const v4u*>(xq + (size_t)br * 2);
        x0[i] = xp[0];
        x1[i] = xp[1];
    }
    __builtin_amdgcn_sched_barrier(0);
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int i = 0; i < NI; i++) {
        int I = 0;
        I = __builtin_amdgcn_sdot4((int)even_x16(w4[i].x), (int)x0[i].x, I, false);
        I = __builtin_amdgcn_sdot4((int)odd_x16(w4[i].x), (int)x0[i].y, I, false);
        I = __builtin_amdgcn_sdot4((int)even_x16(w4[i].y), (int)x0[i].z, I, false);
        I = __builtin_amdgcn_sdot4((int)odd_x16(w4[i].y), (int)x0[i].w, I, false);
        I = __builtin_amdgcn_sdot4((int)even_x16(w4[i].z), (int)x1[i].x, I, false);
        I = __builtin_amdgcn_sdot4((int)odd_x16(w4[i].z), (int)x1[i].y, I, false);
        I = __builtin_amdgcn_sdot4((int)even_x16(w4[i].w), (int)x1[i].z, I, false);
        I = __builtin_amdgcn_sdot4((int)odd_x16(w4[i].w), (int)x1[i].w, I, false);
        I += (int)dpp<0xB1>((uint32_t)I);            // quad_perm [1,0,3,2]
        I += (int)dpp<0x4E>((uint32_t)I);            // quad_perm [2,3,0,1]
        const bool use = leader && okv[i];
        if (GSUM && use) gsum[(size_t)(n0 + rsv[i]) * NG + gv[i]] = I >> 4;
        const int h = rsv[i] * NG + gv[i];           // this piece's fp16 scale in the wave's list
        const uint32_t pr = (uint32_t)__builtin_amdgcn_ds_bpermute((h >> 1) * 4, (int)wsd);
        const float s_a = __int_as_float(__builtin_amdgcn_ds_bpermute(gv[i] * 4, __float_as_int(sad)));
        // the fold of gemv_w4a8_k, fp32(16 I) * (f16(ws)/16 * sa), into this row's sum
        // (a zero scale elsewhere: the term adds an exact zero)
        const float sc = use ? f16_bits_to_f32((uint16_t)((h & 1) ? pr >> 16 : pr & 0xFFFFu)) * 0.0625f * s_a : 0.f;
        acc0 = fmaf((float)I, RPW == 2 && rsv[i] ? 0.f : sc, acc0);
        if (RPW == 2) acc1 = fmaf((float)I, rsv[i] ? sc : 0.f, acc1);
        __builtin_amdgcn_sched_barrier(0);   // piece i's arithmetic waits for piece i's loads only
    }
    // sum of the 16 leaders (lanes 3, 7, ..., 63) per row: within each 16-lane row by
    // two shifted adds (lane 15 of the row), then across rows by the two broadcasts
    // (lane 63)
    auto wave_sum = [&](float v) __attribute__((always_inline)) {
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, true));   // row_shr:4
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, true));   // row_shr:8
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));  // row_bcast:31
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    };
    const float y0 = wave_sum(acc0);
    const float y1 = RPW == 2 ? wave_sum(acc1) : 0.f;
    if (lane == 0) {
        y[n0] = y0;
        if (RPW == 2 && nrows == 2) y[n0 + 1] = y1;
    }
}

// Load instructions per wave of the dot-product form (1 KB each), at most this many
// (128 registers of loads in flight per lane).
constexpr int kDotMaxInst = 8;
inline int dot_inst(int rpw, int K) { return (rpw * (K / 2) + 1023) / 1024; }

template <int RPW, bool GSUM>
hipError_t launch_dot(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                      const float* sa, int N, int K, int wpb, hipStream_t st) {
    const int nw = (N + RPW - 1) / RPW, grid = (nw + wpb - 1) / wpb;
    const dim3 g(grid), b(64 * wpb);
    switch (dot_inst(RPW, K)) {
#define RT4_DOT(NI) \
    case NI: hipLaunchKernelGGL((gemv_w4a8_dot_k<RPW, NI, GSUM>), g, b, 0, st, wq, ws, xq, sa, y, gsum, N, K); break;
        RT4_DOT(1) RT4_DOT(2) RT4_DOT(3) RT4_DOT(4) RT4_DOT(5) RT4_DOT(6) RT4_DOT(7) RT4_DOT(8)
#undef RT4_DOT
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int M, int GPW, int RB, bool GSUM, bool QIN>
hipError_t launch_one(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                      const float* sa, const float* xf, int N, int K, int waves, const GemvSplit& sp,
                      hipStream_t st) {
    const size_t base = (size_t)waves * 16 * GPW * 2 * RB + (size_t)waves * RB * M * 16 * sizeof(float);
    const size_t al = (size_t)waves * gemv_al_bytes<M, GPW>();
    const int grid = sp.full + sp.nrem * sp.S;
    // line-wise activation loads where they apply and their LDS slices fit the
    // default 64 KB of dynamic LDS
    if constexpr (RB == 1 && !QIN && GPW == 4) {
        // row-transposed loads: same results, faster weight stream
        const int NG = K / kGroup;
        if (NG % 4 == 0 && waves <= 8 && gemv_tl_lds<M>(waves) <= 65536) {
            hipLaunchKernelGGL((gemv_w4a8_tl_k<M, GSUM>), dim3(grid), dim3(64 * waves), gemv_tl_lds<M>(waves), st, wq,
                               ws, xq, sa, y, gsum, N, K, sp);
            return hipGetLastError();
        }
    }
    if constexpr (RB == 1 && !QIN) {
        if (base + al <= 65536) {
            // Scales hoisted out of the chunk loop where a wave has at least 3 and at
            // most 8 chunks and the tile has at most 4 waves (measured: gate/up, 4
            // waves x 5 chunks, 11.42 -> 11.30 us; with 16 waves, as at the down and
            // M=1 shapes, the extra loads cost more than they save).
            const int NG = K / kGroup, NC = (NG + GPW - 1) / GPW, per_wave = (NC + waves - 1) / waves;
            if constexpr (GPW == 2) {
                if (!(NG & 1) && waves <= 4 && per_wave >= 3 && per_wave <= 8) {
                    hipLaunchKernelGGL((gemv_w4a8_k<M, GPW, RB, true, GSUM, QIN, true>), dim3(grid),
                                       dim3(64 * waves), base + al, st, wq, ws, xq, sa, xf, y, gsum, N, K, sp);
                    return hipGetLastError();
                }
            }
            hipLaunchKernelGGL((gemv_w4a8_k<M, GPW, RB, true, GSUM, QIN, false>), dim3(grid), dim3(64 * waves),
                               base + al, st, wq, ws, xq, sa, xf, y, gsum, N, K, sp);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv_w4a8_k<M, GPW, RB, false, GSUM, QIN, false>), dim3(grid), dim3(64 * waves), base, st, wq, ws,
                       xq, sa, xf, y, gsum, N, K, sp);
    return hipGetLastError();
}

template <int M, int RB, bool GSUM, bool QIN>
hipError_t launch_g(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                    const float* sa, const float* xf, int N, int K, const GemvCfg& c, const GemvSplit& sp,
                    hipStream_t st) {
    switch (c.gpw) {
        case 2: return launch_one<M, 2, RB, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c.waves, sp, st);
        case 4: return launch_one<M, 4, RB, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c.waves, sp, st);
        case 6: return launch_one<M, 6, RB, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c.waves, sp, st);
        case 8: return launch_one<M, 8, RB, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c.waves, sp, st);
        case 10: return launch_one<M, 10, RB, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c.waves, sp, st);
        case 12: return launch_one<M, 12, RB, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c.waves, sp, st);
    }
    return hipErrorInvalidValue;
}

template <int M, bool GSUM, bool QIN>
hipError_t launch_m(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                    const float* sa, const float* xf, int N, int K, const GemvCfg& c, const GemvSplit& sp,
                    hipStream_t st) {
    return c.rb == 2 ? launch_g<M, 2, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c, sp, st)
                     : launch_g<M, 1, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c, sp, st);
}

template <bool GSUM, bool QIN>
hipError_t launch_rows(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                       const float* sa, const float* xf, int rows, int N, int K, const GemvCfg& c,
                       const GemvSplit& sp, hipStream_t st) {
    switch (rows) {
        case 1: return launch_m<1, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c, sp, st);
        case 2: return launch_m<2, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c, sp, st);
        case 3: return launch_m<3, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c, sp, st);
        case 4: return launch_m<4, GSUM, QIN>(y, gsum, wq, ws, xq, sa, xf, N, K, c, sp, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

GemvCfg gemv_default_cfg(int rows, int N, int K, int cus) {
    // One activation row with K a multiple of 256 up to 8192 and at most 16 tiles of
    // 16 rows per CU: the dot-product form, two weight rows per wave.  Measured on
    // MI355X (us, this form vs the MFMA rule below): K=5120 N=5120 4.9 vs 6.0,
    // N=10240 6.9 vs 7.7, N=17408 9.9 vs 10.8; K=2048 N=8192 4.2 vs 4.8; K=4096
    // N=14336 8.0 vs 8.2; K=8192 N=8192 8.3 vs 9.3, N=28672 20.7 vs 24.3.  (One row
    // per wave: 5.0, 10.6, 7.4, 4.1-4.4.)  At the LM head (N=248320, 61 tiles per
    // CU) its 124,160 small waves lose: 112.4 vs 96.9 us.
    GemvCfg c = gemv_mfma_cfg(rows, N, K, cus);
    const int ncu = cus > 0 ? cus : 256;
    if (rows == 1 && K % 256 == 0 && K / kGroup <= 64 && dot_inst(2, K) <= kDotMaxInst &&
        (N + 15) / 16 <= 16 * ncu)
        c.dot = 2;
    return c;
}

GemvCfg gemv_mfma_cfg(int rows, int N, int K, int cus) {
    const int NG = K / kGroup;
    cus = cus > 0 ? cus : 256;
    GemvCfg c;
    // Two 16-row blocks per tile when each CU has enough tile x group work for
    // the last round's imbalance not to matter, and the activation operand is
    // wide enough for its reuse to pay (3-4 rows).  Measured at 4 rows: LM head
    // (N = 248320) 114 vs 128 us; K = 17408, N = 40960 68 vs 78 us; below about
    // 300 (32-row tile x group) units per CU it is slower (N = 17408 at K =
    // 5120: 13.6 vs 12.7 us).  One row: slower at every N.
    c.rb = rows >= kGemvRb2MinRows && (long long)((N + 31) / 32) * NG >= (long long)kGemvRb2Work * cus ? 2 : 1;
    const int ng_even = (NG + 1) & ~1;
    const int ntiles = (N + 15) / 16;
    // One row block with line-wise activation loads: 2 groups per wave while the
    // grid is at most ~5 tiles per CU (about one residency round), with waves per
    // tile and the leftover-tile split chosen per band.  Measured on MI355X (us,
    // this rule vs the general one below): M=4 K=5120: N=6144 6.3 vs 7.0, 10240
    // 8.0 vs 8.6, 17408 11.3 vs 12.2-12.8, 20480 12.5 vs 13.0; N=24576 (6 tiles
    // per CU) 14.3 vs 15.3 with 8 waves; K=17408: N=5120 11.1 vs 11.6, 10240 20.1
    // vs 21.7, 17408 32.4 vs 35.5; M=1 K=5120: N=5120 5.9 vs 6.2, 10240 7.6 vs
    // 7.8, 17408 10.8 vs 10.9.  Beyond that (the LM head at 1-2 rows: 109 vs 97
    // us) the general rule wins.
    const double tpc = (double)ntiles / cus;
    // Two to four rows with K a multiple of 512: 4 groups per wave, which runs the
    // row-transposed kernel (gemv_w4a8_tl_k).  Measured on MI355X (us, this rule
    // vs the 2-group rule below): M=4 K=5120 N=17408 10.5 vs 11.2, N=10240 7.7
    // vs 8.1; K=17408 N=5120 10.9 vs 11.2, N=17408 31.8 vs 36.0; M=2 K=5120
    // N=17408 10.2 vs 10.9.  One row gains nothing measurable (C0 6.0 either way).
    // Three rows up to 2 tiles per CU (2.75 at K < 16384) take the 2-group form
    // below: M=3 K=17408 N=5120 11.3 vs 13.8 us, N=2048 8.7 vs 10.1; K=5120 N=5120
    // 6.8 vs 8.6, N=10240 8.5 vs 8.7; but K=17408 N=10240 18.8 here vs 20.0.
    const bool three_wide = rows == 3 && (tpc <= 2.0 || (tpc <= 2.75 && K < 16384));
    if (c.rb == 1 && rows >= 2 && NG % 4 == 0 && !three_wide &&
        (tpc <= 5.0 || (rows >= 3 && tpc <= 7.5))) {
        c.gpw = 4;
        int w = tpc <= 2.75 ? 8 : rows == 3 ? 4 : 2;
        const int nc = NG / 4;
        c.waves = w < nc ? w : nc;
        // Leftover tiles in at most 4 K pieces above 3 tiles per CU; below that the
        // pieces keep >= 32 groups (0): whole tiles at K=5120 (M=4 N=5120 6.6 vs
        // 7.7 us in 4 pieces, M=2 6.3 vs 7.5, M=2 N=2048 5.2 vs 6.4), still 4
        // pieces at K=17408.
        c.max_split = tpc > 3.0 ? 4 : 0;
        return c;
    }
    if (c.rb == 1 && (tpc <= 5.0 || (rows >= 3 && tpc <= 7.5))) {
        c.gpw = 2 < ng_even ? 2 : ng_even;
        const int nc = (NG + c.gpw - 1) / c.gpw;
        int w;
        if (tpc <= 2.0 || K >= 16384) w = 16;
        else if (tpc <= 2.75 || tpc > 5.0) w = 8;
        else w = 4;
        w = w < nc ? w : nc;
        c.waves = w < kGemvMaxWaves ? w : kGemvMaxWaves;
        // at most 4 pieces per leftover tile in the middle bands (M=4 K=5120
        // N=8704: 7.7 us vs 9.3 us with 8 pieces of 5 groups, 8.3 us unsplit);
        // 0: pieces keep >= 32 groups
        c.max_split = tpc > 2.0 && tpc <= 5.0 ? 4 : 0;
        return c;
    }
    // General rule (measured before the line-wise loads): one activation row: 10
    // groups per wave at K <= 8192, 6 above; two rows: 8; three or four: 4.
    // Waves: every chunk of the tile at once up to 8, then about a third of the
    // chunks (each wave loops), at most 16.
    c.gpw = rows == 1 ? (NG <= 64 ? 10 : 6) : rows == 2 ? 8 : 4;
    if (c.gpw > ng_even) c.gpw = ng_even;
    const int nc = (NG + c.gpw - 1) / c.gpw;
    int w = (nc + 2) / 3;
    w = w > 8 ? w : 8;
    w = w < nc ? w : nc;
    c.waves = w < kGemvMaxWaves ? w : kGemvMaxWaves;
    c.max_split = 0;
    return c;
}

bool gemv_cfg_valid(const GemvCfg& c, int K) {
    const int NG = K / kGroup;
    if (c.gpw < 2 || c.gpw > 12 || (c.gpw & 1)) return false;
    const int nc = (NG + c.gpw - 1) / c.gpw;
    return c.waves >= 1 && c.waves <= kGemvMaxWaves && c.waves <= nc && c.max_split >= 0 && c.max_split <= kGemvMaxSplit &&
           (c.rb == 1 || c.rb == 2);
}

GemvSplit gemv_split(int N, int K, const GemvCfg& c, int cus) {
    // Whole tiles (16*rb rows) in a multiple of the CU count; the remaining tiles are
    // cut along K into S pieces, about one piece per CU, so every CU streams the
    // same number of weight bytes (a round of whole tiles with a few tiles left
    // over would otherwise run at a fraction of the machine).  The combine costs a
    // round trip through L2, which only pays for deep K: by default a piece keeps
    // at least 32 groups (K = 17408 gains ~25%, K = 5120 loses ~5% when split).
    GemvSplit sp{};
    const int ntiles = (N + 16 * c.rb - 1) / (16 * c.rb);
    if (c.dot) {                // the dot-product form is never split (nor is the fused
        sp.full = ntiles;       // MFMA form that stands in for it)
        sp.S = 1;
        return sp;
    }
    const int NC = (K / kGroup + c.gpw - 1) / c.gpw;
    cus = cus > 0 ? cus : 256;
    sp.full = ntiles / cus * cus;
    sp.nrem = ntiles - sp.full;
    sp.S = 1;
    if (sp.nrem > 0) {
        int S = cus / sp.nrem;
        S = S < NC ? S : NC;
        const int cap = c.max_split > 0 ? c.max_split : (K / kGroup) / 32;
        S = S < cap ? S : cap;
        sp.S = S > 1 ? S : 1;
    }
    if (sp.S == 1) {            // nothing to split: all tiles whole
        sp.full = ntiles;
        sp.nrem = 0;
    }
    return sp;
}

size_t gemv_part_bytes(const GemvSplit& sp, int rows, int rb) {
    return (size_t)sp.nrem * sp.S * rb * rows * 16 * sizeof(float);
}

hipError_t launch_gemv_w4a8(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, const float* xf, int rows, int N, int K,
                            const GemvCfg& cfg, const GemvSplit& sp, hipStream_t st) {
    if (cfg.dot && !xf && rows == 1) {
        if (dot_inst(cfg.dot, K) > kDotMaxInst || K % 256 || K / kGroup > 64) return hipErrorInvalidValue;
        if (cfg.dot == 2)
            return gsum ? launch_dot<2, true>(y, gsum, wq, ws, xq, sa, N, K, kGemvDotWaves, st)
                        : launch_dot<2, false>(y, gsum, wq, ws, xq, sa, N, K, kGemvDotWaves, st);
        return gsum ? launch_dot<1, true>(y, gsum, wq, ws, xq, sa, N, K, kGemvDotWaves, st)
                    : launch_dot<1, false>(y, gsum, wq, ws, xq, sa, N, K, kGemvDotWaves, st);
    }
    if (xf)  // the exact group sums are a test hook of the pre-quantized form only
        return gsum ? hipErrorInvalidValue
                    : launch_rows<false, true>(y, gsum, wq, ws, xq, sa, xf, rows, N, K, cfg, sp, st);
    return gsum ? launch_rows<true, false>(y, gsum, wq, ws, xq, sa, xf, rows, N, K, cfg, sp, st)
                : launch_rows<false, false>(y, gsum, wq, ws, xq, sa, xf, rows, N, K, cfg, sp, st);
}

}  // namespace rt4
