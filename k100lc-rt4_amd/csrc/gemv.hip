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
// * Work split: a workgroup owns one 16-row weight tile; its W waves split the
//   K groups of that tile, GPW groups (an even number) each.  Every wave issues
//   all of its loads up front; W*GPW*16 rows x 64 B is the tile's full K.
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
// * Activations: loaded straight into registers, 16/M groups per register set
//   (lane j holds row j%M of group j/M), and rotated into lanes 0..M-1 for the
//   group being multiplied with DPP row_ror.
// * Weight scales: each wave loads its 16 rows x GPW fp16 scales as dwords into
//   a private LDS slice.  Scales and activations are issued before the weight
//   stream: vmcnt retires in order, so the first group can start as soon as its
//   weights land.
// * fp32 fold once per group: fp32(16I) * (f16(ws)/16 * sa) equals the
//   reference's (ws*sa)*I term bit for bit (power-of-two scaling is exact); only
//   the order of the sum over groups differs from the reference.  The W partial
//   sums of a tile are reduced through LDS.
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

template <int M, int GPW, bool GSUM>
__global__ __launch_bounds__(1024) void gemv_w4a8_k(const uint32_t* __restrict__ wq,
                                                    const uint16_t* __restrict__ ws,
                                                    const int8_t* __restrict__ xq,
                                                    const float* __restrict__ sa,
                                                    float* __restrict__ y,
                                                    int32_t* __restrict__ gsum, int N, int K) {
    constexpr int GPS = 16 / M;                  // groups per activation register set
    constexpr int NSET = (GPW + GPS - 1) / GPS;
    constexpr int NP = GPW / 2;                  // group pairs per wave
    extern __shared__ __align__(16) unsigned char smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int NG = K >> 7, RS = K >> 1;          // groups and bytes per weight row
    const int NC = (NG + GPW - 1) / GPW;         // group chunks per tile
    const int n0 = blockIdx.x * 16;
    // scale slice of this wave: [16 rows][GPW/2] dwords (fp16 pairs), then the
    // reduction area; always accessed as dwords
    uint32_t* wsl = reinterpret_cast<uint32_t*>(smem) + (size_t)w * 8 * GPW;
    float* red = reinterpret_cast<float*>(smem + (size_t)W * 16 * GPW * 2);

    // Load mapping of a group pair (rows n0..n0+15, 128 B each):
    //   instruction 1 covers rows 0-7, instruction 2 rows 8-15, 8 lanes per row;
    //   lane (j<8, q):  inst1 = (row j,    chunk q),   inst2 = (row j+8, chunk 4+q)
    //   lane (j>=8, q): inst1 = (row j-8,  chunk 4+q), inst2 = (row j,   chunk q)
    // so the first group of the pair is sel(j<8 ? inst1 : inst2) and the second
    // is ror8(sel(j<8 ? inst2 : inst1)).
    const bool lo = j < 8;
    int r1 = n0 + (lo ? j : j - 8), r2 = n0 + (lo ? j + 8 : j);
    r1 = r1 < N ? r1 : N - 1;                    // tail rows read a valid row; dropped
    r2 = r2 < N ? r2 : N - 1;
    const unsigned char* p1 = reinterpret_cast<const unsigned char*>(wq) + (size_t)r1 * RS + (lo ? q : 4 + q) * 16;
    const unsigned char* p2 = reinterpret_cast<const unsigned char*>(wq) + (size_t)r2 * RS + (lo ? 4 + q : q) * 16;
    const int rj = n0 + j < N ? n0 + j : N - 1;
    const int jr = j % M, jg = j / M;
    const v4i zero = {0, 0, 0, 0};

    float yacc[M];
#pragma unroll
    for (int r = 0; r < M; r++) yacc[r] = 0.f;

    for (int c = w; c < NC; c += W) {
        const int g0 = uniform(c * GPW);
        // (1) this wave's scales: 16 rows x GPW fp16, as dwords (even NG: every
        //     row starts 4-byte aligned) or as halves (odd NG)
        uint32_t sw[(GPW / 2 + 3) / 4];
#pragma unroll
        for (int d = 0; d < (GPW / 2 + 3) / 4; d++) {
            const int dw = q + 4 * d;
            const int g = g0 + 2 * dw;
            const uint16_t* sp = ws + (size_t)rj * NG;
            uint32_t v = 0;
            if (dw < GPW / 2 && g < NG) {
                if (!(NG & 1))
                    v = *reinterpret_cast<const uint32_t*>(sp + g);
                else
                    v = (uint32_t)sp[g] | (g + 1 < NG ? (uint32_t)sp[g + 1] << 16 : 0u);
            }
            sw[d] = v;
        }
        // (2) activations: set s, lane j holds row j%M of group g0 + s*GPS + j/M
        uint4 ax0[NSET], ax1[NSET];
#pragma unroll
        for (int s = 0; s < NSET; s++) {
            int g = g0 + s * GPS + jg;
            g = g < NG ? g : NG - 1;
            const uint4* ap = reinterpret_cast<const uint4*>(xq + (size_t)jr * K + (size_t)g * 128 + q * 32);
            ax0[s] = ap[0];
            ax1[s] = ap[1];
        }
        // (3) the weight stream.  A pair starting at the last group of an odd NG
        //     has no second group: its lanes read the first group again (in bounds)
        //     and that result is never used.
        v4u a[NP], b[NP];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            int gp = g0 + 2 * p;
            if (gp >= NG) gp = NG >= 2 ? NG - 2 : 0;
            const int tail = (gp + 1 >= NG) ? 64 : 0;
            a[p] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p1 + (size_t)gp * 64 - (lo ? 0 : tail)));
            b[p] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p2 + (size_t)gp * 64 - (lo ? tail : 0)));
        }
#pragma unroll
        for (int d = 0; d < (GPW / 2 + 3) / 4; d++) {
            const int dw = q + 4 * d;
            if (dw < GPW / 2) wsl[j * (GPW / 2) + dw] = sw[d];
        }

#pragma unroll
        for (int p = 0; p < NP; p++) {
            v4u t0, x;
            t0.x = lo ? a[p].x : b[p].x;
            t0.y = lo ? a[p].y : b[p].y;
            t0.z = lo ? a[p].z : b[p].z;
            t0.w = lo ? a[p].w : b[p].w;
            x.x = lo ? b[p].x : a[p].x;
            x.y = lo ? b[p].y : a[p].y;
            x.z = lo ? b[p].z : a[p].z;
            x.w = lo ? b[p].w : a[p].w;
            v4u t1;
            t1.x = dpp<0x128>(x.x);
            t1.y = dpp<0x128>(x.y);
            t1.z = dpp<0x128>(x.z);
            t1.w = dpp<0x128>(x.w);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int u = 2 * p + h, g = g0 + u;
                const v4u qv = h ? t1 : t0;
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
                const v4i b0 = {(int)even_x16(qv.x), (int)odd_x16(qv.x), (int)even_x16(qv.y), (int)odd_x16(qv.y)};
                const v4i b1 = {(int)even_x16(qv.z), (int)odd_x16(qv.z), (int)even_x16(qv.w), (int)odd_x16(qv.w)};
                v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, zero, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, acc, 0, 0, 0);
                // lane l < 16 now holds 16*I[m=r][n0+l] in acc[r]
                if (g < NG) {
                    if (GSUM && lane < 16 && n0 + lane < N)
#pragma unroll
                        for (int r = 0; r < M; r++) gsum[((size_t)r * N + n0 + lane) * NG + g] = acc[r] >> 4;
                    const uint32_t pair = wsl[j * (GPW / 2) + p];
                    const float s16 = f16_bits_to_f32((uint16_t)(h ? pair >> 16 : pair & 0xFFFFu)) * 0.0625f;
#pragma unroll
                    for (int r = 0; r < M; r++) yacc[r] = fmaf((float)acc[r], s16 * sa[(size_t)r * NG + g], yacc[r]);
                }
            }
        }
    }

    if (W == 1) {
        if (lane < 16 && n0 + lane < N)
#pragma unroll
            for (int r = 0; r < M; r++) y[(size_t)r * N + n0 + lane] = yacc[r];
        return;
    }
    if (lane < 16)
#pragma unroll
        for (int r = 0; r < M; r++) red[(w * M + r) * 16 + lane] = yacc[r];
    __syncthreads();
    if (threadIdx.x < M * 16) {
        const int cl = threadIdx.x & 15, r = threadIdx.x >> 4;
        float s = 0.f;
        for (int v = 0; v < W; v++) s += red[(v * M + r) * 16 + cl];
        if (n0 + cl < N) y[(size_t)r * N + n0 + cl] = s;
    }
}

template <int M, int GPW, bool GSUM>
hipError_t launch_one(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                      const float* sa, int N, int K, int waves, hipStream_t st) {
    const size_t smem = (size_t)waves * 16 * GPW * 2 + (size_t)waves * M * 16 * sizeof(float);
    hipLaunchKernelGGL((gemv_w4a8_k<M, GPW, GSUM>), dim3((N + 15) / 16), dim3(64 * waves), smem, st, wq, ws,
                       xq, sa, y, gsum, N, K);
    return hipGetLastError();
}

template <int M, bool GSUM>
hipError_t launch_m(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                    const float* sa, int N, int K, const GemvCfg& c, hipStream_t st) {
    switch (c.gpw) {
        case 2: return launch_one<M, 2, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
        case 4: return launch_one<M, 4, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
        case 6: return launch_one<M, 6, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
        case 8: return launch_one<M, 8, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
        case 10: return launch_one<M, 10, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
        case 12: return launch_one<M, 12, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

GemvCfg gemv_default_cfg(int rows, int N, int K) {
    (void)rows;
    (void)N;
    const int NG = K / kGroup;
    GemvCfg c;
    // measured on MI355X: ~10 groups per wave for the 27B shapes (K = 5120: 4
    // waves per tile; K = 17408: 12 groups -> 12 waves); at most 16 waves, larger
    // K loops over group chunks inside each wave.
    c.gpw = NG >= 120 ? 12 : 10;
    const int ng_even = (NG + 1) & ~1;
    if (c.gpw > ng_even) c.gpw = ng_even;
    int nc = (NG + c.gpw - 1) / c.gpw;
    c.waves = nc < kGemvMaxWaves ? nc : kGemvMaxWaves;
    return c;
}

bool gemv_cfg_valid(const GemvCfg& c, int K) {
    const int NG = K / kGroup;
    if (c.gpw < 2 || c.gpw > 12 || (c.gpw & 1)) return false;
    const int nc = (NG + c.gpw - 1) / c.gpw;
    return c.waves >= 1 && c.waves <= kGemvMaxWaves && c.waves <= nc;
}

hipError_t launch_gemv_w4a8(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, int rows, int N, int K,
                            const GemvCfg& cfg, hipStream_t st) {
    if (gsum) {
        switch (rows) {
            case 1: return launch_m<1, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 2: return launch_m<2, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 3: return launch_m<3, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 4: return launch_m<4, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
        }
    } else {
        switch (rows) {
            case 1: return launch_m<1, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 2: return launch_m<2, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 3: return launch_m<3, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 4: return launch_m<4, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace rt4
