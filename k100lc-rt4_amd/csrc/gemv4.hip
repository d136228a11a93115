// gemv4.hip -- RT4 W4A4 decode GEMV for M = 1..4 rows on gfx950 matrix cores.
//
//   y[m][n] = Σ_j f16(ws[n][j/4]) * sa[m][j] * I[m][n][j],
//   I[m][n][j] = Σ_{k in 32-subgroup j} code[n][k] * acode[m][k]   (exact int32)
//
// Restates gemv_w4a4 (kernels/gemv_w4a4_core.h:47-132) as called by k_gemv_w4a4
// (src/k_gemv.hip:14-42): weights per 128-group scale, activations int4 with one
// scale per 32 elements.  The weight stream is the W4A8 GEMV's (a workgroup owns
// a 16-row tile, its waves split K in chunks of GPW groups, one dwordx4 load
// covers 8 rows x 128 B, the x16 nibble unpack).  What differs is the activation
// operand: the 32-element subgroups carry separate scales, so the A operand of
// v_mfma_i32_16x16x64_i8 is block-diagonal.  Lane (j, q) supplies operand row
// j = 4s + m (row m of subgroup s) for k-block q, non-zero only when s == q; in
// the two MFMAs of a 128-group, k-block q is exactly the two halves of subgroup
// q.  The result lane (n, G) then holds, for every row m, the sum over subgroup
// G alone (acc[m] = 256·I[m][n][4g+G]: both operands x16), which the lane folds
// with its own subgroup's scale; the four subgroup lanes of a row are summed
// once at the end.  Every per-term product equals the reference's
// (ws*sa)*I bit for bit (the 1/256 is an exact power of two); only the order of
// the sums differs.
//
// Activation codes and scales of a chunk (M rows x GPW groups) arrive with one
// whole-wave load each -- per-group loads with 16 active lanes cost ~3 us at the
// 27B gate/up shape -- and are redistributed through a wave-private LDS slice:
// codes [row][group][subgroup] in 16-byte slots plus a zero slot that the lanes
// off the block diagonal read, scales [row][group][subgroup] as floats.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ uint32_t dpp4(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

constexpr int kA4Slots = 4 * 4 * 4;    // 16-byte code slots per wave: [row][group][subgroup], M, GPW <= 4

template <int M, int GPW>
__global__ __launch_bounds__(1024) void gemv_w4a4_k(const uint32_t* __restrict__ wq,
                                                    const uint16_t* __restrict__ ws,
                                                    const uint32_t* __restrict__ aq,
                                                    const float* __restrict__ sa,
                                                    float* __restrict__ y, int N, int K, GemvSplit sp) {
    static_assert(GPW == 2 || GPW == 4, "a chunk's activations: at most one 16-byte slot per lane");
    constexpr int NP = GPW / 2;                  // group pairs per wave
    extern __shared__ __align__(16) unsigned char smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int NG = K >> 7, RS = K >> 1, KD = K >> 3, NS = K >> 5;
    const int NC = (NG + GPW - 1) / GPW;
    // Workgroups [0, npieces) each take one K range of a remainder tile; the rest
    // take whole tiles (the W4A8 GEMV's split, gemv_split).
    const int b = blockIdx.x, npieces = sp.nrem * sp.S;
    const bool piece = b < npieces;
    const int rem = piece ? b / sp.S : 0, pc = piece ? b % sp.S : 0;
    const int tile = piece ? sp.full + rem : b - npieces;
    const int c_lo = piece ? pc * NC / sp.S : 0, c_hi = piece ? (pc + 1) * NC / sp.S : NC;
    const int n0 = tile * 16;
    // LDS: [W] weight-scale slices ([16 rows][GPW/2] dwords), [W] code slices
    // (kA4Slots + 1 zero slot, 16 B each), [W] scale slices (kA4Slots floats), then
    // the reduction area [W][M][16]
    unsigned char* base = smem;
    uint32_t* wsl = reinterpret_cast<uint32_t*>(base) + (size_t)w * 8 * GPW;
    base += (size_t)W * 16 * GPW * 2;
    uint4* acl = reinterpret_cast<uint4*>(base) + (size_t)w * (kA4Slots + 1);
    base += (size_t)W * (kA4Slots + 1) * 16;
    float* asl = reinterpret_cast<float*>(base) + (size_t)w * kA4Slots;
    base += (size_t)W * kA4Slots * sizeof(float);
    float* red = reinterpret_cast<float*>(base);
    if (lane == 0) acl[kA4Slots] = make_uint4(0, 0, 0, 0);

    // weight loads: the mapping of the W4A8 GEMV (two instructions per group
    // pair, 8 rows x 128 B each; the first group of the pair is sel(j<8 ? inst1 :
    // inst2), the second ror8(sel(j<8 ? inst2 : inst1)))
    const bool lo = j < 8;
    int r1 = n0 + (lo ? j : j - 8), r2 = n0 + (lo ? j + 8 : j);
    r1 = r1 < N ? r1 : N - 1;
    r2 = r2 < N ? r2 : N - 1;
    const unsigned char* p1 = reinterpret_cast<const unsigned char*>(wq) + (size_t)r1 * RS + (lo ? q : 4 + q) * 16;
    const unsigned char* p2 = reinterpret_cast<const unsigned char*>(wq) + (size_t)r2 * RS + (lo ? 4 + q : q) * 16;
    const int rj = n0 + j < N ? n0 + j : N - 1;
    // activation operand of this lane: row am of subgroup q, used iff j/4 == q;
    // for group u it is slot (am*GPW + u)*4 + q, the zero slot off the diagonal
    const int am = j & 3;
    const bool aon = (j >> 2) == q && am < M;
    // the chunk's load: lane l < 4*GPW*M takes row l/(4 GPW), group (l/4)%GPW, subgroup l%4
    const int lr = lane / (4 * GPW), lu = (lane >> 2) % GPW, ls = lane & 3;
    const bool lon = lane < 4 * GPW * M;
    const uint32_t* lrow = aq + (size_t)(lon ? lr : 0) * KD + 4 * ls;   // + 16 g
    const float* lsrow = sa + (size_t)(lon ? lr : 0) * NS + ls;         // + 4 g
    // this lane's scale in the fold layout (lane 16G + r: row r, subgroup G)
    const int sslot = j < M ? (j * GPW) * 4 + q : -1;                    // + 4 u
    const v4i zero = {0, 0, 0, 0};

    float yacc[M];
#pragma unroll
    for (int r = 0; r < M; r++) yacc[r] = 0.f;

    for (int c = c_lo + w; c < c_hi; c += W) {
        const int g0 = uniform(c * GPW);
        // (1) weight scales of this wave: 16 rows x GPW fp16, as dwords (even NG)
        //     or as halves (odd NG)
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
        // (2) activation codes and scales of the chunk: one slot / one float per lane
        uint4 lcode = make_uint4(0, 0, 0, 0);
        float lscale = 0.f;
        {
            int g = g0 + lu;
            g = g < NG ? g : NG - 1;
            if (lon) {
                lcode = *reinterpret_cast<const uint4*>(lrow + 16 * g);
                lscale = lsrow[4 * g];
            }
        }
        // (3) the weight stream
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
        // redistribute the chunk's activations (wave-private slices: the LDS
        // operations of one wave complete in order, no barrier)
        if (lon) {
            acl[lane] = lcode;
            asl[lane] = lscale;
        }
        uint4 av[GPW];
        float as[GPW];
#pragma unroll
        for (int u = 0; u < GPW; u++) {
            av[u] = acl[aon ? (am * GPW + u) * 4 + q : kA4Slots];
            const float sv = asl[(sslot >= 0 ? sslot : 0) + 4 * u];
            as[u] = sslot >= 0 ? sv : 0.f;
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
            t1.x = dpp4<0x128>(x.x);
            t1.y = dpp4<0x128>(x.y);
            t1.z = dpp4<0x128>(x.z);
            t1.w = dpp4<0x128>(x.w);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int u = 2 * p + h, g = g0 + u;
                const v4u qv = h ? t1 : t0;
                const uint4 xa = av[u];
                const v4i A0 = {(int)even_x16(xa.x), (int)odd_x16(xa.x), (int)even_x16(xa.y), (int)odd_x16(xa.y)};
                const v4i A1 = {(int)even_x16(xa.z), (int)odd_x16(xa.z), (int)even_x16(xa.w), (int)odd_x16(xa.w)};
                const v4i b0 = {(int)even_x16(qv.x), (int)odd_x16(qv.x), (int)even_x16(qv.y), (int)odd_x16(qv.y)};
                const v4i b1 = {(int)even_x16(qv.z), (int)odd_x16(qv.z), (int)even_x16(qv.w), (int)odd_x16(qv.w)};
                v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, b0, zero, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, b1, acc, 0, 0, 0);
                // lane (n, G) holds 256·I[m][n0+n][4g+G] in acc[m]
                if (g < NG) {
                    const uint32_t pair = wsl[j * (GPW / 2) + p];
                    const float s256 = f16_bits_to_f32((uint16_t)(h ? pair >> 16 : pair & 0xFFFFu)) * (1.f / 256.f);
                    const uint32_t asb = __float_as_uint(as[u]);
                    float a_s[4];
                    // the scale of (row r, subgroup G) sits in lane r of this lane's 16-lane row
                    a_s[0] = __uint_as_float(dpp4<0x150>(asb));
                    a_s[1] = __uint_as_float(dpp4<0x151>(asb));
                    a_s[2] = __uint_as_float(dpp4<0x152>(asb));
                    a_s[3] = __uint_as_float(dpp4<0x153>(asb));
#pragma unroll
                    for (int r = 0; r < M; r++) yacc[r] = fmaf((float)acc[r], s256 * a_s[r], yacc[r]);
                }
            }
        }
    }

    // the four subgroup lanes of each output row, then the waves of the tile
#pragma unroll
    for (int r = 0; r < M; r++) {
        yacc[r] += __shfl_xor(yacc[r], 16);
        yacc[r] += __shfl_xor(yacc[r], 32);
    }
    if (lane < 16)
#pragma unroll
        for (int r = 0; r < M; r++) red[(w * M + r) * 16 + lane] = yacc[r];
    __syncthreads();
    const int cl = threadIdx.x & 15, rr = threadIdx.x >> 4;
    const bool out = threadIdx.x < M * 16;
    float tot = 0.f;
    if (out)
        for (int v = 0; v < W; v++) tot += red[(v * M + rr) * 16 + cl];
    if (!piece) {
        if (out && n0 + cl < N) y[(size_t)rr * N + n0 + cl] = tot;
        return;
    }
    // A K range of a split tile: publish the partial, count the pieces in; the
    // last one sums all pieces in order and resets the counter for the next call.
    __shared__ int s_last;
    if (out) store_dev(sp.part + (size_t)b * M * 16 + threadIdx.x, tot);
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(sp.cnt + rem, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == sp.S - 1;
    __syncthreads();
    if (!s_last) return;
    if (out) {
        float sum = 0.f;
        for (int v = 0; v < sp.S; v++) sum += load_dev(sp.part + (size_t)(rem * sp.S + v) * M * 16 + threadIdx.x);
        if (n0 + cl < N) y[(size_t)rr * N + n0 + cl] = sum;
    }
    if (threadIdx.x == 0) __hip_atomic_store(sp.cnt + rem, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int M, int GPW>
hipError_t launch_g4(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa, int N,
                     int K, int waves, const GemvSplit& sp, hipStream_t st) {
    const size_t smem = (size_t)waves * 16 * GPW * 2 + (size_t)waves * (kA4Slots + 1) * 16 +
                        (size_t)waves * kA4Slots * sizeof(float) + (size_t)waves * M * 16 * sizeof(float);
    const int grid = sp.full + sp.nrem * sp.S;
    hipLaunchKernelGGL((gemv_w4a4_k<M, GPW>), dim3(grid), dim3(64 * waves), smem, st, wq, ws, aq, sa, y, N, K, sp);
    return hipGetLastError();
}

template <int M>
hipError_t launch_m4(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa, int N,
                     int K, const GemvCfg& c, const GemvSplit& sp, hipStream_t st) {
    const int NC = (K / 128 + c.gpw - 1) / c.gpw;
    const int waves = c.waves < NC ? c.waves : NC;
    return c.gpw == 2 ? launch_g4<M, 2>(y, wq, ws, aq, sa, N, K, waves, sp, st)
                      : launch_g4<M, 4>(y, wq, ws, aq, sa, N, K, waves, sp, st);
}

}  // namespace

GemvCfg gemv4_default_cfg(int rows, int N, int K, int cus) {
    (void)rows;
    (void)K;
    cus = cus > 0 ? cus : 256;
    const double tpc = (double)((N + 15) / 16) / cus;   // 16-row tiles per CU
    // Measured bands of tiles per CU (MI355X, K = 5120 unless noted, us, this
    // choice vs the next best): up to 2, 16 waves and deep-K pieces (N = 5120 at
    // K = 17408: 11.0 vs 12.0); up to 3.5, 8 waves and at most 4 pieces per
    // leftover tile (N = 8704: 7.6 vs 8.3 whole, 9.4 with 8 pieces); up to 5,
    // 4 waves and 4 pieces (N = 17408: 11.4 vs 12.2); up to 40, 8 waves, tiles
    // whole (N = 34816: 19.5 vs 19.8); beyond, four groups per wave and 4 waves
    // (N = 248320: 116 vs 117-119).
    if (tpc <= 2.0) return GemvCfg{2, 16, 0, 1};
    if (tpc <= 3.5) return GemvCfg{2, 8, 4, 1};
    if (tpc <= 5.0) return GemvCfg{2, 4, 4, 1};
    if (tpc <= 40.0) return GemvCfg{2, 8, 1, 1};
    return GemvCfg{4, 4, 0, 1};
}

bool gemv4_cfg_valid(const GemvCfg& c) {
    return (c.gpw == 2 || c.gpw == 4) && c.waves >= 1 && c.waves <= kGemvMaxWaves && c.max_split >= 0 &&
           c.max_split <= kGemvMaxSplit && c.rb == 1;
}

hipError_t launch_gemv_w4a4(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa,
                            int rows, int N, int K, const GemvCfg& c, const GemvSplit& sp, hipStream_t st) {
    switch (rows) {
        case 1: return launch_m4<1>(y, wq, ws, aq, sa, N, K, c, sp, st);
        case 2: return launch_m4<2>(y, wq, ws, aq, sa, N, K, c, sp, st);
        case 3: return launch_m4<3>(y, wq, ws, aq, sa, N, K, c, sp, st);
        case 4: return launch_m4<4>(y, wq, ws, aq, sa, N, K, c, sp, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace rt4
