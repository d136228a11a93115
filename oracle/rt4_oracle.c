/*
 * rt4_oracle.c -- CPU restatement of K100LC-RT4's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels are
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function restates one piece of the reference's arithmetic and cites
 * the reference file:line it follows (paths relative to the reference root).
 * Floating-point steps that decide integer codes use the same IEEE single
 * operations as the reference kernels (correctly rounded division, lrintf
 * round-half-to-even under the default rounding mode, fmaxf/fabsf), so the
 * codes are bit-identical.  Build with -ffp-contract=off: nothing here may be
 * fused into an FMA.
 *
 * Pinning (what checks each function independently of this file):
 *   rt4o_dot8_i4        v_dot8 known-answer values, bench/bench_isa2.cpp:128-145
 *   rt4o_code           same KAT + the reference converter's own output
 *                       (tools/convert.c built in oracle/_ref) on a known input
 *   rt4o_f16_to_f32     exhaustive check against numpy.float16 (textbook IEEE)
 *   rt4o_quant_act      closed form + invariants (|q|<=127, argmax -> +-127,
 *                       zero group -> s=1,q=0) + numpy restatement + reference
 *                       GPU build when present
 *   rt4o_quant_rows_a8  closed form + 16h+l == q8 identity + reference GPU build
 *   rt4o_quant_rows_a4  closed form + reference GPU build
 *   rt4o_gemv_*         brute-force integer dot, Σu·a-8Σa identity
 *                       (kernels/gemv_int4.hip:317-336), fp64 fold
 *   rt4o_gemm_*         per-group int = 16*I_h + I_l identity, fp64 fold as in
 *                       bench/int4_gemm2.cpp:104-123
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define RT4O_GROUP 128

/* ------------------------------------------------------------------ codes -- */

/* IEEE binary16 bit pattern -> float.  Same decode as tools/rt4_io.py:8-18 and
 * src/model.cpp:194-199 (sign, 5-bit exponent, 10-bit mantissa, subnormals). */
float rt4o_f16_to_f32(uint16_t h) {
    const uint32_t sg = (h >> 15) & 1u, ex = (h >> 10) & 0x1Fu, ma = h & 0x3FFu;
    float f;
    if (ex == 0)
        f = ldexpf((float)ma / 1024.f, -14);
    else if (ex == 31)
        f = ma ? NAN : INFINITY;
    else
        f = ldexpf(1.f + (float)ma / 1024.f, (int)ex - 15);
    return sg ? -f : f;
}

/* Signed int4 code of element k in an RT4 packed row: dword k/8, nibble k%8,
 * low nibble first, two's complement (docs/FORMAT.md:61-73; packer
 * kernels/gemm_core.h:35-39; writer tools/convert.c:355-360). */
int rt4o_code(const uint32_t* row, int k) {
    const int v = (int)((row[k >> 3] >> (4 * (k & 7))) & 0xFu);
    return v >= 8 ? v - 16 : v;
}

/* Semantics of v_dot8_i32_i4: eight signed nibble products, low nibble first,
 * summed into one int32 (bench/bench_isa2.cpp:128-145, docs/DESIGN-INT4.md:40-44). */
int32_t rt4o_dot8_i4(uint32_t a, uint32_t b, int32_t acc) {
    for (int e = 0; e < 8; e++) {
        int x = (int)((a >> (4 * e)) & 0xFu), y = (int)((b >> (4 * e)) & 0xFu);
        if (x >= 8) x -= 16;
        if (y >= 8) y -= 16;
        acc += x * y;
    }
    return acc;
}

/* Pack 8 int4 codes (low nibble = first) -- kernels/gemm_core.h:35-39. */
uint32_t rt4o_pack8(const int8_t* q) {
    uint32_t w = 0;
    for (int i = 0; i < 8; i++) w |= (uint32_t)(q[i] & 0xF) << (4 * i);
    return w;
}

/* ------------------------------------------------------------- quantizers -- */

/* Decode-side activation quantizer, kernels/gemv_w4a8_core.h:34-66.
 * Per (row m, 128-group g): amax = max|x|, s = amax>0 ? amax/127 : 1,
 * q = clamp(lrintf(x/s), -128, 127), asu = Σq.
 * q is written in natural k order [M][K] (the reference splits it into even/odd
 * halves; that split is a storage detail of its GEMV, not of the codes). */
void rt4o_quant_act(const float* x, int M, int K, int8_t* q, float* sa, int32_t* asu) {
    const int NG = K / RT4O_GROUP;
    for (int m = 0; m < M; m++)
        for (int g = 0; g < NG; g++) {
            const float* src = x + (size_t)m * K + (size_t)g * RT4O_GROUP;
            float amax = 0.f;
            for (int i = 0; i < RT4O_GROUP; i++) amax = fmaxf(amax, fabsf(src[i]));
            const float s = amax > 0.f ? amax / 127.f : 1.f;
            int32_t part = 0;
            for (int i = 0; i < RT4O_GROUP; i++) {
                const float v = src[i] / s;
                int c = (int)lrintf(v);
                c = c > 127 ? 127 : (c < -128 ? -128 : c);
                part += c;
                q[(size_t)m * K + (size_t)g * RT4O_GROUP + i] = (int8_t)c;
            }
            sa[(size_t)m * NG + g] = s;
            if (asu) asu[(size_t)m * NG + g] = part;
        }
}

/* Prefill-side 8-bit quantizer split into two int4 digits, src/k_new.hip:268-301.
 * Per (row, G-group): s = amax>0 ? amax/119 : 1; q8 = clamp(lrintf(x/s), -128, 119);
 * h = (q8+8)>>4 (arithmetic shift = floor), l = q8 - 16h; both packed like RT4
 * weights into qh/ql [rows][K/8]; sc[g][row] = s, sc16[g][row] = 16s (group-major).
 * in_stride == 0 means K (src/k_new.hip:298). */
void rt4o_quant_rows_a8(const float* x, int rows, int K, int G, int in_stride, int in_off,
                        uint32_t* qh, uint32_t* ql, float* sc, float* sc16) {
    if (in_stride == 0) in_stride = K;
    const int NG = K / G;
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < NG; g++) {
            const float* xr = x + (size_t)r * in_stride + in_off + (size_t)g * G;
            float amax = 0.f;
            for (int i = 0; i < G; i++) amax = fmaxf(amax, fabsf(xr[i]));
            const float s = amax > 0.f ? amax / 119.f : 1.f;
            sc[(size_t)g * rows + r] = s;
            sc16[(size_t)g * rows + r] = s * 16.f;
            for (int i = 0; i < G; i += 8) {
                uint32_t wh = 0, wl = 0;
                for (int e = 0; e < 8; e++) {
                    int q8 = (int)lrintf(xr[i + e] / s);
                    q8 = q8 > 119 ? 119 : (q8 < -128 ? -128 : q8);
                    const int h = (q8 + 8) >> 4;
                    const int l = q8 - 16 * h;
                    wh |= (uint32_t)(h & 0xF) << (4 * e);
                    wl |= (uint32_t)(l & 0xF) << (4 * e);
                }
                const size_t d = (size_t)r * (K / 8) + (size_t)(g * G + i) / 8;
                qh[d] = wh;
                ql[d] = wl;
            }
        }
}

/* Same quantizer, but the int8 code itself in natural order (q8 = 16h + l).
 * Used to state what the digits encode; not a reference function. */
void rt4o_quant_rows_i8(const float* x, int rows, int K, int G, int in_stride, int in_off,
                        int8_t* q8out, float* sc) {
    if (in_stride == 0) in_stride = K;
    const int NG = K / G;
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < NG; g++) {
            const float* xr = x + (size_t)r * in_stride + in_off + (size_t)g * G;
            float amax = 0.f;
            for (int i = 0; i < G; i++) amax = fmaxf(amax, fabsf(xr[i]));
            const float s = amax > 0.f ? amax / 119.f : 1.f;
            sc[(size_t)g * rows + r] = s;
            for (int i = 0; i < G; i++) {
                int q8 = (int)lrintf(xr[i] / s);
                q8 = q8 > 119 ? 119 : (q8 < -128 ? -128 : q8);
                q8out[(size_t)r * K + (size_t)g * G + i] = (int8_t)q8;
            }
        }
}

/* int4 activation quantizer (W4A4 A/B path), src/k_new.hip:192-219:
 * s = amax>0 ? amax/7 : 1; c = clamp(lrintf(x/s), -8, 7); packed like RT4;
 * sc[g][row] group-major. */
void rt4o_quant_rows_a4(const float* x, int rows, int K, int G, int in_stride, int in_off,
                        uint32_t* q, float* sc) {
    if (in_stride == 0) in_stride = K;
    const int NG = K / G;
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < NG; g++) {
            const float* xr = x + (size_t)r * in_stride + in_off + (size_t)g * G;
            float amax = 0.f;
            for (int i = 0; i < G; i++) amax = fmaxf(amax, fabsf(xr[i]));
            const float s = amax > 0.f ? amax / 7.f : 1.f;
            sc[(size_t)g * rows + r] = s;
            for (int i = 0; i < G; i += 8) {
                uint32_t w = 0;
                for (int e = 0; e < 8; e++) {
                    int c = (int)lrintf(xr[i + e] / s);
                    c = c > 7 ? 7 : (c < -8 ? -8 : c);
                    w |= (uint32_t)(c & 0xF) << (4 * e);
                }
                q[(size_t)r * (K / 8) + (size_t)(g * G + i) / 8] = w;
            }
        }
}

/* ------------------------------------------------------ weight quantizer -- */

/* float -> binary16 bit pattern with the reference converter's own rounding
 * (tools/convert.c:102-120).  Normal results add 0x1000 plus the kept lsb to the
 * 23-bit mantissa before truncating 13 bits, so exact ties round away from zero
 * (and one pattern just below a tie with an odd kept lsb rounds up too); this is
 * not numpy's round-to-nearest-even, and the scales must match it bit for bit. */
uint16_t rt4o_f32_to_f16_conv(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    const uint32_t s = (u >> 16) & 0x8000u;
    int32_t e = (int32_t)((u >> 23) & 0xFFu) - 127 + 15;
    uint32_t m = u & 0x7FFFFFu;
    if (((u >> 23) & 0xFFu) == 0xFFu) return (uint16_t)(s | 0x7C00u | (m ? 0x200u : 0u));
    if (e >= 0x1F) return (uint16_t)(s | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)s;
        m |= 0x800000u;
        const int sh = 14 - e;
        const uint32_t half = 1u << (sh - 1);
        return (uint16_t)(s | ((m + half - 1 + ((m >> sh) & 1u)) >> sh));
    }
    uint32_t r = m + 0x1000u + ((m >> 13) & 1u);
    if (r & 0x800000u) {
        r = 0;
        if (++e >= 0x1F) return (uint16_t)(s | 0x7C00u);
    }
    return (uint16_t)(s | ((uint32_t)e << 10) | (r >> 13));
}

/* The converter's int4 weight quantizer (tools/convert.c:338-360, bits = 4):
 * per (row, 128-group) s = amax>0 ? amax/7 : 1, stored as f16 with the rounding
 * above; q = clamp(roundf(w * (1/s)), -7, 7) with the fp32 s (not the rounded
 * f16), packed two's complement, low nibble = even k (docs/FORMAT.md:61-73).
 * w f32 [N][K] -> wq u32 [N][K/8], ws u16 [N][K/128]. */
void rt4o_quant_weight_rows(const float* w, int N, int K, uint32_t* wq, uint16_t* ws) {
    const int NG = K / RT4O_GROUP;
    for (int n = 0; n < N; n++)
        for (int g = 0; g < NG; g++) {
            const float* blk = w + (size_t)n * K + (size_t)g * RT4O_GROUP;
            float amax = 0.f;
            for (int i = 0; i < RT4O_GROUP; i++) {
                const float a = fabsf(blk[i]);
                if (a > amax) amax = a;
            }
            const float s = amax > 0.f ? amax / 7.0f : 1.0f;
            ws[(size_t)n * NG + g] = rt4o_f32_to_f16_conv(s);
            const float inv = 1.0f / s;
            for (int d = 0; d < RT4O_GROUP / 8; d++) {
                uint32_t word = 0;
                for (int e = 0; e < 8; e++) {
                    float q = roundf(blk[8 * d + e] * inv);
                    if (q > 7.f) q = 7.f;
                    if (q < -7.f) q = -7.f;
                    word |= ((uint32_t)(int)q & 0xFu) << (4 * e);
                }
                wq[(size_t)n * (K / 8) + (size_t)g * (RT4O_GROUP / 8) + d] = word;
            }
        }
}

/* RT4 row-major fp16 scales -> fp32 group-major, src/model.cpp:190-202. */
void rt4o_make_group_major(const uint16_t* ws, int N, int NG, float* out) {
    for (int n = 0; n < N; n++)
        for (int g = 0; g < NG; g++) out[(size_t)g * N + n] = rt4o_f16_to_f32(ws[(size_t)n * NG + g]);
}

/* ------------------------------------------------------------------- GEMV -- */

/* Unpack RT4 rows [n0, n1) into int8 codes [n1-n0][K]. */
static void unpack_rows(const uint32_t* wq, int K, int n0, int n1, int8_t* out) {
    const int KD = K / 8;
    for (int n = n0; n < n1; n++) {
        const uint32_t* row = wq + (size_t)n * KD;
        int8_t* o = out + (size_t)(n - n0) * K;
        for (int d = 0; d < KD; d++) {
            const uint32_t w = row[d];
            for (int e = 0; e < 8; e++) {
                const int v = (int)((w >> (4 * e)) & 0xFu);
                o[8 * d + e] = (int8_t)(v >= 8 ? v - 16 : v);
            }
        }
    }
}

/* Exact per-group integer dot products of the W4A8 GEMV:
 * I[m][n][g] = Σ_{k in group g} code[n][k] * q[m][k].  This is the quantity
 * gemv_w4a8 forms as Σu·a - 8·Σa with u = code+8 (kernels/gemv_w4a8_core.h:
 * 149-150, 165-168, 194); the identity Σu·a - 8Σa == Σcode·a is exact.
 * Rows are processed in parallel when built with OpenMP. */
void rt4o_gemv_groupsums(const uint32_t* wq, const int8_t* q, int M, int N, int K, int32_t* I) {
    const int NG = K / RT4O_GROUP;
    const int CH = 64;
#pragma omp parallel for schedule(dynamic, 1)
    for (int n0 = 0; n0 < N; n0 += CH) {
        const int n1 = n0 + CH < N ? n0 + CH : N;
        int8_t* codes = (int8_t*)malloc((size_t)(n1 - n0) * K);
        unpack_rows(wq, K, n0, n1, codes);
        for (int n = n0; n < n1; n++) {
            const int8_t* c = codes + (size_t)(n - n0) * K;
            for (int m = 0; m < M; m++) {
                const int8_t* a = q + (size_t)m * K;
                for (int g = 0; g < NG; g++) {
                    int32_t s = 0;
                    for (int i = 0; i < RT4O_GROUP; i++)
                        s += (int32_t)c[g * RT4O_GROUP + i] * (int32_t)a[g * RT4O_GROUP + i];
                    I[((size_t)m * N + n) * NG + g] = s;
                }
            }
        }
        free(codes);
    }
}

/* fp64 fold of the GEMV: y[m][n] = Σ_g f16(ws[n][g]) * sa[m][g] * I[m][n][g]
 * (kernels/gemv_w4a8_core.h:189-197; the reference harness checks against the
 * same fp64 quantity, kernels/gemv_int4.hip:242-272). */
void rt4o_gemv_fold(const int32_t* I, const uint16_t* ws, const float* sa, int M, int N, int K,
                    double* y) {
    const int NG = K / RT4O_GROUP;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++) {
            double acc = 0.0;
            for (int g = 0; g < NG; g++)
                acc += (double)rt4o_f16_to_f32(ws[(size_t)n * NG + g]) * (double)sa[(size_t)m * NG + g] *
                       (double)I[((size_t)m * N + n) * NG + g];
            y[(size_t)m * N + n] = acc;
        }
}

/* The whole decode GEMV as k_gemv_w4a8 does it (src/k_gemv.hip:53-106):
 * quantize each activation row (quant_act), exact group dots, fold.
 * Scratch is allocated here; y is fp64. */
void rt4o_gemv_w4a8(const uint32_t* wq, const uint16_t* ws, const float* x, int M, int N, int K,
                    double* y) {
    const int NG = K / RT4O_GROUP;
    int8_t* q = (int8_t*)malloc((size_t)M * K);
    float* sa = (float*)malloc((size_t)M * NG * sizeof(float));
    int32_t* I = (int32_t*)malloc((size_t)M * N * NG * sizeof(int32_t));
    rt4o_quant_act(x, M, K, q, sa, NULL);
    rt4o_gemv_groupsums(wq, q, M, N, K, I);
    rt4o_gemv_fold(I, ws, sa, M, N, K, y);
    free(q);
    free(sa);
    free(I);
}

/* ------------------------------------------------------------------- GEMM -- */

/* W4A8 prefill GEMM at selected output points, restating k_gemm_i4_a8
 * (src/k_gemm.hip:22-34): two int4xint4 passes, c = GEMM(h, sc16) + GEMM(l, sc),
 * each pass C[m][n] = Σ_g I_g * SA[g][m] * SB[g][n] (kernels/gemm_core.h:153-166).
 * Outputs, per point p = (mi[p], ni[p]):
 *   c[p]          fp64  Σ_g (sc16[g][m]*sb[g][n]*I_h + sc[g][m]*sb[g][n]*I_l)
 *   Ig[p][g]      int32 16*I_h + I_l, which equals Σ code*q8 exactly
 * Either output may be NULL.  sb is the fp32 group-major weight scale. */
void rt4o_gemm_w4a8_points(const uint32_t* wq, const float* sb, const uint32_t* ah,
                           const uint32_t* al, const float* sc, const float* sc16, int M, int N,
                           int K, const int32_t* mi, const int32_t* ni, int npts, double* c,
                           int32_t* Ig) {
    const int NG = K / RT4O_GROUP, KD = K / 8;
#pragma omp parallel for schedule(static)
    for (int p = 0; p < npts; p++) {
        const int m = mi[p], n = ni[p];
        const uint32_t* w = wq + (size_t)n * KD;
        const uint32_t* h = ah + (size_t)m * KD;
        const uint32_t* l = al + (size_t)m * KD;
        double acc = 0.0;
        for (int g = 0; g < NG; g++) {
            int32_t ih = 0, il = 0;
            for (int d = g * 16; d < g * 16 + 16; d++) {
                ih = rt4o_dot8_i4(h[d], w[d], ih);
                il = rt4o_dot8_i4(l[d], w[d], il);
            }
            const double s_b = (double)sb[(size_t)g * N + n];
            acc += (double)sc16[(size_t)g * M + m] * s_b * (double)ih +
                   (double)sc[(size_t)g * M + m] * s_b * (double)il;
            if (Ig) Ig[(size_t)p * NG + g] = 16 * ih + il;
        }
        if (c) c[p] = acc;
    }
}

/* int4 x int4 GEMM at selected points, restating gemm_w4a4 (kernels/gemm_core.h:
 * 59-206) as called by k_gemm_i4 (src/k_gemm.hip:8-17): C = Σ_g I_g*sa[g][m]*sb[g][n]. */
void rt4o_gemm_w4a4_points(const uint32_t* wq, const float* sb, const uint32_t* aq,
                           const float* sa, int M, int N, int K, const int32_t* mi,
                           const int32_t* ni, int npts, double* c, int32_t* Ig) {
    const int NG = K / RT4O_GROUP, KD = K / 8;
#pragma omp parallel for schedule(static)
    for (int p = 0; p < npts; p++) {
        const int m = mi[p], n = ni[p];
        const uint32_t* w = wq + (size_t)n * KD;
        const uint32_t* a = aq + (size_t)m * KD;
        double acc = 0.0;
        for (int g = 0; g < NG; g++) {
            int32_t s = 0;
            for (int d = g * 16; d < g * 16 + 16; d++) s = rt4o_dot8_i4(a[d], w[d], s);
            acc += (double)sa[(size_t)g * M + m] * (double)sb[(size_t)g * N + n] * (double)s;
            if (Ig) Ig[(size_t)p * NG + g] = s;
        }
        if (c) c[p] = acc;
    }
}
