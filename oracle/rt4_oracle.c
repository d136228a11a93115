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
 *   rt4o_quant_act4     closed form + invariants (|q|<=8, argmax -> +-7, zero
 *                       subgroup -> s=1) + numpy restatement + the reference's
 *                       quant_act4 built for gfx950 (GPU test)
 *   rt4o_gemv_w4a4_*    brute-force integer dots (numpy), fp64 fold
 *   rt4o_gemm_*         per-group int = 16*I_h + I_l identity, fp64 fold as in
 *                       bench/int4_gemm2.cpp:104-123
 *   rt4o_quant_weight_rows, rt4o_f32_to_f16_conv
 *                       the reference converter (tools/convert.c) built in
 *                       oracle/_ref, bit-identical output on a BF16 input
 *   rt4o_attn_q_quant, rt4o_kv_append_k/v
 *                       numpy restatement, split-append invariance of the V
 *                       stage, and the reference's own feeder kernels built for
 *                       gfx950 (GPU test)
 *   rt4o_fa_rows        mode 0 against a numpy exact softmax over the dequantized
 *                       cache; mode 1 against a numpy restatement of the tile
 *                       algorithm and against mode 0 where the fixed-point scheme
 *                       is exact (all scores equal)
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

/* ------------------------------------------------------------- W4A4 GEMV -- */
#define RT4O_SG 32

/* Decode int4 activation quantizer, restating quant_act4
 * (kernels/gemv_w4a4_core.h:22-44): per (row m, 32-element subgroup j)
 * s = amax>0 ? amax/7 : 1, q = clamp(lrintf(x/s), -8, 7); codes packed 8 per
 * dword in the RT4 order (low nibble = even k), scales sa[m][j]. */
void rt4o_quant_act4(const float* x, int M, int K, uint32_t* aq, float* sa) {
    const int NS = K / RT4O_SG;
    for (int m = 0; m < M; m++)
        for (int j = 0; j < NS; j++) {
            const float* src = x + (size_t)m * K + (size_t)j * RT4O_SG;
            float amax = 0.f;
            for (int i = 0; i < RT4O_SG; i++) amax = fmaxf(amax, fabsf(src[i]));
            const float s = amax > 0.f ? amax / 7.f : 1.f;
            sa[(size_t)m * NS + j] = s;
            for (int d = 0; d < RT4O_SG / 8; d++) {
                uint32_t w = 0;
                for (int e = 0; e < 8; e++) {
                    int c = (int)lrintf(src[8 * d + e] / s);
                    c = c > 7 ? 7 : (c < -8 ? -8 : c);
                    w |= ((uint32_t)c & 0xFu) << (4 * e);
                }
                aq[(size_t)m * (K / 8) + (size_t)j * 4 + d] = w;
            }
        }
}

/* Exact per-subgroup dots of the W4A4 GEMV: I[m][n][j] = Σ_{k in subgroup j}
 * code[n][k] * acode[m][k] (gemv_w4a4, kernels/gemv_w4a4_core.h:101-110, four
 * v_dot8 per lane = one 32-element subgroup). */
void rt4o_gemv_w4a4_sums(const uint32_t* wq, const uint32_t* aq, int M, int N, int K, int32_t* I) {
    const int NS = K / RT4O_SG, KD = K / 8;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++)
            for (int j = 0; j < NS; j++) {
                int32_t s = 0;
                for (int d = 4 * j; d < 4 * j + 4; d++) s = rt4o_dot8_i4(aq[(size_t)m * KD + d], wq[(size_t)n * KD + d], s);
                I[((size_t)m * N + n) * NS + j] = s;
            }
}

/* fp64 fold: y[m][n] = Σ_j f16(ws[n][j/4]) * sa[m][j] * I[m][n][j]
 * (kernels/gemv_w4a4_core.h:111-117: weight group scale per 128, activation
 * scale per 32). */
void rt4o_gemv_w4a4_fold(const int32_t* I, const uint16_t* ws, const float* sa, int M, int N, int K, double* y) {
    const int NS = K / RT4O_SG, NG = K / RT4O_GROUP;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++)
        for (int m = 0; m < M; m++) {
            double acc = 0.0;
            for (int j = 0; j < NS; j++)
                acc += (double)rt4o_f16_to_f32(ws[(size_t)n * NG + j / 4]) * (double)sa[(size_t)m * NS + j] *
                       (double)I[((size_t)m * N + n) * NS + j];
            y[(size_t)m * N + n] = acc;
        }
}

/* The whole W4A4 decode linear as k_gemv_w4a4 does it (src/k_gemv.hip:14-42). */
void rt4o_gemv_w4a4(const uint32_t* wq, const uint16_t* ws, const float* x, int M, int N, int K, double* y) {
    const int NS = K / RT4O_SG;
    uint32_t* aq = (uint32_t*)malloc((size_t)M * (K / 8) * sizeof(uint32_t));
    float* sa = (float*)malloc((size_t)M * NS * sizeof(float));
    int32_t* I = (int32_t*)malloc((size_t)M * N * NS * sizeof(int32_t));
    rt4o_quant_act4(x, M, K, aq, sa);
    rt4o_gemv_w4a4_sums(wq, aq, M, N, K, I);
    rt4o_gemv_w4a4_fold(I, ws, sa, M, N, K, y);
    free(aq);
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

/* -------------------------------------------------- int4-KV attention -- */
/* Head dim 256, Q/K quantized per (row, 128-dim group), V per (64-key tile, dim). */
#define RT4O_HD 256
#define RT4O_KD (RT4O_HD / 8)
#define RT4O_QG 128
#define RT4O_NQG (RT4O_HD / RT4O_QG)
#define RT4O_BN 64

/* int4 code of one element: s = amax>0 ? amax/7 : 1 applied by the caller. */
static uint32_t rt4o_i4(float x, float s) {
    int c = (int)lrintf(x / s);
    c = c > 7 ? 7 : (c < -8 ? -8 : c);
    return (uint32_t)c & 0xFu;
}

/* Q quantizer of all heads, restating attn_q_quant_k (src/k_new.hip:228-253):
 * x f32 [T][H][D] -> qq u32 [H][TP][D/8], qs f32 [H][D/G][TP]; rows >= T untouched. */
void rt4o_attn_q_quant(uint32_t* qq, float* qs, const float* x, int T, int H, int D, int G, int TP) {
    const int ng = D / G;
    for (int h = 0; h < H; h++)
        for (int r = 0; r < T; r++)
            for (int g = 0; g < ng; g++) {
                const float* xr = x + ((size_t)r * H + h) * D + (size_t)g * G;
                float amax = 0.f;
                for (int j = 0; j < G; j++) amax = fmaxf(amax, fabsf(xr[j]));
                const float s = amax > 0.f ? amax / 7.f : 1.f;
                qs[((size_t)h * ng + g) * TP + r] = s;
                uint32_t* qr = qq + ((size_t)h * TP + r) * (D / 8) + (size_t)(g * G) / 8;
                for (int j = 0; j < G; j += 8) {
                    uint32_t w = 0;
                    for (int e = 0; e < 8; e++) w |= rt4o_i4(xr[j + e], s) << (4 * e);
                    qr[j / 8] = w;
                }
            }
}

/* K cache append, restating kv_append_k_k (src/k_new.hip:327-347): kf f32 [T][H][D]
 * -> kc u32 [H][kv_total][D/8], ksc f32 [H][D/G][kv_total] at keys t0..t0+T-1. */
void rt4o_kv_append_k(uint32_t* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                      int kv_total) {
    const int ng = D / G;
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++)
            for (int g = 0; g < ng; g++) {
                const int kv = t0 + t;
                const float* xr = kf + ((size_t)t * H + h) * D + (size_t)g * G;
                float amax = 0.f;
                for (int i = 0; i < G; i++) amax = fmaxf(amax, fabsf(xr[i]));
                const float s = amax > 0.f ? amax / 7.f : 1.f;
                ksc[((size_t)h * ng + g) * kv_total + kv] = s;
                uint32_t* qr = kc + ((size_t)h * kv_total + kv) * (D / 8) + (size_t)(g * G) / 8;
                for (int i = 0; i < G; i += 8) {
                    uint32_t w = 0;
                    for (int e = 0; e < 8; e++) w |= rt4o_i4(xr[i + e], s) << (4 * e);
                    qr[i / 8] = w;
                }
            }
}

/* V cache append, restating kv_append_v_k (src/k_new.hip:351-392): the f32 stage
 * [H][BG][D] holds the current partial tile; every tile the append touches is
 * re-quantized from its valid slots (s = amax/7 per (tile, dim), slots beyond the
 * last valid one are zero codes) into vc u32 [H][kv_total/8][D] (8 keys per dword,
 * low nibble = even key) and vsc f32 [H][kv_total/BG][D]. */
void rt4o_kv_append_v(uint32_t* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H,
                      int D, int BG, int kv_total) {
    for (int h = 0; h < H; h++)
        for (int d = 0; d < D; d++) {
            float* st = stage + (size_t)h * BG * D + d;
            uint32_t* out = vc + (size_t)h * (kv_total / 8) * D;
            int done = 0;
            while (done < T) {
                const int kv = t0 + done, tile = kv / BG, slot0 = kv % BG;
                const int n = (T - done < BG - slot0) ? (T - done) : (BG - slot0);
                for (int i = 0; i < n; i++) st[(size_t)(slot0 + i) * D] = vf[((size_t)(done + i) * H + h) * D + d];
                const int nval = slot0 + n;
                float amax = 0.f;
                for (int i = 0; i < nval; i++) amax = fmaxf(amax, fabsf(st[(size_t)i * D]));
                const float s = amax > 0.f ? amax / 7.f : 1.f;
                vsc[((size_t)h * (kv_total / BG) + tile) * D + d] = s;
                for (int i = 0; i < BG; i += 8) {
                    uint32_t w = 0;
                    for (int e = 0; e < 8; e++) {
                        const float v = (i + e < nval) ? st[(size_t)(i + e) * D] : 0.f;
                        w |= rt4o_i4(v, s) << (4 * e);
                    }
                    out[((size_t)tile * (BG / 8) + i / 8) * D + d] = w;
                }
                done += n;
            }
        }
}

static int rt4o_nib(const uint32_t* row, int idx, int e) {
    const int c = (int)((row[idx] >> (4 * e)) & 0xFu);
    return c >= 8 ? c - 16 : c;
}

/* Dequantized operands of one q head / its kv head (values the kernel sees). */
static double fa_q(const uint32_t* Q, const float* Qs, int n_q, int i, int d) {
    return (double)rt4o_nib(Q + (size_t)i * RT4O_KD, d / 8, d % 8) * (double)Qs[(size_t)(d / RT4O_QG) * n_q + i];
}
static double fa_k(const uint32_t* K, const float* Ks, int kv_cap, int j, int d) {
    return (double)rt4o_nib(K + (size_t)j * RT4O_KD, d / 8, d % 8) * (double)Ks[(size_t)(d / RT4O_QG) * kv_cap + j];
}
static double fa_v(const uint32_t* V, const float* Vs, int j, int d) {
    return (double)rt4o_nib(V + (size_t)(j / 8) * RT4O_HD, d, j % 8) * (double)Vs[(size_t)(j / RT4O_BN) * RT4O_HD + d];
}

/* For query row i of q head `head`: its absolute position is off + i and it sees
 * keys j <= min(off + i, n_kv - 1).  Layouts as fa_int4 reads them
 * (kernels/flash_attn_core.h:74-112): qq [H][n_q][32], qsc [H][2][n_q],
 * kc [KVH][kv_cap][32], ksc [KVH][2][kv_cap], vc [KVH][kv_cap/8][256],
 * vsc [KVH][kv_cap/64][256], KV head = head / ratio.
 *
 * mode 0: exact softmax in fp64 over the same quantized Q/K/V, restating ref_rows
 *         (kernels/flash_attn_int4.hip:146-170);
 * mode 1: the kernel's fixed-point algorithm in fp64, restating ref_alg
 *         (kernels/flash_attn_int4.hip:175-217): per 64-key tile the row max mt,
 *         P = round(7 exp(s - mt)) in [0, 7], online rescale alpha = exp(r_old - r_new),
 *         beta = exp(mt - r_new) / 7, out = O / L.  For n_kv that is not a
 *         multiple of 64, where ref_alg (whole tiles only) is not defined, the
 *         reference kernel's loads decide (kernels/flash_attn_core.h:143-152): the
 *         partial last tile is processed, and V is read per whole 8-key group only,
 *         so the keys of a partial group (n_kv % 8 != 0) count in P and L with a V
 *         of zero.  (K past n_kv reads as zero codes there too; causality already
 *         hides those keys.)
 * out f64 [nrows][256]. */
void rt4o_fa_rows(const uint32_t* qq, const float* qsc, const uint32_t* kc, const float* ksc,
                  const uint32_t* vc, const float* vsc, int n_q, int n_kv, int off, int kv_cap, int ratio,
                  int head, const int32_t* rows, int nrows, int mode, double* out) {
    const int vh = head / ratio;
    const uint32_t* Q = qq + (size_t)head * n_q * RT4O_KD;
    const float* Qs = qsc + (size_t)head * RT4O_NQG * n_q;
    const uint32_t* K = kc + (size_t)vh * kv_cap * RT4O_KD;
    const float* Ks = ksc + (size_t)vh * RT4O_NQG * kv_cap;
    const uint32_t* V = vc + (size_t)vh * (kv_cap / 8) * RT4O_HD;
    const float* Vs = vsc + (size_t)vh * (kv_cap / RT4O_BN) * RT4O_HD;
#pragma omp parallel for schedule(dynamic, 1)
    for (int r = 0; r < nrows; r++) {
        const int gi = rows[r];
        const int pos = off + gi < n_kv - 1 ? off + gi : n_kv - 1;
        double q[RT4O_HD], O[RT4O_HD];
        for (int d = 0; d < RT4O_HD; d++) q[d] = fa_q(Q, Qs, n_q, gi, d);
        double* s = (double*)malloc(sizeof(double) * (size_t)(pos + 1));
        for (int j = 0; j <= pos; j++) {
            double acc = 0.0;
            for (int d = 0; d < RT4O_HD; d++) acc += q[d] * fa_k(K, Ks, kv_cap, j, d);
            s[j] = acc;
        }
        double* o = out + (size_t)r * RT4O_HD;
        if (mode == 0) {
            double mx = -1e300, sum = 0.0;
            for (int j = 0; j <= pos; j++) mx = s[j] > mx ? s[j] : mx;
            for (int d = 0; d < RT4O_HD; d++) O[d] = 0.0;
            for (int j = 0; j <= pos; j++) {
                const double p = exp(s[j] - mx);
                sum += p;
                for (int d = 0; d < RT4O_HD; d++) O[d] += p * fa_v(V, Vs, j, d);
            }
            for (int d = 0; d < RT4O_HD; d++) o[d] = O[d] / sum;
        } else {
            double r_old = -1e300, L = 0.0;
            for (int d = 0; d < RT4O_HD; d++) O[d] = 0.0;
            for (int j0 = 0; j0 <= pos; j0 += RT4O_BN) {
                const int j1 = j0 + RT4O_BN - 1 < pos ? j0 + RT4O_BN - 1 : pos;
                double mt = -1e300;
                for (int j = j0; j <= j1; j++) mt = s[j] > mt ? s[j] : mt;
                double p[RT4O_BN], psum = 0.0;
                for (int j = j0; j <= j1; j++) {
                    p[j - j0] = round(7.0 * exp(s[j] - mt));
                    psum += p[j - j0];
                }
                const double r_new = r_old > mt ? r_old : mt;
                const double alpha = exp(r_old - r_new), beta = exp(mt - r_new) / 7.0;
                const int jv = (n_kv / 8) * 8;   /* keys j >= jv: partial 8-group, V read as zero */
                for (int d = 0; d < RT4O_HD; d++) {
                    double acc = 0.0;
                    for (int j = j0; j <= j1 && j < jv; j++) acc += p[j - j0] * fa_v(V, Vs, j, d);
                    O[d] = O[d] * alpha + beta * acc;
                }
                L = L * alpha + beta * psum;
                r_old = r_new;
            }
            for (int d = 0; d < RT4O_HD; d++) o[d] = O[d] / L;
        }
        free(s);
    }
}
