// shim.cpp -- the reference runtime's kernel API (src/kernels.h) on top of the
// rt4_* C ABI.  Same names, argument meaning and error behaviour as the
// reference wrappers: null stream, print and exit(1) on any failure.
#include <cstdio>
#include <cstdlib>

#include "rt4_kernels.h"
#include "rt4k.h"

namespace {
[[noreturn]] void die(const char* who) {
    printf("%s: %s\n", who, rt4_last_error());
    fflush(stdout);
    exit(1);
}
}  // namespace

// src/k_gemv.hip:53-106
void k_gemv_w4a8(float* y, const u32* wq, const float* wsc, const float* x, int rows, int N, int K) {
    if (rt4_gemv_w4a8(y, wq, reinterpret_cast<const uint16_t*>(wsc), x, rows, N, K, nullptr) != RT4_OK)
        die("k_gemv_w4a8");
}

// src/k_new.hip:296-301
void k_quant_rows_a8(u32* qh, u32* ql, float* sc, float* sc16, const float* x, int rows, int K,
                     int G, int in_stride, int in_off) {
    if (rt4_quant_rows_a8(qh, ql, sc, sc16, x, rows, K, G, in_stride, in_off, nullptr) != RT4_OK)
        die("k_quant_rows_a8");
}

// src/k_new.hip:213-219
void k_quant_rows(u32* q, float* sc, const float* x, int rows, int K, int G, int in_stride,
                  int in_off) {
    if (rt4_quant_rows_a4(q, sc, x, rows, K, G, in_stride, in_off, nullptr) != RT4_OK)
        die("k_quant_rows");
}

// src/k_gemm.hip:22-34
void k_gemm_i4_a8(float* c, float* c2, const u32* wq, const float* wsc_gm, const u32* ah,
                  const u32* al, const float* sc, const float* sc16, int M, int N, int K) {
    if (rt4_gemm_w4a8(c, c2, wq, wsc_gm, ah, al, sc, sc16, M, N, K, nullptr) != RT4_OK)
        die("k_gemm_i4_a8");
}
