// ref_bind.hip -- C-callable handles onto the reference's own hot-path kernels,
// compiled in place from /root/reference for gfx950 by oracle/Makefile into
// oracle/_ref/libref_hip.so.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin the CPU oracle (and our HIP
// kernels) against the reference implementation on the same seeded inputs.
// Nothing in the product library links this.
//
// The reference's GEMV wrapper keeps its quantized activations in file-static
// scratch (src/k_gemv.hip:47-51); this TU compiles that file as part of itself so
// the codes it produced can be read back for a bit-exact comparison.
#include "../src/k_gemv.hip"  // resolved through -I<reference>/kernels

extern "C" {

// k_gemv_w4a8, src/k_gemv.hip:53-106 (null stream; exits on shape errors).
void ref_gemv_w4a8(float* y, const u32* wq, const uint16_t* ws, const float* x, int rows, int N,
                   int K) {
    k_gemv_w4a8(y, wq, (const float*)ws, x, rows, N, K);
}

// Read back the activation quantization of the last ref_gemv_w4a8 call:
// even/odd int8 halves [rows][K/2], scales and sums [rows][K/128].
void ref_gemv_last_quant(int8_t* ae, int8_t* ao, float* asc, int* asu, int rows, int K) {
    hipDeviceSynchronize();
    hipMemcpy(ae, s_ae, (size_t)rows * (K / 2), hipMemcpyDeviceToHost);
    hipMemcpy(ao, s_ao, (size_t)rows * (K / 2), hipMemcpyDeviceToHost);
    hipMemcpy(asc, s_asc, (size_t)rows * (K / GRP) * 4, hipMemcpyDeviceToHost);
    hipMemcpy(asu, s_asu, (size_t)rows * (K / GRP) * 4, hipMemcpyDeviceToHost);
}

// k_gemv_w4a4, src/k_gemv.hip:14-42.
void ref_gemv_w4a4(float* y, const u32* wq, const uint16_t* ws, const float* x, int rows, int N,
                   int K) {
    k_gemv_w4a4(y, wq, (const float*)ws, x, rows, N, K);
}

// k_quant_rows_a8, src/k_new.hip:296-301.
void ref_quant_rows_a8(u32* qh, u32* ql, float* sc, float* sc16, const float* x, int rows, int K,
                       int G, int in_stride, int in_off) {
    k_quant_rows_a8(qh, ql, sc, sc16, x, rows, K, G, in_stride, in_off);
}

// k_quant_rows, src/k_new.hip:213-219.
void ref_quant_rows(u32* q, float* sc, const float* x, int rows, int K, int G, int in_stride,
                    int in_off) {
    k_quant_rows(q, sc, x, rows, K, G, in_stride, in_off);
}

// k_gemm_i4_a8, src/k_gemm.hip:22-34.
void ref_gemm_i4_a8(float* c, float* c2, const u32* wq, const float* wsc_gm, const u32* ah,
                    const u32* al, const float* sc, const float* sc16, int M, int N, int K) {
    k_gemm_i4_a8(c, c2, wq, wsc_gm, ah, al, sc, sc16, M, N, K);
}

// k_gemm_i4, src/k_gemm.hip:8-17.
void ref_gemm_i4(float* c, const u32* wq, const float* wsc_gm, const u32* aq, const float* asc_gm,
                 int M, int N, int K) {
    k_gemm_i4(c, wq, wsc_gm, aq, asc_gm, M, N, K);
}

void ref_sync(void) { hipDeviceSynchronize(); }

}  // extern "C"
