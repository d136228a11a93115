// ref_bind.hip -- C-callable handles onto the reference's own activation
// quantizer kernels, compiled in place from /root/reference for gfx950 by
// oracle/Makefile into oracle/_ref/libref_hip.so.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ as a third-party check of the CPU
// oracle (and of our HIP quantizers) on the same seeded inputs.  Nothing in the
// product library links this.
//
// Only the quantizers (activation quantizers and the attention feeders) are
// bound here.  They are plain C++ float/integer code, so their gfx950 build
// computes what the gfx926 build does.  The reference's
// GEMV/GEMM kernels are deliberately left out: their dot products are inline
// assembly (v_dot4_i32_i8, kernels/gemv_w4a8_core.h:25-29; v_dot8_i32_i4,
// kernels/gemm_core.h:167) written for gfx926, and a gfx950 build of
// k_gemv_w4a8 was observed to return outputs ~4e5x off while the quantizer
// output of the same call was bit-exact -- so they are not the reference's
// arithmetic on this target and are never run.
#include "gemv_w4a8_core.h"  // quant_act (kernels/gemv_w4a8_core.h:34-66); resolved via -I<reference>/kernels
#include "kernels.h"         // k_quant_rows_a8 / k_quant_rows (src/k_new.hip), -I<reference>/src

extern "C" {

// quant_act, kernels/gemv_w4a8_core.h:34-66, launched as src/k_gemv.hip:70 does:
// grid (K/128, rows) x 32 threads.  Outputs the even/odd int8 halves
// [rows][K/2], scales and sums [rows][K/128] into caller device buffers.
void ref_quant_act(const float* x, int8_t* ae, int8_t* ao, float* asc, int* asu, int rows, int K) {
    quant_act<<<dim3(K / GRP, rows), 32>>>(x, ae, ao, asc, asu, rows, K);
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

// attention feeders (src/k_new.hip:228-399): Q quantizer and KV cache appends.
void ref_attn_q_quant(u32* qq, float* qs, const float* x, int T, int H, int D, int G, int TP) {
    k_attn_q_quant(qq, qs, x, T, H, D, G, TP);
}
void ref_kv_append_k(u32* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                     int kv_total) {
    k_kv_append_k(kc, ksc, kf, t0, T, H, D, G, kv_total);
}
void ref_kv_append_v(u32* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H, int D,
                     int BG, int kv_total) {
    k_kv_append_v(vc, vsc, stage, vf, t0, T, H, D, BG, kv_total);
}

void ref_sync(void) { hipDeviceSynchronize(); }

}  // extern "C"
