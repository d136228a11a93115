// rt4_kernels.h -- the reference runtime's kernel API for the RT4 matmul path,
// implemented by librt4k.so on top of the C ABI in rt4k.h.
//
// These are the exact C++ prototypes (names, argument order and meaning,
// default arguments) of the reference's src/kernels.h, so the reference's
// src/model.cpp links against librt4k.so without edits.  Behaviour matches the
// reference wrappers: asynchronous on the null stream, no return value, and a
// violated precondition or launch failure prints a message and calls exit(1)
// (src/k_gemv.hip:54-55, :105; src/k_gemm.hip:24-28, :32).
//
// The reference's model.cpp includes its own src/kernels.h, which declares the
// same functions; this header is for other callers.  Do not include both.
#pragma once
#include <cstdint>

typedef uint32_t u32;

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

// src/kernels.h:27 -- W4A8 decode GEMV, rows <= 4: y[rows][N] = W[N][K] . x[rows][K].
// wsc points at the RT4 fp16 row-major scales (typed float* by the reference).
void k_gemv_w4a8(float* y, const u32* wq, const float* wsc, const float* x, int rows, int N, int K);

// src/kernels.h:32 -- W4A8 prefill GEMM on activations quantized by k_quant_rows_a8.
// c2 is scratch of at least M*N floats (contents unspecified on return).
void k_gemm_i4_a8(float* c, float* c2, const u32* wq, const float* wsc_gm, const u32* ah,
                  const u32* al, const float* sc, const float* sc16, int M, int N, int K);

// src/kernels.h:43 -- 8-bit activation quantizer split into two int4 digits.
void k_quant_rows_a8(u32* qh, u32* ql, float* sc, float* sc16, const float* x, int rows, int K,
                     int G, int in_stride = 0, int in_off = 0);

// src/kernels.h:36 -- int4 activation quantizer (RT_ACT4 A/B path).
void k_quant_rows(u32* q, float* sc, const float* x, int rows, int K, int G, int in_stride = 0,
                  int in_off = 0);

// src/kernels.h:25 -- W4A4 decode GEMV (RT_ACT4 path), rows <= 4: activations
// quantized to int4 per 32 elements, then the GEMV.
void k_gemv_w4a4(float* y, const u32* wq, const float* wsc, const float* x, int rows, int N, int K);

// src/kernels.h:29 -- int4 x int4 prefill GEMM on activations from k_quant_rows.
void k_gemm_i4(float* c, const u32* wq, const float* wsc_gm, const u32* aq, const float* asc_gm,
               int M, int N, int K);

// src/kernels.h:40 -- Q quantizer of all heads for the attention kernel.
void k_attn_q_quant(u32* qq, float* qs, const float* x, int T, int H, int D, int G, int TP);

// src/kernels.h:50,53 -- KV cache appends (K per (key, 128-dim group); V per (64-key tile, dim)).
void k_kv_append_k(u32* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                   int kv_total);
void k_kv_append_v(u32* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H, int D,
                   int BG, int kv_total);

// src/kernels.h:81 -- int4-KV causal attention.  The prefill branch runs this
// library's kernel; the single-row decode branch (n_row == 1, off + 1 == n_kv)
// calls the caller's own k_attention_decode (src/k_fa.hip:244-259) when the
// executable defines it, else the prefill kernel (the reference's RT_ATTN_OLD=1
// path).  pout/pmax/psum/max_split are the decode routine's split-KV scratch.
void k_attention(float* out, const u32* qq, const float* qsc, const u32* kc, const float* ksc,
                 const u32* vc, const float* vsc, int n_q, int n_row, int n_kv, int off, int n_tile,
                 int n_heads, int ratio, int kv_cap, float* pout, float* pmax, float* psum,
                 int max_split);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
