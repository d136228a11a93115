/*
 * rt4_probe.h -- C ABI of librt4probe.so: gfx950 ceiling probes for the
 * roofline figures of the RT4 benchmark.  Measurement only; no reference
 * counterpart in the drop-in API (the reference's own probes for gfx926 are
 * the stand-alone programs bench/bench_bw.cpp and bench/bench_isa2.cpp).
 *
 * Every pointer is a device pointer; `stream` is a hipStream_t as void*.
 * Returns 0, 1 (bad argument) or 3 (launch failure).  `sink` must hold one
 * 4-byte word per block; it is written only in a practically impossible case
 * (it keeps the probed work from being optimised away).
 */
#ifndef RT4_PROBE_H
#define RT4_PROBE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* Stream `bytes` (multiple of 16) of `buf` through dwordx4 loads, `blocks` x 256 threads. */
int rt4p_hbm_read(const void* buf, size_t bytes, void* sink, int blocks, void* stream);
/* One pass over `bytes` (multiple of 16): `blocks` workgroups of `threads` (64..1024,
 * a multiple of 64) each read one contiguous slice, every lane issuing all of its
 * dwordx4 loads (at most 16; returns 1 if the slice needs more) before using any;
 * nontemporal != 0 marks them non-temporal. */
int rt4p_read_burst(const void* buf, size_t bytes, void* sink, int blocks, int threads, int nontemporal,
                    void* stream);
/* dst[0:bytes] = src[0:bytes] (bytes multiple of 16), `blocks` x 256 threads. */
int rt4p_copy(void* dst, const void* src, size_t bytes, int blocks, void* stream);
/* `iters` x 4 independent int8 MFMAs per wave: big != 0 selects
 * v_mfma_i32_32x32x32_i8 (32768 MACs each), else v_mfma_i32_16x16x64_i8 (16384). */
int rt4p_mfma_i8(void* sink, int big, int iters, int blocks, void* stream);
/* `iters` x 8 independent v_fma_f32 per lane. */
int rt4p_valu_fma(void* sink, int iters, int blocks, void* stream);
/* The decode GEMV's memory requests alone, for a launch plan (rt4_gemv_launch_plan)
 * of one 16-row block, `groups_per_wave` 2 (8 rows x 128 B per weight load, up to
 * 16 waves) or 4 (the row-transposed form, 4 rows x 256 B, up to 8 waves), `waves`
 * waves and `k_splits` pieces per leftover tile, or groups_per_wave 0: the one-row
 * dot-product form (rows 1, K a multiple of 256 up to 8192, `waves` 1..4 per
 * workgroup of two weight rows each).  wq/ws/xq/sa as rt4_gemv_w4a8_q takes them,
 * `cus` the device's CU count.  rows 1..4, K a multiple of 128*groups_per_wave. */
int rt4p_gemv_loads(const void* wq, const void* ws, const void* xq, const void* sa, void* sink, int rows, int N,
                    int K, int groups_per_wave, int waves, int k_splits, int cus, void* stream);
/* An empty kernel of `blocks` x `threads`. */
int rt4p_empty(int blocks, int threads, void* stream);
/* `iters` x 4 independent v_mfma_scale_f32_32x32x64_f8f6f4 per wave (65536 MACs
 * each), 512 threads per block; fmt 0 FP8 E4M3, 2 FP6 E2M3, 4 FP4 E2M1 for both
 * operands. */
int rt4p_mfma_f8f6f4(void* sink, int fmt, int iters, int blocks, void* stream);
/* `iters` x 8 independent v_mfma_f32_16x16x128_f8f6f4 per wave (FP8 E4M3 operands,
 * no block scale, 32768 MACs each), 512 threads per block: the instruction the
 * attention kernel issues. */
int rt4p_mfma_f8_16x16(void* sink, int iters, int blocks, void* stream);
/* `units` iterations of the prefill GEMM's per-unit instruction skeleton (registers
 * only) per wave, 512 threads per block: variant 0 the int8 form, 1 the FP8-digit
 * form (see probe.hip). */
int rt4p_gemm_unit(void* sink, int variant, int units, int blocks, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif

#endif /* RT4_PROBE_H */
