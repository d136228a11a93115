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

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif

#endif /* RT4_PROBE_H */
