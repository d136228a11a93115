/*
 * rt4k.h -- C ABI of the MI355X (gfx950) RT4 quantized-matmul library, librt4k.so.
 *
 * Plain pointers and sizes only.  Every pointer argument is a device pointer
 * owned by the caller unless stated otherwise; `stream` is a hipStream_t passed
 * as void* (NULL = the null stream, which is what the reference runtime uses).
 * Every entry point is asynchronous on `stream` and returns RT4_OK or an error
 * code; rt4_last_error() then describes the failure (thread-local).
 *
 * Library scratch: the drop-in linears' quantized activations, the split
 * workspaces of the GEMVs (W4A8 and W4A4 share one, partials plus counters that
 * every launch leaves at zero), of the GEMM and of the attention prefill, and the
 * prefill's staged K/V copy (32 KB per key tile and KV head) are one buffer per
 * device and kind, grown on demand like the reference's static
 * scratch (src/k_gemv.hip:16-23).  Calls that may run at the same time on one
 * device (different streams) therefore race on it; the caller orders them, as
 * it must for the reference.  An outgrown buffer is kept allocated until
 * rt4_release_scratch or the end of the process (the reference frees it on
 * growth), so a HIP graph captured before a larger call still replays into valid
 * memory; growth is by half at least.
 * Nothing is allocated while `stream` is being captured: a call that would
 * have to grow a scratch buffer then fails with RT4_E_CAPTURE, except that the
 * split GEMV and the attention prefill (automatic split count) fall back to
 * their unsplit forms, which need no workspace, and the prefill without room for
 * its staged K/V copy stages the tiles in every workgroup (same results).
 *
 * Formats (docs/FORMAT.md:61-73 of the reference, unchanged here):
 *   wq   uint32 [N][K/8]   RT4 int4 weights: dword d holds k = 8d..8d+7, nibble e
 *                          = bits 4e..4e+3, two's complement, low nibble first.
 *   ws   uint16 [N][K/128] fp16 bit patterns of the per-128-group weight scales,
 *                          row-major (the reference passes these as `const float*`).
 *   wsc_gm float [K/128][N] fp32 group-major weight scales (src/model.cpp:190-202):
 *                          the fp16 scales of ws widened to fp32, as
 *                          rt4_make_group_major writes them, or any other finite
 *                          fp32 values: the prefill GEMMs keep all 24 significant
 *                          bits in their scale products.
 *   xq   int8  [rows][K]   activation codes in "interleaved" order: for each
 *                          8-element block b, bytes [a(8b+0) a(8b+2) a(8b+4) a(8b+6)
 *                          a(8b+1) a(8b+3) a(8b+5) a(8b+7)].  Internal to this
 *                          library; it matches the even/odd nibble split of wq.
 *
 * Each entry cites the reference interface it replaces (reference file:line).
 */
#ifndef RT4K_H
#define RT4K_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#define RT4_OK 0
#define RT4_E_SHAPE 1    /* a shape precondition of the reference is violated */
#define RT4_E_ARG 2      /* null pointer, unsupported group size or config */
#define RT4_E_HIP 3      /* HIP runtime or kernel launch failure */
#define RT4_E_CAPTURE 4  /* library scratch would have to grow while the stream is being
                            captured into a HIP graph: make one eager call at the largest
                            shape first (nothing is allocated under capture) */

/* Description of the last failure on this thread ("" if none). */
const char* rt4_last_error(void);
/* ABI version of this header (bumped on incompatible change). */
int rt4_abi_version(void);

/* Frees the library scratch of the current device: the buffers in use and every
 * outgrown one kept for graphs captured earlier.  Waits for the device first
 * (hipDeviceSynchronize), so no call already issued can still use them; the next
 * call that needs scratch allocates it again.  Graphs captured before this call
 * must not be replayed afterwards (they would write into freed memory): call it
 * when such graphs are destroyed or at shutdown.  The static array of
 * rt4_gemv_w4a8_noalloc is not affected.  Not a graph operation (fails under
 * capture through hipDeviceSynchronize).  No reference counterpart: the
 * reference frees its scratch only when it grows (src/k_gemv.hip:16-23). */
int rt4_release_scratch(void);

/* ------------------------------------------------------------ decode path -- */

/* Decode-side activation quantizer.  Replaces the quant_act launch of
 * k_gemv_w4a8 (kernels/gemv_w4a8_core.h:34-66, launched at src/k_gemv.hip:70).
 * x f32 [rows][K] -> xq int8 [rows][K] interleaved, sa f32 [rows][K/128]
 * (s = amax/127 per group, 1 for an all-zero group), asu int32 [rows][K/128]
 * = per-group sum of the codes (optional, may be NULL).  K % 128 == 0. */
int rt4_quant_act_a8(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows, int K,
                     void* stream);

/* Per-row activation quantizer: one scale per row (G = K).  No counterpart in
 * the reference, which quantizes per (row, 128-group); it is an opt-in mode for
 * callers that want activations "quantized per row", as the benchmark configs
 * describe them.  The row's scale is written into every 128-group slot of the
 * per-group layout, so the GEMV and GEMM entries consume it unchanged.
 *   mode 0, the GEMV form: s = amax/127 (1 for an all-zero row), codes
 *     clamp(lrintf(x/s), -128, 127), xq int8 [rows][K] interleaved as
 *     rt4_quant_act_a8 writes it, sa f32 [rows][K/128], asu (optional, may be
 *     NULL) int32 [rows][K/128] = Σq per group; for rt4_gemv_w4a8_q.
 *   mode 1, the GEMM form: s = amax/119, codes clamp(..., -128, 119), xq as
 *     rt4_quant_rows_i8 writes it, sa f32 [K/128][rows] group-major; for
 *     rt4_gemm_w4a8_i8.
 * K % 128 == 0; x rows of K floats, contiguous. */
int rt4_quant_act_rowwise(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows, int K, int mode,
                          void* stream);

/* W4A8 GEMV on pre-quantized activations.  Replaces the gemv_w4a8<M,SMEM,NROW>
 * launch of k_gemv_w4a8 (kernels/gemv_w4a8_core.h:76-209, src/k_gemv.hip:96-103).
 * y f32 [rows][N] = Σ_g f16(ws[n][g]) * sa[m][g] * Σ_{k∈g} code[n][k]*xq[m][k].
 * rows in [1,4], K % 128 == 0 (src/k_gemv.hip:54-55). */
int rt4_gemv_w4a8_q(float* y, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                    const float* sa, int rows, int N, int K, void* stream);

/* Same, with an explicit launch configuration (tuning and tests).  A
 * workgroup owns one tile of row_blocks x 16 weight rows (row_blocks 1 or 2:
 * with 2 each wave applies its activations to two 16-row blocks);
 * groups_per_wave (even, 2..12) is the number of 128-wide K groups each wave
 * streams per pass, waves (1..16, at most the number of such chunks) the waves
 * per workgroup.  When the tile count is not a multiple of the CU count, the
 * leftover tiles can be cut along K into pieces that run on otherwise idle
 * CUs: k_splits 1 keeps every tile whole, S >= 2 allows up to S pieces per
 * leftover tile.  0 selects the default for each parameter; all four 0 is the
 * default launch, which for one activation row (K a multiple of 256, at most
 * 8192, N at most 256 rows per CU) is a dot-product form outside this parameter
 * space, and any non-zero parameter selects a tiled matrix-core form.
 * Configurations differ only in the order of the fp32 sums over K groups; a
 * configuration gives the same y bit for bit on every call. */
int rt4_gemv_w4a8_q_cfg(float* y, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                        const float* sa, int rows, int N, int K, int groups_per_wave, int waves,
                        int k_splits, int row_blocks, void* stream);

/* The launch configuration rt4_gemv_w4a8_q picks for this shape on the
 * current device: groups per wave, waves per workgroup, the number of K
 * pieces per leftover tile (1: all tiles whole) and the 16-row blocks per tile;
 * groups_per_wave = row_blocks = 0 for the one-row dot-product form (waves: per
 * workgroup, two weight rows each).  No counterpart in the reference (its
 * launch is fixed per M); for tuning and reports. */
int rt4_gemv_launch_plan(int rows, int N, int K, int* groups_per_wave, int* waves, int* k_splits,
                         int* row_blocks);

/* Test hook: the same kernel, also writing the exact per-group int32 dot
 * products gsum int32 [rows][N][K/128] = Σ_{k∈g} code[n][k]*xq[m][k]. */
int rt4_gemv_w4a8_groupsums(int32_t* gsum, float* y, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, int rows, int N, int K,
                            void* stream);

/* The whole decode linear: quantize x per (row, 128-group) to int8, then the
 * GEMV.  Replaces k_gemv_w4a8 (src/kernels.h:27, src/k_gemv.hip:53-106), which
 * is two launches (quant_act, then the GEMV), as is this one.  x f32
 * [rows][K] contiguous.  The quantized activations go to library-owned
 * scratch, grown with hipMalloc on first use per device (as the reference
 * does, src/k_gemv.hip:56-67); not re-entrant across threads. */
int rt4_gemv_w4a8(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows,
                  int N, int K, void* stream);

/* No counterpart in the reference: rt4_gemv_w4a8 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, the same two launches and
 * the same split, so y is bit-identical to rt4_gemv_w4a8's; it calls no
 * hipMalloc, hipFree or other allocating routine.  Its scratch is one static
 * device array per GPU (about 0.4 MB, held until the process ends): K <= 65536
 * and at most 320 CUs, else RT4_E_SHAPE / RT4_E_ARG.  Every call on a GPU shares
 * that GPU's array, so calls that overlap on one GPU (other streams, other host
 * threads) race; order them.  The first call on a device clears the array's
 * counters with a kernel on `stream`. */
int rt4_gemv_w4a8_noalloc(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows, int N,
                          int K, void* stream);

/* rt4_gemv_w4a8 as ONE launch, with an explicit launch configuration
 * (parameters as rt4_gemv_w4a8_q_cfg; tuning and tests): the GEMV's waves
 * quantize the activations in registers, codes and scales bit-identical to
 * rt4_quant_act_a8, so y equals the two-launch result bit for bit.  No
 * library scratch.  x must be 16-byte aligned. */
int rt4_gemv_w4a8_cfg(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows, int N, int K,
                      int groups_per_wave, int waves, int k_splits, int row_blocks, void* stream);

/* ----------------------------------------------------------- prefill path -- */

/* Prefill-side 8-bit quantizer split into two int4 digits.  Replaces
 * k_quant_rows_a8 (src/kernels.h:43, src/k_new.hip:268-301), same outputs bit
 * for bit: qh, ql uint32 [rows][K/8] nibble-packed like wq with q8 = 16h + l,
 * sc, sc16 f32 group-major [K/G][rows], s = amax/119, sc16 = 16*s.
 * Row r is read at x + r*in_stride + in_off (in_stride 0 means K).
 * G must be a power of two in [8, 512] dividing K (the runtime uses 128). */
int rt4_quant_rows_a8(uint32_t* qh, uint32_t* ql, float* sc, float* sc16, const float* x,
                      int rows, int K, int G, int in_stride, int in_off, void* stream);

/* Same quantizer writing the int8 codes q8 themselves (interleaved [rows][K])
 * and sc [K/128][rows]: the input of rt4_gemm_w4a8_i8.  No reference
 * counterpart; it fuses k_quant_rows_a8 with the digit recombination that
 * rt4_gemm_w4a8 otherwise performs.  G = 128. */
int rt4_quant_rows_i8(int8_t* xq, float* sc, const float* x, int rows, int K, int in_stride,
                      int in_off, void* stream);

/* h/l digit planes -> interleaved int8 codes q8 = 16h + l. */
int rt4_digits_to_i8(int8_t* xq, const uint32_t* qh, const uint32_t* ql, int rows, int K,
                     void* stream);

/* W4A8 prefill GEMM.  Replaces k_gemm_i4_a8 (src/kernels.h:32, src/k_gemm.hip:
 * 22-34, kernel gemm_w4a4 of kernels/gemm_core.h:59-206 run twice plus
 * k_add_inplace), with the same preconditions (M % 128, N % 64, K % 128 == 0)
 * and arguments: c f32 [M][N] = Σ_g sb[g][n] * (sc16[g][m]*I_h + sc[g][m]*I_l)
 * where I_h, I_l are the per-group int4 x int4 dots of the digit planes ah, al
 * (uint32 [M][K/8], from rt4_quant_rows_a8) with wq.  Here the digits are
 * recombined into q8 = 16h + l and contracted once, so each group's integer
 * 16*I_h + I_l = Σ code*q8 is exact and scaled by sc[g][m]*wsc_gm[g][n]; sc16
 * must be 16*sc as rt4_quant_rows_a8 writes it and is not read.  c2 (M*N
 * floats, as in the reference) is scratch: it holds the recombined int8 codes
 * when 4*N >= K, otherwise library scratch (grown with hipMalloc) is used. */
int rt4_gemm_w4a8(float* c, float* c2, const uint32_t* wq, const float* wsc_gm, const uint32_t* ah,
                  const uint32_t* al, const float* sc, const float* sc16, int M, int N, int K,
                  void* stream);

/* The same GEMM on int8 codes: xq int8 [M][K] interleaved (rt4_quant_rows_i8
 * output), sc f32 [K/128][M].  No reference counterpart (it is k_gemm_i4_a8
 * without the digit planes).  M >= 1, N >= 1, K % 128 == 0.  Each group's scale
 * product sc*wsc_gm is formed to within a few units in the last place of fp32 (the
 * reference rounds it once); an infinite sc gives NaN outputs in its row. */
int rt4_gemm_w4a8_i8(float* c, const uint32_t* wq, const float* wsc_gm, const int8_t* xq,
                     const float* sc, int M, int N, int K, void* stream);

/* Test hook: rt4_gemm_w4a8_i8 that also writes the exact per-group int32 dot
 * products gsum int32 [M][N][K/128] = Σ_{k∈g} q8[m][k]*code[n][k]. */
int rt4_gemm_w4a8_groupsums(int32_t* gsum, float* c, const uint32_t* wq, const float* wsc_gm,
                            const int8_t* xq, const float* sc, int M, int N, int K, void* stream);

/* RT4 fp16 row-major scales -> fp32 group-major.  Replaces the host helper
 * make_group_major (src/model.cpp:190-202), on the device. */
int rt4_make_group_major(float* wsc_gm, const uint16_t* ws, int N, int K, void* stream);

/* ------------------------------------------------ int4-KV attention ------ */
/* Head dim 256; Q and K quantized per (row, 128-dim group), V per (64-key tile,
 * dim), all s = amax/7 with codes clamp(lrintf(x/s), -8, 7).  Layouts:
 *   qq u32 [H][TP][D/8], qsc f32 [H][D/G][TP]
 *   kc u32 [KVH][cap][D/8], ksc f32 [KVH][D/G][cap]
 *   vc u32 [KVH][cap/8][D] (8 consecutive keys per dword, low nibble = even key),
 *   vsc f32 [KVH][cap/BG][D];  x, kf, vf f32 [T][H][D]. */

/* Q quantizer of all heads.  Replaces k_attn_q_quant (src/kernels.h:40,
 * src/k_new.hip:228-260), bit for bit; rows >= T are not written. */
int rt4_attn_q_quant(uint32_t* qq, float* qs, const float* x, int T, int H, int D, int G, int TP,
                     void* stream);

/* K cache append at keys t0..t0+T-1.  Replaces k_kv_append_k (src/kernels.h:50,
 * src/k_new.hip:327-350), bit for bit. */
int rt4_kv_append_k(uint32_t* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                    int kv_total, void* stream);

/* V cache append through the f32 stage [H][BG][D] of the current partial tile:
 * every touched tile is re-quantized from its valid slots.  Replaces
 * k_kv_append_v (src/kernels.h:53, src/k_new.hip:351-399), bit for bit. */
int rt4_kv_append_v(uint32_t* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H,
                    int D, int BG, int kv_total, void* stream);

/* Causal int4 FlashAttention prefill, GQA (KV head = head / ratio), out f32
 * [n_heads][n_q][256] = softmax(Q K^T) V with the reference's fixed-point
 * algorithm: per 64-key tile P = clamp(int(7 exp(s - m_tile) + 0.5), 0, 7) and
 * online rescaling (the running reference moves only when a tile's max exceeds
 * it by more than a factor 2^8: the same O and L, rounded differently).  Query
 * row i has position off + i.  K/V are staged once per call (codes unpacked into
 * the MFMA operand bytes, 32 KB per key tile and KV head of library scratch; at
 * most 4 GiB, beyond which each workgroup stages its own tiles), then DMA'd into
 * LDS by the workgroups.  Replaces the prefill
 * branch of k_attention (src/kernels.h:81, src/k_fa.hip:282-300; kernel fa_int4,
 * kernels/flash_attn_core.h:74-435).  n_q % 64 == 0, kv_cap % 64 == 0,
 * n_tile * 64 <= kv_cap, kv_cap <= 16777152 (2^24 - 64: one KV head's cache is
 * addressed with 32-bit offsets); BG of the V cache must be 64. */
int rt4_attention_prefill(float* out, const uint32_t* qq, const float* qsc, const uint32_t* kc,
                          const float* ksc, const uint32_t* vc, const float* vsc, int n_q, int n_kv,
                          int off, int n_tile, int n_heads, int ratio, int kv_cap, void* stream);

/* Same, with an explicit number of KV splits per (64-row query block, head)
 * (tuning and tests; 0 selects the default that balances the grid over the
 * device's CUs).  With more than one split each split writes its partial state
 * (unnormalised output, running max, denominator) to library scratch (grown
 * with hipMalloc, with one counter per (query block, head)), and the split that
 * finishes last for a (query block, head) combines them in split order within
 * the same launch. */
int rt4_attention_prefill_cfg(float* out, const uint32_t* qq, const float* qsc, const uint32_t* kc,
                              const float* ksc, const uint32_t* vc, const float* vsc, int n_q, int n_kv,
                              int off, int n_tile, int n_heads, int ratio, int kv_cap, int kv_splits,
                              void* stream);

/* ----------------------------------------- W4A4 siblings (RT_ACT4 path) ---- */

/* int4 activation quantizer.  Replaces k_quant_rows (src/kernels.h:36,
 * src/k_new.hip:192-219): q uint32 [rows][K/8], sc f32 [K/G][rows], s = amax/7. */
int rt4_quant_rows_a4(uint32_t* q, float* sc, const float* x, int rows, int K, int G,
                      int in_stride, int in_off, void* stream);

/* Decode int4 activation quantizer, the first launch of k_gemv_w4a4 (quant_act4,
 * kernels/gemv_w4a4_core.h:22-44): per (row, 32-element subgroup)
 * s = amax>0 ? amax/7 : 1, q = clamp(lrintf(x/s), -8, 7).  aq uint32 [rows][K/8]
 * (RT4 nibble order), sa f32 [rows][K/32].  K % 32 == 0. */
int rt4_quant_act_a4(uint32_t* aq, float* sa, const float* x, int rows, int K, void* stream);

/* W4A4 GEMV on quantized activations (gemv_w4a4, kernels/gemv_w4a4_core.h:47-132):
 * y f32 [rows][N] = Σ_j f16(ws[n][j/4]) * sa[m][j] * Σ_{k∈j} code[n][k]*acode[m][k]
 * over the 32-element subgroups j.  rows in [1,4], K % 128 == 0. */
int rt4_gemv_w4a4_q(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa, int rows,
                    int N, int K, void* stream);

/* rt4_gemv_w4a4_q with an explicit launch configuration (no counterpart in the
 * reference, whose launch is fixed; for tuning and tests): groups_per_wave 2 or
 * 4 K groups per wave pass, waves 1..16 waves per 16-row tile (capped at the
 * number of such chunks), k_splits as rt4_gemv_w4a8_q_cfg (1: every tile whole,
 * S >= 2: leftover tiles cut along K into at most S pieces).  0 selects the
 * default for each parameter.  Configurations differ only in the order of the
 * fp32 sums over K groups. */
int rt4_gemv_w4a4_q_cfg(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa,
                        int rows, int N, int K, int groups_per_wave, int waves, int k_splits, void* stream);

/* The whole W4A4 decode linear: quantize x, then the GEMV.  Replaces k_gemv_w4a4
 * (src/kernels.h:25, src/k_gemv.hip:14-42).  The quantized activations go to
 * library scratch grown with hipMalloc (as the reference does, :16-23).  The
 * reference checks only rows <= 4; K % 128 == 0 is required here (the RT4 scale
 * layout has one scale per 128 weights). */
int rt4_gemv_w4a4(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows, int N, int K,
                  void* stream);

/* int4 x int4 prefill GEMM.  Replaces k_gemm_i4 (src/kernels.h:29,
 * src/k_gemm.hip:8-17): C f32 [M][N] = Σ_g I_g * asc_gm[g][m] * wsc_gm[g][n] with
 * I_g = Σ_{k∈g} code_w*code_a exact.  aq uint32 [M][K/8] int4 codes (from
 * k_quant_rows with G = 128), asc_gm f32 [K/128][M].  M % 128, N % 64, K % 128 == 0,
 * as the reference requires.  The codes are sign-extended to int8 in library
 * scratch and run through the W4A8 GEMM kernel (same integers per group). */
int rt4_gemm_w4a4(float* c, const uint32_t* wq, const float* wsc_gm, const uint32_t* aq, const float* asc_gm, int M,
                  int N, int K, void* stream);

/* ------------------------------------------------------------ RT4 files ---- */

/* The converter's output (tools/convert.c:338-381, manifest :546-560) opened as
 * the reference runtime does (RT4::load / RT4::upload, src/model.cpp:141-185):
 * the manifest is parsed, the weight file memory-mapped read-only, every
 * tensor's regions checked to lie inside it (and, for i4/i8, to start 256-byte
 * aligned).  Handles are not thread-safe; host pointers stay valid until
 * rt4_file_close. */
typedef struct rt4_tensor_info {
    const char* name;      /* owned by the file handle */
    char kind[8];          /* "i4", "i8" (codes + fp16 group scales), or a plain kind ("f32", "f16", ...) */
    int ndim;
    int64_t shape[4];      /* i4/i8: [N, K] */
    int64_t group;         /* scale group along K (128) */
    int64_t q_off, s_off;  /* byte offsets of the codes (or the plain data) and of the scales (-1: none) */
    int64_t q_bytes, s_bytes;
    double relerr, src_rms;  /* the converter's quantization report */
} rt4_tensor_info;

/* Open a manifest; weight_path NULL uses its "weight_file" (tried as written,
 * then next to the manifest). */
int rt4_file_open(const char* manifest_path, const char* weight_path, void** file);
int rt4_file_close(void* file);
int rt4_file_count(void* file, int* count);
int rt4_file_find(void* file, const char* name, int* index);
int rt4_file_info(void* file, int index, rt4_tensor_info* info);
/* Host pointers into the mapping (s is NULL for plain kinds). */
int rt4_file_data(void* file, int index, const void** q, const void** s);
int rt4_file_size(void* file, int64_t* bytes);
/* The whole file into one device buffer of at least rt4_file_size bytes, in
 * 256 MB pieces as src/model.cpp:178-184; a tensor then sits at dev + q_off /
 * dev + s_off (wq and ws of the kernels here).  Returns after the copy. */
int rt4_file_upload(void* file, void* dev, int64_t dev_bytes, void* stream);
/* One tensor: codes to q_dev (q_bytes), scales to s_dev (s_bytes).  Returns
 * after the copy. */
int rt4_file_upload_tensor(void* file, int index, void* q_dev, void* s_dev, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif

#endif /* RT4K_H */
