// capi.hip -- extern "C" entry points of librt4k.so (declared in include/rt4k.h).
// Validates shapes the way the reference wrappers do, owns the lazily grown
// scratch of the composite entry points, and maps failures to status codes.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <vector>

#include "rt4_internal.h"
#include "rt4k.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return RT4_OK;
    return fail(RT4_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Library-owned device scratch, one buffer per (device, slot), grown on demand.
// A buffer that is outgrown is retired, not freed: a HIP graph captured earlier
// keeps its address and may still be replayed (freeing it would leave such a
// graph writing into released memory).  Growth is geometric (x1.5 at least), so
// the retired buffers of a slot add up to at most twice its final size.  Not
// safe for concurrent calls from several threads (the reference's scratch has
// the same property, src/k_gemv.hip:47-51).
enum Slot { kSlotActQ = 0, kSlotActS = 1, kSlotGemmA = 2, kSlotGemmPart = 3, kSlotGemmCnt = 4, kSlotAttnPart = 5, kSlotGemvPart = 6, kSlotGemvCnt = 7, kSlotAttnCnt = 8, kSlotAttnKV = 9, kSlots = 10 };
constexpr int kMaxDev = 64;
struct Buf {
    void* p = nullptr;
    size_t cap = 0;
};
std::mutex g_mu;
Buf g_buf[kMaxDev][kSlots];
std::vector<void*> g_retired[kMaxDev];   // outgrown buffers, freed only by rt4_release_scratch

// Whether this device's scratch slot already holds at least `bytes`.
bool scratch_has(Slot slot, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_buf[dev][slot].cap >= bytes;
}

// Whether work on `st` is being recorded into a HIP graph (nothing may be
// allocated then: hipMalloc is not a graph operation).  A failed query counts as
// not capturing, so that work after a capture the runtime invalidated can still
// allocate.  (Measured on ROCm 7.2: asked about the legacy stream while another
// stream captures in global mode, the query reports no capture; the hipMalloc
// that follows is refused by the runtime, so such a call fails with RT4_E_HIP
// having allocated nothing -- using the legacy stream there is the caller's
// error under global capture, which invalidates that capture in any case.)
bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cap) != hipSuccess) {
        (void)hipGetLastError();   // not left for the caller's next HIP call
        return false;
    }
    return cap != hipStreamCaptureStatusNone;
}

// The slot's buffer, grown to at least `bytes` (counters zeroed on `st` when
// `zero`).  Growth under stream capture is refused with RT4_E_CAPTURE: one
// eager call at the largest shape first sizes the scratch, after which capture
// allocates nothing.
int lib_scratch(Slot slot, size_t bytes, void** out, hipStream_t st, bool zero = false) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDev) return fail(RT4_E_ARG, "device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_mu);
    Buf& b = g_buf[dev][slot];
    if (b.cap < bytes) {
        if (capturing(st))
            return fail(RT4_E_CAPTURE,
                        "library scratch (slot %d) must grow from %zu to %zu bytes while the stream is being "
                        "captured; make one eager call at this shape before capturing",
                        (int)slot, b.cap, bytes);
        const size_t grown = b.cap + b.cap / 2;
        const size_t want = ((bytes > grown ? bytes : grown) + 255) & ~size_t(255);
        void* p = nullptr;
        e = hipMalloc(&p, want);
        if (e != hipSuccess) return hip_status(e, "hipMalloc(scratch)");
        if (b.p) g_retired[dev].push_back(b.p);   // outgrown: stays allocated (see above)
        b.p = p;
        b.cap = want;
        if (zero) {
            e = rt4::launch_zero_i32(static_cast<int*>(b.p), want / sizeof(int), st);
            if (e != hipSuccess) return hip_status(e, "zeroing scratch");
        }
    }
    *out = b.p;
    return RT4_OK;
}

int check_gemv_shape(const char* who, int rows, int N, int K) {
    if (rows < 1 || rows > 4) return fail(RT4_E_SHAPE, "%s: rows=%d not in [1,4] (prefill uses the GEMM)", who, rows);
    if (K <= 0 || K % 128) return fail(RT4_E_SHAPE, "%s: K=%d is not a positive multiple of 128", who, K);
    if (N <= 0) return fail(RT4_E_SHAPE, "%s: N=%d must be positive", who, N);
    if (N > 65535 * 16) return fail(RT4_E_SHAPE, "%s: N=%d too large", who, N);
    return RT4_OK;
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// The GEMV reads weights and activations with 16-byte vector loads.
int check_gemv_align(const char* who, const void* y, const uint32_t* wq, const uint16_t* ws,
                     const int8_t* xq, const float* sa) {
    if (!aligned(wq, 16) || !aligned(xq, 16) || !aligned(y, 4) || !aligned(sa, 4) || !aligned(ws, 4))
        return fail(RT4_E_ARG, "%s: misaligned pointer (wq and xq need 16 bytes, ws 4)", who);
    return RT4_OK;
}

int check_gemm_args(const char* who, int M, int N, int K) {
    if (M < 1 || N < 1) return fail(RT4_E_SHAPE, "%s: M=%d N=%d must be positive", who, M, N);
    if (K <= 0 || K % 128) return fail(RT4_E_SHAPE, "%s: K=%d is not a positive multiple of 128", who, K);
    if (M > 65535 * 128) return fail(RT4_E_SHAPE, "%s: M=%d too large", who, M);
    if (N >= (1 << 23)) return fail(RT4_E_SHAPE, "%s: N=%d too large (at most 2^23 - 1 columns)", who, N);
    // the kernels address a row block of A and of W with 32-bit byte offsets
    if ((unsigned long long)M * (unsigned long long)K >= (1ull << 32) ||
        (unsigned long long)N * (unsigned long long)(K / 2) >= (1ull << 32))
        return fail(RT4_E_SHAPE, "%s: M*K=%llu or N*K/2=%llu bytes exceeds the 32-bit offset range", who,
                    (unsigned long long)M * K, (unsigned long long)N * (K / 2));
    return RT4_OK;
}

int device_cus(int* cus) {
    static int cache[kMaxDev] = {0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDev) return fail(RT4_E_ARG, "device %d out of range", dev);
    if (!cache[dev]) {
        int v = 0;
        e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return hip_status(e, "hipDeviceGetAttribute");
        cache[dev] = v > 0 ? v : 256;
    }
    *cus = cache[dev];
    return RT4_OK;
}

// The GEMM launch with its library-owned split-tile workspace.
int run_gemm(const char* who, int32_t* gsum, float* c, const uint32_t* wq, const float* wsc_gm,
             const int8_t* xq, const float* sc, int M, int N, int K, hipStream_t st) {
    int cus = 0, rc = device_cus(&cus);
    if (rc) return rc;
    const rt4::GemmPlan plan = rt4::gemm_plan(M, N, K, cus);
    void *part = nullptr, *cnt = nullptr;
    if ((rc = lib_scratch(kSlotGemmPart, plan.part_bytes, &part, st))) return rc;
    if ((rc = lib_scratch(kSlotGemmCnt, plan.cnt_bytes, &cnt, st, true))) return rc;
    return hip_status(rt4::launch_gemm_w4a8(c, gsum, xq, wq, sc, wsc_gm, M, N, K, plan, static_cast<float*>(part),
                                            static_cast<int*>(cnt), st),
                      who);
}

// The GEMV launch with its balanced grid: split tiles need a small partial
// workspace and self-resetting counters (library scratch, zeroed once).
// xf (fp32 activations, 16-byte aligned) selects the fused form that quantizes
// inside the GEMV; otherwise xq/sa are the pre-quantized activations.
// Workspace of a split GEMV launch (partials and self-resetting counters),
// shared by the W4A8 and W4A4 GEMVs.  Sized once for the largest split any shape
// can need (at most one piece per CU, 4 rows, two row blocks), so only the first
// split launch on a device allocates.  Under graph capture nothing may be
// allocated: if the workspace does not exist yet, the launch runs unsplit (same
// results up to the order of the fp32 sums, less balanced).
int gemv_split_ws(rt4::GemvSplit* sp, int cus, hipStream_t st) {
    if (sp->nrem == 0) return RT4_OK;
    const size_t pb = (size_t)cus * rt4::kGemvMaxRb * 4 * 16 * sizeof(float), cb = (size_t)cus * sizeof(int);
    if (capturing(st) && !(scratch_has(kSlotGemvPart, pb) && scratch_has(kSlotGemvCnt, cb))) {
        sp->full += sp->nrem;
        sp->nrem = 0;
        sp->S = 1;
        return RT4_OK;
    }
    void *part = nullptr, *cnt = nullptr;
    int rc = lib_scratch(kSlotGemvPart, pb, &part, st);
    if (rc || (rc = lib_scratch(kSlotGemvCnt, cb, &cnt, st, true))) return rc;
    sp->part = static_cast<float*>(part);
    sp->cnt = static_cast<int*>(cnt);
    return RT4_OK;
}

int run_gemv(const char* who, int32_t* gsum, float* y, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
             const float* sa, const float* xf, int rows, int N, int K, const rt4::GemvCfg& c, hipStream_t st) {
    int cus = 0, rc = device_cus(&cus);
    if (rc) return rc;
    rt4::GemvSplit sp = rt4::gemv_split(N, K, c, cus);
    if ((rc = gemv_split_ws(&sp, cus, st))) return rc;
    return hip_status(rt4::launch_gemv_w4a8(y, gsum, wq, ws, xq, sa, xf, rows, N, K, c, sp, st), who);
}

int run_gemv4(const char* who, float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa,
              int rows, int N, int K, const rt4::GemvCfg& c, hipStream_t st) {
    int cus = 0, rc = device_cus(&cus);
    if (rc) return rc;
    rt4::GemvSplit sp = rt4::gemv_split(N, K, c, cus);
    if ((rc = gemv_split_ws(&sp, cus, st))) return rc;
    return hip_status(rt4::launch_gemv_w4a4(y, wq, ws, aq, sa, rows, N, K, c, sp, st), who);
}

// W4A4 GEMV configuration: this device's default with the caller's overrides
// (0 keeps a default), the overrides checked before the device is queried.
int gemv4_cfg(const char* who, int rows, int N, int K, int groups_per_wave, int waves, int k_splits,
              rt4::GemvCfg* out) {
    if ((groups_per_wave != 0 && groups_per_wave != 2 && groups_per_wave != 4) || waves < 0 ||
        waves > rt4::kGemvMaxWaves || k_splits < 0 || k_splits > rt4::kGemvMaxSplit)
        return fail(RT4_E_ARG, "%s: bad config groups_per_wave=%d waves=%d k_splits=%d", who, groups_per_wave,
                    waves, k_splits);
    int cus = 0, rc = device_cus(&cus);
    if (rc) return rc;
    rt4::GemvCfg c = rt4::gemv4_default_cfg(rows, N, K, cus);
    if (groups_per_wave > 0) c.gpw = groups_per_wave;
    if (waves > 0) c.waves = waves;
    if (k_splits > 0) c.max_split = k_splits;
    if (!rt4::gemv4_cfg_valid(c))
        return fail(RT4_E_ARG, "%s: bad config groups_per_wave=%d waves=%d k_splits=%d", who, groups_per_wave,
                    waves, k_splits);
    *out = c;
    return RT4_OK;
}

// The default launch configuration of a shape on the current device.
int default_cfg(int rows, int N, int K, rt4::GemvCfg* out) {
    int cus = 0, rc = device_cus(&cus);
    if (rc) return rc;
    *out = rt4::gemv_default_cfg(rows, N, K, cus);
    return RT4_OK;
}

// Default launch configuration with the caller's overrides (0 keeps a default).
int gemv_cfg(const char* who, int K, int rows, int N, int groups_per_wave, int waves, int k_splits,
             int row_blocks, rt4::GemvCfg* out) {
    // The overrides are checked before the device is queried (argument errors
    // come first), then merged into this device's defaults (which depend on the
    // CU count).
    rt4::GemvCfg c = rt4::gemv_default_cfg(rows, N, K, 0);
    if (groups_per_wave > 0) {
        c.gpw = groups_per_wave;
        const int nc = (K / 128 + c.gpw - 1) / c.gpw;
        c.waves = nc < rt4::kGemvMaxWaves ? nc : rt4::kGemvMaxWaves;
    }
    if (waves > 0) c.waves = waves;
    if (k_splits > 0) c.max_split = k_splits;
    if (row_blocks > 0) c.rb = row_blocks;
    if (groups_per_wave < 0 || waves < 0 || k_splits < 0 || row_blocks < 0 || !rt4::gemv_cfg_valid(c, K))
        return fail(RT4_E_ARG, "%s: bad config groups_per_wave=%d waves=%d k_splits=%d row_blocks=%d", who,
                    groups_per_wave, waves, k_splits, row_blocks);
    // the defaults of this device for whatever was left at 0
    rt4::GemvCfg d;
    int rc = default_cfg(rows, N, K, &d);
    if (rc) return rc;
    if (row_blocks > 0) d.rb = row_blocks;
    if (groups_per_wave > 0) {
        d.gpw = groups_per_wave;
        const int nc = (K / 128 + d.gpw - 1) / d.gpw;
        d.waves = nc < rt4::kGemvMaxWaves ? nc : rt4::kGemvMaxWaves;
    }
    if (waves > 0) d.waves = waves;
    if (k_splits > 0) d.max_split = k_splits;
    if (groups_per_wave > 0 || waves > 0 || k_splits > 0 || row_blocks > 0) d.dot = 0;   // an MFMA form
    if (!rt4::gemv_cfg_valid(d, K))
        return fail(RT4_E_ARG, "%s: bad config groups_per_wave=%d waves=%d k_splits=%d row_blocks=%d", who,
                    groups_per_wave, waves, k_splits, row_blocks);
    *out = d;
    return RT4_OK;
}

// ---- The no-allocation decode linear (rt4_gemv_w4a8_noalloc).  Its scratch
// is one file-scope device array, held by every device the library runs on until
// the process ends: the quantized activations (4 rows of at most kNaMaxK codes
// and their scales), then the split GEMV's partials and counters (sized, like the
// allocated workspace, for one piece per CU, at most kNaMaxCus CUs).  In host code
// `scratch` is not a device address: every use goes through the per-device
// pointer that hipGetSymbolAddress returns.
constexpr int kNaMaxK = 65536;
constexpr int kNaMaxCus = 320;
constexpr size_t kNaQ = (size_t)4 * kNaMaxK;                                       // int8 codes
constexpr size_t kNaS = (size_t)4 * (kNaMaxK / 128) * sizeof(float);             // their scales
constexpr size_t kNaP = (size_t)kNaMaxCus * rt4::kGemvMaxRb * 4 * 16 * sizeof(float);  // split partials
constexpr size_t kNaC = (size_t)kNaMaxCus * sizeof(int);                          // split counters
constexpr size_t kNaBytes = kNaQ + kNaS + kNaP + kNaC;
static_assert(kNaQ % 256 == 0 && kNaS % 256 == 0 && kNaP % 256 == 0, "sections stay 256-byte aligned");

int gemm_i8_common(const char* who, int32_t* gsum, float* c, const uint32_t* wq, const float* wsc_gm,
                   const int8_t* xq, const float* sc, int M, int N, int K, void* stream) {
    if (!c || !wq || !wsc_gm || !xq || !sc) return fail(RT4_E_ARG, "%s: null pointer", who);
    int rc = check_gemm_args(who, M, N, K);
    if (rc) return rc;
    if (!aligned(wq, 16) || !aligned(xq, 16) || !aligned(c, 4) || !aligned(sc, 4) || !aligned(wsc_gm, 4))
        return fail(RT4_E_ARG, "%s: misaligned pointer (wq and xq need 16 bytes, ws 4)", who);
    return run_gemm(who, gsum, c, wq, wsc_gm, xq, sc, M, N, K, as_stream(stream));
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNaBytes];

namespace {
std::mutex g_na_mu;
unsigned char* g_na_ptr[kMaxDev] = {};

// This device's address of `scratch`, looked up (and its split counters cleared
// with a fill kernel on `st`) on the first call on the device.
int noalloc_scratch(unsigned char** out, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDev) return fail(RT4_E_ARG, "device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (!g_na_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
        e = rt4::launch_zero_i32(reinterpret_cast<int*>(static_cast<unsigned char*>(ptr) + kNaQ + kNaS + kNaP),
                                 kNaC / sizeof(int), st);
        if (e != hipSuccess) return hip_status(e, "clearing the split counters");
        g_na_ptr[dev] = static_cast<unsigned char*>(ptr);
    }
    *out = g_na_ptr[dev];
    return RT4_OK;
}
}  // namespace

namespace rt4 {
int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace rt4

extern "C" {

const char* rt4_last_error(void) { return g_err; }
int rt4_abi_version(void) { return 1; }

int rt4_release_scratch(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDev) return fail(RT4_E_ARG, "device %d out of range", dev);
    // every call already issued on any stream of this device may still use the buffers
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_status(e, "hipDeviceSynchronize");
    std::lock_guard<std::mutex> lk(g_mu);
    for (void* p : g_retired[dev]) {
        e = hipFree(p);
        if (e != hipSuccess) return hip_status(e, "hipFree(retired scratch)");
    }
    g_retired[dev].clear();
    for (int s = 0; s < kSlots; s++) {
        Buf& b = g_buf[dev][s];
        if (b.p) {
            e = hipFree(b.p);
            if (e != hipSuccess) return hip_status(e, "hipFree(scratch)");
        }
        b.p = nullptr;
        b.cap = 0;
    }
    return RT4_OK;
}

int rt4_quant_act_a8(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows, int K,
                     void* stream) {
    if (!xq || !sa || !x) return fail(RT4_E_ARG, "rt4_quant_act_a8: null pointer");
    if (rows < 1 || rows > 65535) return fail(RT4_E_SHAPE, "rt4_quant_act_a8: rows=%d", rows);
    if (K <= 0 || K % 128) return fail(RT4_E_SHAPE, "rt4_quant_act_a8: K=%d is not a positive multiple of 128", K);
    if (!aligned(xq, 8) || !aligned(x, 4) || !aligned(sa, 4) || !aligned(asu, 4))
        return fail(RT4_E_ARG, "rt4_quant_act_a8: misaligned pointer (xq needs 8 bytes)");
    return hip_status(rt4::launch_quant_act_a8(xq, sa, asu, x, rows, K, as_stream(stream)),
                      "rt4_quant_act_a8 launch");
}

int rt4_quant_act_rowwise(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows, int K, int mode,
                          void* stream) {
    if (!xq || !sa || !x) return fail(RT4_E_ARG, "rt4_quant_act_rowwise: null pointer");
    if (mode != 0 && mode != 1) return fail(RT4_E_ARG, "rt4_quant_act_rowwise: mode=%d (0: GEMV form, 1: GEMM form)", mode);
    if (rows < 1) return fail(RT4_E_SHAPE, "rt4_quant_act_rowwise: rows=%d", rows);
    if (K <= 0 || K % 128) return fail(RT4_E_SHAPE, "rt4_quant_act_rowwise: K=%d is not a positive multiple of 128", K);
    if (!aligned(xq, 8) || !aligned(x, 4) || !aligned(sa, 4) || !aligned(asu, 4))
        return fail(RT4_E_ARG, "rt4_quant_act_rowwise: misaligned pointer (xq needs 8 bytes)");
    return hip_status(rt4::launch_quant_row(xq, sa, asu, x, rows, K, mode, as_stream(stream)),
                      "rt4_quant_act_rowwise launch");
}

int rt4_gemv_w4a8_q_cfg(float* y, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                        const float* sa, int rows, int N, int K, int groups_per_wave, int waves,
                        int k_splits, int row_blocks, void* stream) {
    if (!y || !wq || !ws || !xq || !sa) return fail(RT4_E_ARG, "rt4_gemv_w4a8: null pointer");
    int rc = check_gemv_shape("rt4_gemv_w4a8", rows, N, K);
    if (rc || (rc = check_gemv_align("rt4_gemv_w4a8", y, wq, ws, xq, sa))) return rc;
    rt4::GemvCfg c;
    if ((rc = gemv_cfg("rt4_gemv_w4a8", K, rows, N, groups_per_wave, waves, k_splits, row_blocks, &c))) return rc;
    return run_gemv("rt4_gemv_w4a8 launch", nullptr, y, wq, ws, xq, sa, nullptr, rows, N, K, c, as_stream(stream));
}

int rt4_gemv_launch_plan(int rows, int N, int K, int* groups_per_wave, int* waves, int* k_splits,
                         int* row_blocks) {
    if (!groups_per_wave || !waves || !k_splits || !row_blocks)
        return fail(RT4_E_ARG, "rt4_gemv_launch_plan: null pointer");
    int rc = check_gemv_shape("rt4_gemv_launch_plan", rows, N, K);
    int cus = 0;
    if (rc || (rc = device_cus(&cus))) return rc;
    const rt4::GemvCfg c = rt4::gemv_default_cfg(rows, N, K, cus);
    const rt4::GemvSplit sp = rt4::gemv_split(N, K, c, cus);
    *groups_per_wave = c.dot ? 0 : c.gpw;   // 0: the dot-product form
    *waves = c.dot ? rt4::kGemvDotWaves : c.waves;
    *k_splits = sp.nrem > 0 ? sp.S : 1;
    *row_blocks = c.dot ? 0 : c.rb;
    return RT4_OK;
}

int rt4_gemv_w4a8_q(float* y, const uint32_t* wq, const uint16_t* ws, const int8_t* xq,
                    const float* sa, int rows, int N, int K, void* stream) {
    return rt4_gemv_w4a8_q_cfg(y, wq, ws, xq, sa, rows, N, K, 0, 0, 0, 0, stream);
}

int rt4_gemv_w4a8_groupsums(int32_t* gsum, float* y, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, int rows, int N, int K,
                            void* stream) {
    if (!gsum || !y || !wq || !ws || !xq || !sa) return fail(RT4_E_ARG, "rt4_gemv_w4a8_groupsums: null pointer");
    int rc = check_gemv_shape("rt4_gemv_w4a8_groupsums", rows, N, K);
    if (rc || (rc = check_gemv_align("rt4_gemv_w4a8_groupsums", y, wq, ws, xq, sa))) return rc;
    rt4::GemvCfg c;
    if ((rc = default_cfg(rows, N, K, &c))) return rc;
    return run_gemv("rt4_gemv_w4a8_groupsums launch", gsum, y, wq, ws, xq, sa, nullptr, rows, N, K, c,
                    as_stream(stream));
}

int rt4_gemv_w4a8_cfg(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows, int N, int K,
                      int groups_per_wave, int waves, int k_splits, int row_blocks, void* stream) {
    if (!y || !wq || !ws || !x) return fail(RT4_E_ARG, "rt4_gemv_w4a8_cfg: null pointer");
    int rc = check_gemv_shape("rt4_gemv_w4a8_cfg", rows, N, K);
    if (rc) return rc;
    if (!aligned(wq, 16) || !aligned(y, 4) || !aligned(x, 16) || !aligned(ws, 4))
        return fail(RT4_E_ARG, "rt4_gemv_w4a8_cfg: misaligned pointer (wq and x need 16 bytes, ws 4)");
    rt4::GemvCfg c;
    if ((rc = gemv_cfg("rt4_gemv_w4a8_cfg", K, rows, N, groups_per_wave, waves, k_splits, row_blocks, &c)))
        return rc;
    return run_gemv("rt4_gemv_w4a8_cfg launch", nullptr, y, wq, ws, nullptr, nullptr, x, rows, N, K, c,
                    as_stream(stream));
}

int rt4_gemv_w4a8(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows,
                  int N, int K, void* stream) {
    if (!y || !wq || !ws || !x) return fail(RT4_E_ARG, "rt4_gemv_w4a8: null pointer");
    int rc = check_gemv_shape("k_gemv_w4a8", rows, N, K);
    if (rc) return rc;
    if (!aligned(wq, 16) || !aligned(y, 4) || !aligned(x, 4) || !aligned(ws, 4))
        return fail(RT4_E_ARG, "k_gemv_w4a8: misaligned pointer (wq needs 16 bytes, ws 4)");
    rt4::GemvCfg c;
    if ((rc = default_cfg(rows, N, K, &c))) return rc;
    // Two launches, as the reference: the activation quantizer into library
    // scratch, then the GEMV.  (The fused one-launch form, rt4_gemv_w4a8_cfg,
    // re-quantizes the activations in every tile and measures slower.)
    hipStream_t st = as_stream(stream);
    void *q = nullptr, *s = nullptr;
    if ((rc = lib_scratch(kSlotActQ, (size_t)rows * K, &q, st))) return rc;
    if ((rc = lib_scratch(kSlotActS, (size_t)rows * (K / 128) * sizeof(float), &s, st))) return rc;
    hipError_t e = rt4::launch_quant_act_a8(static_cast<int8_t*>(q), static_cast<float*>(s), nullptr, x, rows, K, st);
    if (e != hipSuccess) return hip_status(e, "k_gemv_w4a8 quant launch");
    return run_gemv("k_gemv_w4a8 launch", nullptr, y, wq, ws, static_cast<const int8_t*>(q),
                    static_cast<const float*>(s), nullptr, rows, N, K, c, st);
}

int rt4_gemv_w4a8_noalloc(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows, int N,
                          int K, void* stream) {
    if (!y || !wq || !ws || !x) return fail(RT4_E_ARG, "rt4_gemv_w4a8_noalloc: null pointer");
    int rc = check_gemv_shape("rt4_gemv_w4a8_noalloc", rows, N, K);
    if (rc) return rc;
    if (K > kNaMaxK)
        return fail(RT4_E_SHAPE, "rt4_gemv_w4a8_noalloc: K=%d exceeds the static scratch (K <= %d)", K, kNaMaxK);
    if (!aligned(wq, 16) || !aligned(y, 4) || !aligned(x, 4) || !aligned(ws, 4))
        return fail(RT4_E_ARG, "rt4_gemv_w4a8_noalloc: misaligned pointer (wq needs 16 bytes, ws 4)");
    int cus = 0;
    if ((rc = device_cus(&cus))) return rc;
    if (cus > kNaMaxCus)
        return fail(RT4_E_ARG, "rt4_gemv_w4a8_noalloc: %d CUs exceed the static scratch (at most %d)", cus,
                    kNaMaxCus);
    rt4::GemvCfg c;
    if ((rc = default_cfg(rows, N, K, &c))) return rc;
    hipStream_t st = as_stream(stream);
    unsigned char* p = nullptr;
    if ((rc = noalloc_scratch(&p, st))) return rc;
    int8_t* q = reinterpret_cast<int8_t*>(p);
    float* s = reinterpret_cast<float*>(p + kNaQ);
    // the same two launches and the same split as rt4_gemv_w4a8, so y is bit-identical
    hipError_t e = rt4::launch_quant_act_a8(q, s, nullptr, x, rows, K, st);
    if (e != hipSuccess) return hip_status(e, "rt4_gemv_w4a8_noalloc quant launch");
    rt4::GemvSplit sp = rt4::gemv_split(N, K, c, cus);
    if (sp.nrem > 0) {
        sp.part = reinterpret_cast<float*>(p + kNaQ + kNaS);
        sp.cnt = reinterpret_cast<int*>(p + kNaQ + kNaS + kNaP);
    }
    return hip_status(rt4::launch_gemv_w4a8(y, nullptr, wq, ws, q, s, nullptr, rows, N, K, c, sp, st),
                      "rt4_gemv_w4a8_noalloc launch");
}

int rt4_quant_rows_a8(uint32_t* qh, uint32_t* ql, float* sc, float* sc16, const float* x,
                      int rows, int K, int G, int in_stride, int in_off, void* stream) {
    if (!qh || !ql || !sc || !sc16 || !x) return fail(RT4_E_ARG, "rt4_quant_rows_a8: null pointer");
    if (!rt4::quant_group_supported(G) || K <= 0 || K % G)
        return fail(RT4_E_ARG, "rt4_quant_rows_a8: group G=%d unsupported for K=%d", G, K);
    if (rows < 1 || rows > 65535 || in_stride < 0 || in_off < 0)
        return fail(RT4_E_SHAPE, "rt4_quant_rows_a8: rows=%d in_stride=%d in_off=%d", rows, in_stride, in_off);
    return hip_status(rt4::launch_quant_rows_a8(qh, ql, sc, sc16, nullptr, x, rows, K, G, in_stride, in_off,
                                                as_stream(stream)),
                      "rt4_quant_rows_a8 launch");
}

int rt4_quant_rows_i8(int8_t* xq, float* sc, const float* x, int rows, int K, int in_stride,
                      int in_off, void* stream) {
    if (!xq || !sc || !x) return fail(RT4_E_ARG, "rt4_quant_rows_i8: null pointer");
    if (K <= 0 || K % 128) return fail(RT4_E_SHAPE, "rt4_quant_rows_i8: K=%d is not a positive multiple of 128", K);
    if (rows < 1 || rows > 65535 || in_stride < 0 || in_off < 0)
        return fail(RT4_E_SHAPE, "rt4_quant_rows_i8: rows=%d in_stride=%d in_off=%d", rows, in_stride, in_off);
    if (!aligned(xq, 8) || !aligned(x, 4) || !aligned(sc, 4))
        return fail(RT4_E_ARG, "rt4_quant_rows_i8: misaligned pointer (xq needs 8 bytes)");
    return hip_status(rt4::launch_quant_rows_a8(nullptr, nullptr, sc, nullptr, xq, x, rows, K, 128, in_stride,
                                                in_off, as_stream(stream)),
                      "rt4_quant_rows_i8 launch");
}

int rt4_digits_to_i8(int8_t* xq, const uint32_t* qh, const uint32_t* ql, int rows, int K,
                     void* stream) {
    if (!xq || !qh || !ql) return fail(RT4_E_ARG, "rt4_digits_to_i8: null pointer");
    if (rows < 1 || K <= 0 || K % 8) return fail(RT4_E_SHAPE, "rt4_digits_to_i8: rows=%d K=%d", rows, K);
    if (!aligned(xq, 8) || !aligned(qh, 4) || !aligned(ql, 4))
        return fail(RT4_E_ARG, "rt4_digits_to_i8: misaligned pointer (xq needs 8 bytes)");
    return hip_status(rt4::launch_hl_to_i8(xq, qh, ql, rows, K, as_stream(stream)), "rt4_digits_to_i8 launch");
}

int rt4_quant_rows_a4(uint32_t* q, float* sc, const float* x, int rows, int K, int G,
                      int in_stride, int in_off, void* stream) {
    if (!q || !sc || !x) return fail(RT4_E_ARG, "rt4_quant_rows_a4: null pointer");
    if (!rt4::quant_group_supported(G) || K <= 0 || K % G)
        return fail(RT4_E_ARG, "rt4_quant_rows_a4: group G=%d unsupported for K=%d", G, K);
    if (rows < 1 || rows > 65535 || in_stride < 0 || in_off < 0)
        return fail(RT4_E_SHAPE, "rt4_quant_rows_a4: rows=%d in_stride=%d in_off=%d", rows, in_stride, in_off);
    return hip_status(rt4::launch_quant_rows_a4(q, sc, x, rows, K, G, in_stride, in_off, as_stream(stream)),
                      "rt4_quant_rows_a4 launch");
}

int rt4_quant_act_a4(uint32_t* aq, float* sa, const float* x, int rows, int K, void* stream) {
    if (!aq || !sa || !x) return fail(RT4_E_ARG, "rt4_quant_act_a4: null pointer");
    if (rows < 1 || rows > 65535) return fail(RT4_E_SHAPE, "rt4_quant_act_a4: rows=%d", rows);
    if (K <= 0 || K % 32) return fail(RT4_E_SHAPE, "rt4_quant_act_a4: K=%d is not a positive multiple of 32", K);
    if (!aligned(aq, 4) || !aligned(x, 4) || !aligned(sa, 4))
        return fail(RT4_E_ARG, "rt4_quant_act_a4: misaligned pointer");
    return hip_status(rt4::launch_quant_act_a4(aq, sa, x, rows, K, as_stream(stream)), "rt4_quant_act_a4 launch");
}

int rt4_gemv_w4a4_q_cfg(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa,
                        int rows, int N, int K, int groups_per_wave, int waves, int k_splits, void* stream) {
    if (!y || !wq || !ws || !aq || !sa) return fail(RT4_E_ARG, "rt4_gemv_w4a4: null pointer");
    int rc = check_gemv_shape("rt4_gemv_w4a4", rows, N, K);
    if (rc) return rc;
    if (!aligned(wq, 16) || !aligned(aq, 16) || !aligned(y, 4) || !aligned(sa, 4) || !aligned(ws, 4))
        return fail(RT4_E_ARG, "rt4_gemv_w4a4: misaligned pointer (wq and aq need 16 bytes, ws 4)");
    rt4::GemvCfg c;
    if ((rc = gemv4_cfg("rt4_gemv_w4a4", rows, N, K, groups_per_wave, waves, k_splits, &c))) return rc;
    return run_gemv4("rt4_gemv_w4a4 launch", y, wq, ws, aq, sa, rows, N, K, c, as_stream(stream));
}

int rt4_gemv_w4a4_q(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa, int rows,
                    int N, int K, void* stream) {
    return rt4_gemv_w4a4_q_cfg(y, wq, ws, aq, sa, rows, N, K, 0, 0, 0, stream);
}

int rt4_gemv_w4a4(float* y, const uint32_t* wq, const uint16_t* ws, const float* x, int rows, int N, int K,
                  void* stream) {
    if (!y || !wq || !ws || !x) return fail(RT4_E_ARG, "k_gemv_w4a4: null pointer");
    int rc = check_gemv_shape("k_gemv_w4a4", rows, N, K);
    if (rc) return rc;
    if (!aligned(wq, 16) || !aligned(y, 4) || !aligned(x, 4) || !aligned(ws, 4))
        return fail(RT4_E_ARG, "k_gemv_w4a4: misaligned pointer (wq needs 16 bytes, ws 4)");
    hipStream_t st = as_stream(stream);
    void *q = nullptr, *s = nullptr;
    if ((rc = lib_scratch(kSlotActQ, (size_t)rows * K / 2, &q, st))) return rc;
    if ((rc = lib_scratch(kSlotActS, (size_t)rows * (K / 32) * sizeof(float), &s, st))) return rc;
    hipError_t e = rt4::launch_quant_act_a4(static_cast<uint32_t*>(q), static_cast<float*>(s), x, rows, K, st);
    if (e != hipSuccess) return hip_status(e, "k_gemv_w4a4 quant launch");
    rt4::GemvCfg c;
    if ((rc = gemv4_cfg("k_gemv_w4a4", rows, N, K, 0, 0, 0, &c))) return rc;
    return run_gemv4("k_gemv_w4a4 launch", y, wq, ws, static_cast<const uint32_t*>(q), static_cast<const float*>(s),
                     rows, N, K, c, st);
}

int rt4_gemm_w4a4(float* c, const uint32_t* wq, const float* wsc_gm, const uint32_t* aq, const float* asc_gm, int M,
                  int N, int K, void* stream) {
    if (!c || !wq || !wsc_gm || !aq || !asc_gm) return fail(RT4_E_ARG, "k_gemm_i4: null pointer");
    // the reference's tile preconditions (src/k_gemm.hip:10-14)
    if (M <= 0 || N <= 0 || K <= 0 || M % 128 || N % 64 || K % 128)
        return fail(RT4_E_SHAPE, "k_gemm_i4: shape must be multiples of BM=128/BN=64/G=128 (M=%d N=%d K=%d)", M, N,
                    K);
    int rc = check_gemm_args("k_gemm_i4", M, N, K);
    if (rc) return rc;
    if (!aligned(aq, 4) || !aligned(wq, 16) || !aligned(c, 4) || !aligned(asc_gm, 4) || !aligned(wsc_gm, 4))
        return fail(RT4_E_ARG, "k_gemm_i4: misaligned pointer");
    // The same per-group integers as the reference's int4 x int4 contraction, from
    // the codes sign-extended to int8 (library scratch: the caller hands over no
    // buffer for them).
    hipStream_t st = as_stream(stream);
    void* q = nullptr;
    if ((rc = lib_scratch(kSlotGemmA, (size_t)M * K, &q, st))) return rc;
    hipError_t e = rt4::launch_hl_to_i8(static_cast<int8_t*>(q), nullptr, aq, M, K, st);
    if (e != hipSuccess) return hip_status(e, "k_gemm_i4 code expansion");
    return run_gemm("k_gemm_i4 launch", nullptr, c, wq, wsc_gm, static_cast<const int8_t*>(q), asc_gm, M, N, K, st);
}


int rt4_gemm_w4a8_i8(float* c, const uint32_t* wq, const float* wsc_gm, const int8_t* xq,
                     const float* sc, int M, int N, int K, void* stream) {
    return gemm_i8_common("rt4_gemm_w4a8_i8", nullptr, c, wq, wsc_gm, xq, sc, M, N, K, stream);
}

int rt4_gemm_w4a8_groupsums(int32_t* gsum, float* c, const uint32_t* wq, const float* wsc_gm,
                            const int8_t* xq, const float* sc, int M, int N, int K, void* stream) {
    if (!gsum) return fail(RT4_E_ARG, "rt4_gemm_w4a8_groupsums: null pointer");
    return gemm_i8_common("rt4_gemm_w4a8_groupsums", gsum, c, wq, wsc_gm, xq, sc, M, N, K, stream);
}

int rt4_gemm_w4a8(float* c, float* c2, const uint32_t* wq, const float* wsc_gm, const uint32_t* ah,
                  const uint32_t* al, const float* sc, const float* sc16, int M, int N, int K,
                  void* stream) {
    if (!c || !c2 || !wq || !wsc_gm || !ah || !al || !sc || !sc16)
        return fail(RT4_E_ARG, "k_gemm_i4_a8: null pointer");
    // the reference's tile preconditions (src/k_gemm.hip:24-28)
    if (M <= 0 || N <= 0 || K <= 0 || M % 128 || N % 64 || K % 128)
        return fail(RT4_E_SHAPE, "k_gemm_i4_a8: shape must be multiples of BM=128/BN=64/G=128 (M=%d N=%d K=%d)",
                    M, N, K);
    int rc = check_gemm_args("k_gemm_i4_a8", M, N, K);
    if (rc) return rc;
    if (!aligned(ah, 4) || !aligned(al, 4) || !aligned(c2, 16))
        return fail(RT4_E_ARG, "k_gemm_i4_a8: misaligned pointer");
    // Recombine the digit planes into int8 codes q8 = 16h + l.  The caller's c2
    // (M*N floats of scratch, src/k_gemm.hip:31) holds them when large enough.
    const size_t need = (size_t)M * K;
    hipStream_t st = as_stream(stream);
    void* q = c2;
    if ((size_t)M * N * sizeof(float) < need && (rc = lib_scratch(kSlotGemmA, need, &q, st))) return rc;
    hipError_t e = rt4::launch_hl_to_i8(static_cast<int8_t*>(q), ah, al, M, K, st);
    if (e != hipSuccess) return hip_status(e, "k_gemm_i4_a8 digit recombination");
    return run_gemm("k_gemm_i4_a8 launch", nullptr, c, wq, wsc_gm, static_cast<const int8_t*>(q), sc, M, N, K, st);
}

int rt4_make_group_major(float* wsc_gm, const uint16_t* ws, int N, int K, void* stream) {
    if (!wsc_gm || !ws) return fail(RT4_E_ARG, "rt4_make_group_major: null pointer");
    if (N <= 0 || K <= 0 || K % 128) return fail(RT4_E_SHAPE, "rt4_make_group_major: N=%d K=%d", N, K);
    return hip_status(rt4::launch_make_group_major(wsc_gm, ws, N, K / 128, as_stream(stream)),
                      "rt4_make_group_major launch");
}

// ------------------------------------------------------------- attention --

int rt4_attn_q_quant(uint32_t* qq, float* qs, const float* x, int T, int H, int D, int G, int TP,
                     void* stream) {
    if (!qq || !qs || !x) return fail(RT4_E_ARG, "k_attn_q_quant: null pointer");
    if (G != 64 && G != 128 && G != 256) return fail(RT4_E_ARG, "k_attn_q_quant: group G=%d unsupported", G);
    if (T < 0 || H < 1 || D <= 0 || D % G || TP < T)
        return fail(RT4_E_SHAPE, "k_attn_q_quant: T=%d H=%d D=%d G=%d TP=%d", T, H, D, G, TP);
    if (!aligned(x, 4) || !aligned(qq, 4) || !aligned(qs, 4)) return fail(RT4_E_ARG, "k_attn_q_quant: misaligned");
    return hip_status(rt4::launch_attn_q_quant(qq, qs, x, T, H, D, G, TP, as_stream(stream)), "k_attn_q_quant launch");
}

int rt4_kv_append_k(uint32_t* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                    int kv_total, void* stream) {
    if (!kc || !ksc || !kf) return fail(RT4_E_ARG, "k_kv_append_k: null pointer");
    if (G != 64 && G != 128 && G != 256) return fail(RT4_E_ARG, "k_kv_append_k: group G=%d unsupported", G);
    if (t0 < 0 || T < 0 || H < 1 || D <= 0 || D % G || (long long)t0 + T > kv_total)
        return fail(RT4_E_SHAPE, "k_kv_append_k: t0=%d T=%d H=%d D=%d G=%d kv_total=%d", t0, T, H, D, G, kv_total);
    return hip_status(rt4::launch_kv_append_k(kc, ksc, kf, t0, T, H, D, G, kv_total, as_stream(stream)),
                      "k_kv_append_k launch");
}

int rt4_kv_append_v(uint32_t* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H, int D,
                    int BG, int kv_total, void* stream) {
    if (!vc || !vsc || !stage || !vf) return fail(RT4_E_ARG, "k_kv_append_v: null pointer");
    if (t0 < 0 || T < 0 || H < 1 || D <= 0 || BG <= 0 || BG % 8 || kv_total % BG || (long long)t0 + T > kv_total ||
        (T > 0 && (t0 + T - 1) / BG - t0 / BG + 1 > 65535) || (D + 63) / 64 > 65535)
        return fail(RT4_E_SHAPE, "k_kv_append_v: t0=%d T=%d H=%d D=%d BG=%d kv_total=%d", t0, T, H, D, BG,
                    kv_total);
    return hip_status(rt4::launch_kv_append_v(vc, vsc, stage, vf, t0, T, H, D, BG, kv_total, as_stream(stream)),
                      "k_kv_append_v launch");
}

// The prefill kernel addresses one KV head's cache through 32-bit buffer offsets
// (kv_cap * 128 bytes of K codes, plus up to three tiles read past the end).
constexpr int kMaxKvCap = (1 << 24) - 64;
// Largest staged K/V copy the prefill allocates (4 GiB: 65536 tiles x KV heads).
constexpr size_t kMaxKvxBytes = (size_t)4 << 30;

int rt4_attention_prefill_cfg(float* out, const uint32_t* qq, const float* qsc, const uint32_t* kc,
                              const float* ksc, const uint32_t* vc, const float* vsc, int n_q, int n_kv, int off,
                              int n_tile, int n_heads, int ratio, int kv_cap, int kv_splits, void* stream) {
    if (!out || !qq || !qsc || !kc || !ksc || !vc || !vsc) return fail(RT4_E_ARG, "k_attention: null pointer");
    if (n_q < 64 || n_q % 64 || n_kv < 1 || n_kv > kv_cap || off < 0 || kv_cap % 64 || n_tile < 1 ||
        (long long)n_tile * 64 > kv_cap || n_heads < 1 || ratio < 1 || n_heads % ratio || n_q > 65535 * 64 ||
        n_heads > 65535 || kv_cap > kMaxKvCap)
        return fail(RT4_E_SHAPE,
                    "k_attention: n_q=%d (multiple of 64) n_kv=%d off=%d n_tile=%d n_heads=%d ratio=%d kv_cap=%d "
                    "(at most 16777152)",
                    n_q, n_kv, off, n_tile, n_heads, ratio, kv_cap);
    if (kv_splits < 0 || kv_splits > 64) return fail(RT4_E_ARG, "k_attention: kv_splits=%d (0..64)", kv_splits);
    if (!aligned(qq, 16) || !aligned(kc, 16) || !aligned(vc, 4) || !aligned(out, 16) || !aligned(qsc, 4) ||
        !aligned(ksc, 4) || !aligned(vsc, 4))
        return fail(RT4_E_ARG, "k_attention: misaligned pointer (qq, kc, out need 16 bytes)");
    int cus = 0, rc = device_cus(&cus);
    if (rc) return rc;
    hipStream_t st = as_stream(stream);
    int nsplit = kv_splits > 0 ? kv_splits : rt4::fa_splits(n_q, n_heads, n_tile, cus);
    // Under graph capture an automatic split count that would need a larger
    // workspace falls back to one split (no workspace; same algorithm, the fp32
    // sums of O and L in one order instead of a combine of partial ranges).
    if (nsplit > 1 && kv_splits == 0 && capturing(st) &&
        !(scratch_has(kSlotAttnPart, rt4::fa_part_bytes(n_q, n_heads, nsplit)) &&
          scratch_has(kSlotAttnCnt, rt4::fa_cnt_bytes(n_q, n_heads, nsplit))))
        nsplit = 1;
    void *part = nullptr, *cnt = nullptr;
    if (nsplit > 1 && ((rc = lib_scratch(kSlotAttnPart, rt4::fa_part_bytes(n_q, n_heads, nsplit), &part, st)) ||
                       (rc = lib_scratch(kSlotAttnCnt, rt4::fa_cnt_bytes(n_q, n_heads, nsplit), &cnt, st, true))))
        return rc;
    // The staged K/V copy for the DMA form (one staging pass per call instead of per
    // workgroup), up to kMaxKvxBytes; beyond that, or under capture while the copy
    // would have to grow, each workgroup stages its own tiles (same results).
    const size_t xb = rt4::fa_kvx_bytes(n_heads, ratio, n_tile);
    void* kvx = nullptr;
    if (xb <= kMaxKvxBytes && !(capturing(st) && !scratch_has(kSlotAttnKV, xb)) &&
        (rc = lib_scratch(kSlotAttnKV, xb, &kvx, st)))
        return rc;
    return hip_status(rt4::launch_fa_int4(out, qq, qsc, kc, ksc, vc, vsc, n_q, n_kv, off, n_tile, n_heads, ratio,
                                          kv_cap, nsplit, static_cast<float*>(part), static_cast<int*>(cnt), kvx, st),
                      "k_attention launch");
}

int rt4_attention_prefill(float* out, const uint32_t* qq, const float* qsc, const uint32_t* kc,
                          const float* ksc, const uint32_t* vc, const float* vsc, int n_q, int n_kv, int off,
                          int n_tile, int n_heads, int ratio, int kv_cap, void* stream) {
    return rt4_attention_prefill_cfg(out, qq, qsc, kc, ksc, vc, vsc, n_q, n_kv, off, n_tile, n_heads, ratio, kv_cap,
                                     0, stream);
}

}  // extern "C"
