// attn.hip -- int4-KV causal FlashAttention prefill, gfx950 (its feeders, the Q
// quantizer and the K/V cache appends, are in attn_feed.hip).
//
// Formats (the reference's KV cache, kernels/flash_attn_core.h:74-112 and
// src/k_new.hip:228-399; head dim D = 256, quantization group 128 along D):
//   qq  u32 [H][TP][32]      Q int4 codes, 8 dims per dword, low nibble = even dim
//   qsc f32 [H][2][TP]       Q scale per (row, 128-dim group), s = amax/7
//   kc  u32 [KVH][cap][32]   K codes, same packing;  ksc f32 [KVH][2][cap]
//   vc  u32 [KVH][cap/8][256] V codes transposed: dword = 8 consecutive keys of
//                             one dim, low nibble = even key
//   vsc f32 [KVH][cap/64][256] V scale per (64-key tile, dim)
//   out f32 [H][TP][256]
//
// Prefill kernel (restates fa_int4, kernels/flash_attn_core.h:74-435).  Per
// 64-key tile and query row: S = Σ_g I_g·sq_g·sk_g over the two 128-dim groups
// (I_g exact int32 dot products of the codes), causal mask, tile row max mt,
// P = clamp(int(7·2^((S-mt)·log2e) + 0.5), 0, 7), online rescale alpha =
// 2^((r_old-r_new)·log2e), beta = 2^((mt-r_new)·log2e), L = L·alpha + Σp·beta/7,
// O = O·alpha + (Σ_k P·Vcode)·(beta/7)·vsc; out = O / L.
//
// MI355X design.  A workgroup is 64 query rows of one head, 4 waves of 16 rows.
// Both contractions run on v_mfma_f32_16x16x128_f8f6f4 with FP8 E4M3 operands
// that hold the integer codes exactly, so the products come out as fp32 with no
// int-to-float conversion:
//   - K and V codes c enter as the byte c + 8 (the nibble xor 8), which is the
//     E4M3 encoding of (c + 8)·2^-9: the subnormals 0..7 and the first normal
//     binade 8..15 are spaced 2^-9 apart.  The offset's contribution, 8 times the
//     other operand's sum, is taken off through the accumulator input C.
//   - Q codes enter as their exact E4M3 values (converted once), P codes 0..7 as
//     the subnormals p·2^-9, which v_cvt_scalef32_pk_fp8_f32 (scale 512) produces
//     from p rounded to the nearest code.
// Every partial sum is an integer times a power of two below 2^24, so each
// MFMA result is exact.  The contractions are in transposed form so that a lane
// always owns one query row:
//   S^T[key][q] = K·Q^T   one MFMA per subtile of 16 keys and 128-dim group
//                         (K = 128 is the quantization group), A = K operand
//                         bytes, B = the wave's resident Q bytes, C = -8·Σq·2^-9;
//                         result I·2^-9.  A lane holds query q = lane%16 and, in
//                         register r of subtile t, key 16t + 8(G/2) + 2r + G%2
//                         (G = lane/16): the K rows are fed in that order, so
//                         lane group G holds the even (G even) or odd keys of
//                         one 8-key group.
//   O^T[d][q]  = V^T·P^T  the 64 keys of a tile fill half of K = 128: B = P
//                         straight from those registers (the lane's 16 keys) in
//                         one half and zeros in the other, A = the V operands of
//                         two dim tiles laid out in LDS with the same key order
//                         (one per half), so one A register block serves two
//                         MFMAs; C = -8·ΣP·2^-18 from a fifth MFMA against
//                         -2^-6 bytes, which also gives the row sum of P.  With
//                         that key order a V operand dword is exactly the even-
//                         or odd-key bytes of one V cache dword.
// Row max over a query's 64 keys is 15 in-lane ops plus two cross-lane steps
// (xor 16, xor 32).  The K/V tiles reach LDS in MFMA operand order (16 bytes per
// (subtile, group, half, lane)), so the waves only issue ds_read_b128 of ready
// operands.  A pre-pass (fa_expand_kv_k) unpacks every tile once per call into a
// copy in memory with exactly that layout, and the workgroups move each tile into
// LDS with global_load_lds_dwordx4 (no registers, no unpacking, no LDS stores):
// unpacking in every workgroup repeated it once per query block and split, about a
// tenth of the kernel at C4.  Without room for the copy (graph capture before the
// first eager call, or a copy beyond 4 GiB) each workgroup stages its tiles itself
// from the packed cache, with the same bytes.  Tiles past the workgroup's last query
// position are skipped: the reference processes them but every entry is masked,
// which leaves its state bit-for-bit unchanged.  The tile loop is a two-tile
// pipeline (S and P of the next tile beside the PV product of the current one;
// see the loop), the scale products of both contractions run on
// v_mfma_f32_16x16x1f32 (four 16x16 tiles per instruction: 2 per tile for S, 4
// for O; four v_mfma_f32_4x4x1f32 cost about twice the matrix-core time of one),
// and K/V are read with range-checked buffer loads.  The power-of-two factors of
// the operand encodings (2^-9 for S, 2^-18 for O) are folded into the Q scale and
// the P scale, so every rounded operation is the one the integer form had.  The
// online rescale keeps its reference until a tile max exceeds it by more than 8
// (log2 units): the same O / L as the reference's running-max form, rounded
// differently, with the 64-multiply rescale of O rare instead of frequent.
#include <type_traits>

#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

namespace {

constexpr int HD = 256;           // head dim
constexpr int KDW = HD / 8;       // dwords per K / Q row
constexpr int BNK = 64;           // keys per tile
constexpr int QROWS = 64;         // query rows per workgroup
constexpr int NTA = 256;          // 4 waves
constexpr float L2E = 1.4426950408889634f;
constexpr int KU_BYTES = 4 * 4 * 64 * 16;   // unpacked K operands of one tile
constexpr int VU_BYTES = 16 * 64 * 16;      // unpacked V operands of one tile
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef short v2s __attribute__((ext_vector_type(2)));

// D = A·B + C on 16x16x128 FP8 E4M3 operands (format 0 for both, no block scale).
__device__ __forceinline__ v4f mfma_e4m3(v8i a, v8i b, v4f c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
__device__ __forceinline__ v8i cat8(v4i lo, v4i hi) {
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// Offset-code bytes of one code dword w8 = w ^ 0x88888888 (every nibble c -> c + 8):
// nibbles 0, 2, 4, 6 (even) or 1, 3, 5, 7 (odd) as the bytes c + 8 = E4M3 of (c + 8)·2^-9.
__device__ __forceinline__ uint32_t even_e4m3(uint32_t w8) { return w8 & 0x0F0F0F0Fu; }
__device__ __forceinline__ uint32_t odd_e4m3(uint32_t w8) { return (w8 >> 4) & 0x0F0F0F0Fu; }
// E4M3 encoding of an integer -8..8: magnitudes 0..7 are the bytes 00 38 40 44 48
// 4A 4C 4E (exponent bias 7, 3 mantissa bits), 8 is 0x50; sign in bit 7.
__device__ __forceinline__ uint32_t e4m3_of_int(int c) {
    const uint32_t m = (uint32_t)(c < 0 ? -c : c);
    const uint32_t b = m < 8 ? (uint32_t)(0x4E4C4A4844403800ull >> (8 * m)) & 0xFFu : 0x50u;
    return b | (c < 0 ? 0x80u : 0u);
}

// Key order within a 16-key subtile: output register r of lane group G holds key
// key_of_slot(G, r); the K row fed to the MFMA at slot 4G + r is that key.
__device__ __forceinline__ int key_of_slot(int G, int r) { return 8 * (G >> 1) + 2 * r + (G & 1); }
__device__ __forceinline__ int slot_of_key(int k) { return 4 * (2 * (k >> 3) + (k & 1)) + ((k & 7) >> 1); }

// Products x[4G + r] * y[i] for four 16x16 tiles b in their accumulator layout
// (lane l = 16G + i holds rows 4G..4G+3 of column i, tile b in registers 4b..4b+3),
// on the matrix core: v_mfma_f32_16x16x1f32 (four blocks, k = 1) gives lane l,
// register 4b + r, the A operand of lane 16b + 4(l >> 4) + r times the B operand of
// lane 16b + (l & 15) (lane layout checked on the card), so tile b's x[j] comes
// from lane 16b + j and every lane supplies its own column's y.  Each output is the
// one fp32 rounding of the product, as a v_mul_f32 would give.
__device__ __forceinline__ v16f outer16(float x_of_lane, float y) {
    const v16f z = {};
    return __builtin_amdgcn_mfma_f32_16x16x1f32(x_of_lane, y, z, 0, 0, 0);
}

__device__ __forceinline__ int sext4(uint32_t w, int e) { return ((int)(w << (28 - 4 * e))) >> 28; }

constexpr int kRsrcW3 = 0x00020000;    // dword 3 of a buffer resource: 32-bit data format

// The staged form of a 64-key tile: the MFMA operand bytes in the order the waves
// read them, 16 KB for K and 16 KB for V.  These write one thread's share of a
// tile's block (in LDS, or its copy in memory for the DMA path).
//
// K: key kk = tid % 64, dims 64p .. 64p + 63 (p = tid / 64, code dwords j = 0..7,
// k0 then k1): group p/2, lane group G' = 2(p%2) + j/4 of the operand, half (j/2)%2
// of its 32 bytes.  Piece (subtile, group, half) is 64 lanes x 16 bytes; the key's
// lane in it is 16G' + slot of kk%16.  Every nibble c becomes the byte c + 8.
__device__ __forceinline__ void put_k_slots(unsigned char* blk, v4u k0, v4u k1, int tid) {
    const int kk = tid & 63, p = tid >> 6;
    const uint32_t d[8] = {k0.x ^ 0x88888888u, k0.y ^ 0x88888888u, k0.z ^ 0x88888888u, k0.w ^ 0x88888888u,
                           k1.x ^ 0x88888888u, k1.y ^ 0x88888888u, k1.z ^ 0x88888888u, k1.w ^ 0x88888888u};
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const uint4 v = make_uint4(even_e4m3(d[2 * g]), odd_e4m3(d[2 * g]), even_e4m3(d[2 * g + 1]),
                                   odd_e4m3(d[2 * g + 1]));
        const int piece = ((kk >> 4) * 2 + (p >> 1)) * 2 + (g & 1);
        *reinterpret_cast<uint4*>(blk + (piece * 64 + 16 * (2 * (p & 1) + (g >> 1)) + slot_of_key(kk & 15)) * 16) = v;
    }
}
// V: dim tid, the code dwords of its eight 8-key groups.  Lane G*16 + d%16 of dim
// tile d/16 gets, in dword t = 0..3, the offset-code bytes of the even (G even) or
// odd keys of 8-key group 2t + G/2 -- keys 16t + key_of_slot(G, r), r = 0..3, as P
// holds them.
__device__ __forceinline__ void put_v_slots(unsigned char* blk, const uint32_t (&vw)[8], int tid) {
    uint32_t e[8], o[8];
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t w8 = vw[g] ^ 0x88888888u;
        e[g] = even_e4m3(w8);
        o[g] = odd_e4m3(w8);
    }
#pragma unroll
    for (int G = 0; G < 4; G++) {
        const uint32_t* src = (G & 1) ? o : e;
        const uint4 v = make_uint4(src[G >> 1], src[2 + (G >> 1)], src[4 + (G >> 1)], src[6 + (G >> 1)]);
        *reinterpret_cast<uint4*>(blk + ((tid >> 4) * 64 + G * 16 + (tid & 15)) * 16) = v;
    }
}

}  // namespace

// ---------------------------------------------------------------- prefill --

template <bool DMA>
__global__ __launch_bounds__(NTA, 2) void fa_int4_k(const uint32_t* __restrict__ qq,
                                                    const float* __restrict__ qsc,
                                                    const uint32_t* __restrict__ kc,
                                                    const float* __restrict__ ksc,
                                                    const uint32_t* __restrict__ vc,
                                                    const float* __restrict__ vsc, float* __restrict__ out,
                                                    int n_q, int n_kv, int off, int n_tile, int ratio,
                                                    int kv_cap, int nsplit, float* __restrict__ opart,
                                                    float2* __restrict__ mlpart, int* __restrict__ cnt,
                                                    const unsigned char* __restrict__ kx,
                                                    const unsigned char* __restrict__ vx) {
    __shared__ __align__(16) unsigned char ku[2 * KU_BYTES];   // x2: [subtile][k-step][lane] x 16 B
    __shared__ __align__(16) unsigned char vu[2 * VU_BYTES];   // x2: [dim tile][lane] x 16 B
    __shared__ __align__(16) float ks_l[2][2 * BNK];
    __shared__ __align__(16) float vs_l[2][HD];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, w = uniform(tid >> 6);
    const int qi = lane & 15, G = lane >> 4;
    // the key whose scale this lane supplies to the S scale products: outer16 gives
    // lane l, register 4kt + r, the operand of lane 16kt + 4(l >> 4) + r, so lane j
    // supplies the key of register j & 3 of lane group (j >> 2) & 3 in subtile j >> 4
    const int kslot = 16 * G + key_of_slot((lane >> 2) & 3, lane & 3);
    const int head = blockIdx.y, vh = head / ratio;
    const int q0 = blockIdx.x * QROWS;
    const int qrow = q0 + 16 * w + qi;
    qq += (size_t)head * n_q * KDW;
    qsc += (size_t)head * 2 * n_q;
    kc += (size_t)vh * kv_cap * KDW;
    ksc += (size_t)vh * 2 * kv_cap;
    vc += (size_t)vh * (kv_cap / 8) * HD;
    vsc += (size_t)vh * (kv_cap / BNK) * HD;
    out += (size_t)head * n_q * HD;

    // tiles holding keys at or before this workgroup's last query position
    int nt = (off + q0 + QROWS - 1) / BNK + 1;
    nt = nt < n_tile ? nt : n_tile;
    // split-KV: this workgroup takes tiles [t0, t1) of them
    const int split = blockIdx.z;
    const int t0 = (int)((long long)nt * split / nsplit), t1 = (int)((long long)nt * (split + 1) / nsplit);

    // Resident Q operand of group g: dims 128g + 32G .. +31, the 4 code dwords w_m
    // (dims 8m..8m+7 of that range) as E4M3 bytes in the order even(w0) odd(w0)
    // even(w1) ... odd(w3), the order the K operand bytes are staged in.  cS[g] =
    // -8·Σq·2^-9 over the group's 128 dims takes the K offset back off.
    v8i qop[2];
    float cS[2];
#pragma unroll
    for (int g = 0; g < 2; g++) {
        const uint4 wd = *reinterpret_cast<const uint4*>(qq + (size_t)qrow * KDW + 16 * g + 4 * G);
        const uint32_t w[4] = {wd.x, wd.y, wd.z, wd.w};
        int qs = 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            uint32_t ev = 0, od = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int ce = sext4(w[m], 2 * j), co = sext4(w[m], 2 * j + 1);
                qs += ce + co;
                ev |= e4m3_of_int(ce) << (8 * j);
                od |= e4m3_of_int(co) << (8 * j);
            }
            qop[g][2 * m] = (int)ev;
            qop[g][2 * m + 1] = (int)od;
        }
        qs += __shfl_xor(qs, 16);
        qs += __shfl_xor(qs, 32);
        cS[g] = (float)(-8 * qs) * (1.f / 512.f);
    }
    // S in log2 units: fold log2(e) and the 2^9 of the offset K operand into the Q scales
    const float A0 = qsc[qrow] * (L2E * 512.f), A1 = qsc[n_q + qrow] * (L2E * 512.f);

    float O[16][4];
#pragma unroll
    for (int dt = 0; dt < 16; dt++)
#pragma unroll
        for (int r = 0; r < 4; r++) O[dt][r] = 0.f;
    float rref = -1e30f, L = 0.f;

    // Pipeline over the 64-key tiles.  P of a tile uses that tile's own max, so
    // S, the mask, the tile max and P of tile t+1 do not depend on tile t: each
    // iteration runs the O update and PV product of tile t ("back") beside S and P
    // of tile t+1 ("front"), two independent chains for the scheduler.  K runs one
    // tile ahead of V: during iteration t the LDS buffers hold K(t+1) (read by
    // front) and V(t) (read by back) while the other K and V buffers take K(t+2)
    // and V(t+1) from registers staged during the previous iteration, whose global
    // loads (K(t+3), V(t+2)) are issued right after; one barrier per tile orders
    // every write after the reads of the buffer's previous tile.  Loads and stores
    // past the split's last tile are harmless (range-checked buffer loads, LDS
    // slots nobody reads) and are left unguarded, so an iteration is one basic
    // block apart from the O rescale, which comes first.
    struct StageK {
        v4u k0, k1;                     // key tid%64, dwords 8p..8p+7 (p = tid/64)
        float ks;
    };
    struct StageV {
        uint32_t v[8];                  // dim tid, 8-key groups 0..7
        float vs;
    };
    // Buffer loads: a per-lane offset fixed for the whole loop plus a per-tile
    // scalar offset, and the buffer's range check (which includes the scalar
    // offset) supplies the reference's zero codes -- the K resource ends at key
    // n_kv, the V resource at the last whole 8-key group (flash_attn_core.h:
    // 143-152), so reads past them return 0 with no memory access.  Scales past
    // kv_cap are replaced by 1 when the stage is unpacked.  No load is conditional
    // or clamped: selecting right after a load, or loading under a condition,
    // makes the compiler wait for the load there, which would defeat the prefetch.
    const __amdgpu_buffer_rsrc_t rs_k =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(kc), 0, n_kv * KDW * 4, kRsrcW3);
    const __amdgpu_buffer_rsrc_t rs_v =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(vc), 0, (n_kv / 8) * HD * 4, kRsrcW3);
    const __amdgpu_buffer_rsrc_t rs_ks =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ksc), 0, 2 * kv_cap * 4, kRsrcW3);
    const __amdgpu_buffer_rsrc_t rs_vs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vsc), 0, (kv_cap / BNK) * HD * 4, kRsrcW3);
    const int off_k = ((tid & 63) * KDW + 8 * (tid >> 6)) * 4;          // + tile * BNK * KDW * 4
    const int off_ks = (((tid >> 6) & 1) * kv_cap + (tid & 63)) * 4;    // + tile * BNK * 4
    // Tile byte offsets are formed in 32-bit unsigned arithmetic: the prefetch reads
    // up to three tiles past the last one, and at the largest accepted cache
    // (kv_cap = 2^24 - 64) that tile's K offset is 2^31, beyond int.  The range check
    // compares the unsigned offset with the resource's size, so such a tile reads
    // zeros (checked on the CPU by tests/test_attention.py).
    auto load_k = [&](StageK& S, int t) {
        const int sk = (int)((uint32_t)t * (uint32_t)(BNK * KDW * 4));
        if constexpr (!DMA) {
            S.k0 = __builtin_amdgcn_raw_buffer_load_b128(rs_k, off_k, sk, 0);
            S.k1 = __builtin_amdgcn_raw_buffer_load_b128(rs_k, off_k + 16, sk, 0);
        }
        S.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_ks, off_ks, t * BNK * 4, 0));
    };
    auto load_v = [&](StageV& S, int t) {
        const int sv = (int)((uint32_t)t * (uint32_t)(BNK / 8 * HD * 4));
        if constexpr (!DMA) {
#pragma unroll
            for (int g = 0; g < 8; g++)
                S.v[g] = __builtin_amdgcn_raw_buffer_load_b32(rs_v, tid * 4 + (g & 3) * HD * 4,
                                                              sv + (g >> 2) * 4 * HD * 4, 0);
        }
        S.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_vs, tid * 4, t * HD * 4, 0));
    };
    auto store_k = [&](const StageK& S, int b, int t) {
        // codes (unless DMA brings them) and scales; keys >= n_kv read as zero codes
        // (flash_attn_core.h:143-147), i.e. bytes 8
        if constexpr (!DMA) put_k_slots(ku + b * KU_BYTES, S.k0, S.k1, tid);
        if (tid < 2 * BNK) ks_l[b][tid] = t * BNK + (tid & 63) < kv_cap ? S.ks : 1.f;
    };
    auto store_v = [&](const StageV& S, int b, int t) {
        // a group of 8 keys is read only if it is whole (flash_attn_core.h:150-152),
        // else zero codes
        if constexpr (!DMA) put_v_slots(vu + b * VU_BYTES, S.v, tid);
        vs_l[b][tid] = t < kv_cap / BNK ? S.vs : 1.f;
    };
    // DMA path: tiles t of K and V as staged blocks from the expanded copy (kx, vx:
    // [KV head][tile][16 KB]) straight into LDS buffers bk / bv, one 1 KB piece per
    // instruction, four per wave.  Tiles past the last one (the prefetch runs ahead)
    // read the last tile instead, into buffers nobody reads.
    auto dma_k = [&](int t, int b) {
        t = t < n_tile - 1 ? t : n_tile - 1;
        const unsigned char* src = kx + ((size_t)vh * n_tile + t) * KU_BYTES;
        const uint32_t dst = lds_addr(ku) + b * KU_BYTES + 4 * w * 1024;
        dma16<0>(lane * 16 + 4 * w * 1024, src, dst);
        dma16<1024>(lane * 16 + (4 * w + 1) * 1024, src, dst);
        dma16<2048>(lane * 16 + (4 * w + 2) * 1024, src, dst);
        dma16<3072>(lane * 16 + (4 * w + 3) * 1024, src, dst);
    };
    auto dma_v = [&](int t, int b) {
        t = t < n_tile - 1 ? t : n_tile - 1;
        const unsigned char* src = vx + ((size_t)vh * n_tile + t) * VU_BYTES;
        const uint32_t dst = lds_addr(vu) + b * VU_BYTES + 4 * w * 1024;
        dma16<0>(lane * 16 + 4 * w * 1024, src, dst);
        dma16<1024>(lane * 16 + (4 * w + 1) * 1024, src, dst);
        dma16<2048>(lane * 16 + (4 * w + 2) * 1024, src, dst);
        dma16<3072>(lane * 16 + (4 * w + 3) * 1024, src, dst);
    };

    const v4f cS0 = {cS[0], cS[0], cS[0], cS[0]}, cS1 = {cS[1], cS[1], cS[1], cS[1]};
    // front of tile t (K in buffer b): S^T = K Q^T for the 4 subtiles of 16 keys,
    // the causal mask (MASK: the tile may reach past a row of this workgroup), the
    // tile max m of each row, the P codes as the PV operand and -8·ΣP·2^-18.
    struct Front {
        v8i p_lo, p_hi; // the P codes in the low / high half of a PV operand, zeros in the other
        float m;
        v4f corr;       // the same value in all four registers (every output row)
    };
    auto front = [&](int t, int b, auto mask_tag) -> Front {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int kb = t * BNK;
        const unsigned char* kub = ku + b * KU_BYTES;
        const float* ksb = ks_l[b];
        float sv[4][4];
        // key scale x query scale of every entry (subtile kt in registers 4kt..4kt+3)
        const v16f c0 = outer16(ksb[kslot], A0);
        const v16f c1 = outer16(ksb[BNK + kslot], A1);
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            // pieces (kt, group, half) at ((kt * 2 + group) * 2 + half) * 64
            const v4i* kp = reinterpret_cast<const v4i*>(kub) + (kt * 4) * 64 + lane;
            const v4f a0 = mfma_e4m3(cat8(kp[0], kp[64]), qop[0], cS0);
            const v4f a1 = mfma_e4m3(cat8(kp[128], kp[192]), qop[1], cS1);
#pragma unroll
            for (int r = 0; r < 4; r++) sv[kt][r] = fmaf(a1[r], c1[4 * kt + r], a0[r] * c0[4 * kt + r]);
        }
        if constexpr (MASK) {
            if (kb + BNK - 1 > off + q0 + 16 * w) {     // this wave has masked entries in the tile
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (kb + 16 * kt + key_of_slot(G, r) > off + qrow) sv[kt][r] = -__builtin_inff();
            }
        }
        // ---- tile row max over the 64 keys of this lane's query
        float m = sv[0][0];
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) m = fmaxf(m, sv[kt][r]);
        {   // xor 16 and xor 32 partners: each swap leaves a lane its value and its partner's
            const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
            m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
            const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
            m = fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
        }
        // Fully masked row in this tile: take the running reference (the state after
        // the previous tile), so nothing is rescaled and every P is 2^(-inf) = 0.  (The
        // reference masks with -1e30 and reaches this only after a visible tile;
        // -inf gives the same P there and also keeps a row that has seen nothing
        // yet -- possible at the start of a KV split -- at zero.)
        if (m < -1e29f) m = rref;
        // ---- P = clamp(int(7 * 2^(S - m) + 0.5), 0, 7), packed as the PV operand,
        // with the 7 inside the exponent: p = 2^(S - (m - log2 7)).  That moves p by
        // a few ulp, which can flip a code where 7 * 2^(S - m) + 0.5 lies within them
        // of an integer, as the exp2 itself (v_exp_f32, within 1 ulp) already does
        // against the reference's.  v_cvt_scalef32_pk_fp8_f32 with scale 512 gives
        // the E4M3 byte of p/512 rounded to the nearest subnormal, i.e. p rounded to
        // the nearest integer code, as the byte of that code (ties go to even where
        // the reference rounds up: p exactly k + 1/2, inside the few-ulp band above).
        // The clamp never binds: m is the max of the row's S (fmaxf returns one of
        // its operands), so S - m <= 0 and p <= 7 (1 + a few ulp) < 7.5; a fully
        // masked row has m = rref, S - m = -inf and P = 0.
        const float m7 = m - 2.807354922057604f;   // m - log2(7)
        uint32_t pk[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            // v_exp_f32 directly: the arguments are <= log2 7 and any result below
            // 0.5 converts to code 0, so denormal handling is irrelevant here
            float p[4];
#pragma unroll
            for (int r = 0; r < 4; r++) p[r] = __builtin_amdgcn_exp2f(sv[kt][r] - m7);
            v2s w;
            asm volatile("" : "=v"(w));          // both halves are written below
            w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, p[0], p[1], 512.f, false);
            w = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(w, p[2], p[3], 512.f, true);
            pk[kt] = __builtin_bit_cast(uint32_t, w);
        }
        Front f;
        f.p_lo = v8i{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3], 0, 0, 0, 0};
        f.p_hi = v8i{0, 0, 0, 0, (int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]};
        f.m = m;
        // -8·Σ_k P·2^-18 of the row over the tile's 64 keys on the matrix pipe: A
        // bytes -2^-6 (E4M3 0x88) against the P bytes give it in every output row.
        // Two chained 16x16x32 FP8 MFMAs over the code dwords as they are (a lane's
        // column is its query row, as in the PV operand): their 2-register constant
        // operand is kept, where the 8-register one of a 16x16x128 MFMA was rebuilt
        // with moves every tile.  Every product and partial sum is exact.
        const long neg2 = (long)0x8888888888888888ull;
        const v4f c01 = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
            neg2, (long)(((uint64_t)pk[1] << 32) | pk[0]), v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        f.corr = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(neg2, (long)(((uint64_t)pk[3] << 32) | pk[2]), c01,
                                                            0, 0, 0);
        return f;
    };
    // Online update with a tile's (m, -8·ΣP·2^-18): the running reference, L, and O
    // rescaled by alpha.  Returns the P scale beta/7 times the 2^18 of the PV
    // operand bytes.
    //
    // The running reference rref moves only when a tile max exceeds it by more than
    // 8 (log2 units) in some row of the wave; otherwise beta = 2^(m - rref) <= 2^8
    // carries the difference.  O and L are then both 2^(max - rref) times the
    // reference's (flash_attn_core.h, running max), so O / L and the split combine
    // (which rescales by the stored rref) are the same quantities, rounded
    // differently; the rescale of O (64 multiplies) runs a few times per split
    // instead of on about a third of the tiles (configs[4] 802 -> 764 us).  With
    // beta <= 2^8, O stays finite for V scales below about 10^28.
    auto update = [&](const Front& f) -> float {
        if (__any(f.m > rref + 8.f)) {      // a wave-uniform branch
            const float r_new = fmaxf(rref, f.m);
            // v_exp_f32 directly: the argument is <= 0, and a factor below 2^-126
            // (flushed to zero) scales contributions that no longer count
            const float alpha = __builtin_amdgcn_exp2f(rref - r_new);
            L *= alpha;
            rref = r_new;
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++) O[dt][r] *= alpha;
        }
        const float beta = __builtin_amdgcn_exp2f(f.m - rref);
        const float pb = beta * (1.f / 7.f);
        L += (f.corr[0] * -32768.f) * pb;     // corr * -2^15 = ΣP exactly
        return pb * 262144.f;
    };
    // back: O^T += (V^T P^T) * vsc * pbv per dim tile, V in buffer b.  One A
    // register block holds the V operands of dim tiles 2j and 2j + 1 (halves 0 and
    // 1); the MFMA of tile 2j takes B = (P, 0), that of 2j + 1 B = (0, P), and both C
    // = -8·ΣP·2^-18, so each result is ΣP·c·2^-18.  The V operands of the next four
    // dim tiles are read while the current four are multiplied and folded (left to
    // itself the compiler reads each pair just before its MFMAs and waits for it).
    auto back = [&](const v8i p_lo, const v8i p_hi, const v4f cc, float pbv, int b) {
        const unsigned char* vub = vu + b * VU_BYTES;
        const float* vsb = vs_l[b];
        // raised issue priority over the PV block: the other wave on the SIMD then
        // fills the matrix-core gaps with its S/P work (configs[4] 830 -> 816 us)
        __builtin_amdgcn_s_setprio(1);
        v4i vn[4];
#pragma unroll
        for (int d4 = 0; d4 < 4; d4++) vn[d4] = *(reinterpret_cast<const v4i*>(vub) + d4 * 64 + lane);
#pragma unroll
        for (int dq = 0; dq < 4; dq++) {
            v4i vcur[4];
#pragma unroll
            for (int d4 = 0; d4 < 4; d4++) vcur[d4] = vn[d4];
            if (dq < 3) {
#pragma unroll
                for (int d4 = 0; d4 < 4; d4++) vn[d4] = *(reinterpret_cast<const v4i*>(vub) + (4 * dq + 4 + d4) * 64 + lane);
            }
            const v16f ps = outer16(vsb[64 * dq + lane], pbv);   // vsc * pbv of dim tiles 4dq..4dq+3
#pragma unroll
            for (int d2 = 0; d2 < 4; d2 += 2) {
                const v8i a = cat8(vcur[d2], vcur[d2 + 1]);
                const v4f acc0 = mfma_e4m3(a, p_lo, cc);
                const v4f acc1 = mfma_e4m3(a, p_hi, cc);
                const int dt = 4 * dq + d2;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    O[dt][r] = fmaf(acc0[r], ps[4 * d2 + r], O[dt][r]);
                    O[dt + 1][r] = fmaf(acc1[r], ps[4 * d2 + 4 + r], O[dt + 1][r]);
                }
            }
        }
        __builtin_amdgcn_s_setprio(0);
    };

    if (t0 < t1) {      // uniform over the workgroup
        // tiles from t_mask on may reach past the position of some row of this
        // workgroup (row q0 of wave 0 is the first): their front takes the masked form
        const int t_mask = (off + q0 + 1) / BNK;
        StageK sk;
        StageV sv;
        if constexpr (DMA) {
            dma_k(t0, t0 & 1);
            dma_v(t0, t0 & 1);
            dma_k(t0 + 1, (t0 + 1) & 1);
        }
        load_k(sk, t0);
        load_v(sv, t0);
        store_k(sk, t0 & 1, t0);
        store_v(sv, t0 & 1, t0);
        load_k(sk, t0 + 1);
        store_k(sk, (t0 + 1) & 1, t0 + 1);
        load_k(sk, t0 + 2);
        load_v(sv, t0 + 1);
        if constexpr (DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        Front f = t0 >= t_mask ? front(t0, t0 & 1, std::true_type{}) : front(t0, t0 & 1, std::false_type{});
        __syncthreads();     // K buffer t0&1 is rewritten in the first iteration
        auto step = [&](int t, const Front& fc, auto mask_tag) -> Front {
            const float pbv = update(fc);
            store_k(sk, t & 1, t + 2);
            store_v(sv, (t + 1) & 1, t + 1);
            // K(t + 2) into the buffer K(t) left, V(t + 1) into the one V(t - 1) left.
            // Issued after the scale stores above: the compiler does not count these
            // loads, and its wait for the scale loads it issued last iteration would
            // otherwise wait for them too.
            if constexpr (DMA) {
                dma_k(t + 2, t & 1);
                dma_v(t + 1, (t + 1) & 1);
            }
            load_k(sk, t + 3);
            load_v(sv, t + 2);
            // keep the loads here: left to itself the compiler sinks them next to
            // their use at the top of the next iteration, exposing their latency
            asm volatile("" ::: "memory");
            const Front fn = front(t + 1, (t + 1) & 1, mask_tag);
            back(fc.p_lo, fc.p_hi, fc.corr, pbv, t & 1);
            // the tiles DMA'd above have landed in LDS before the barrier.  (All loads
            // are waited for, the scale loads issued after the DMAs too: the wait is
            // not exposed -- without it the kernel measures the same.)
            if constexpr (DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            return fn;
        };
        // Unmasked tiles two per trip: the P operands of consecutive tiles then
        // alternate between two register sets instead of being copied every tile.
        int t = t0;
        const int t_um = t1 < t_mask ? t1 : t_mask;     // unmasked steps: t + 1 < t_um
        for (; t + 2 < t_um; t += 2) {
            const Front g = step(t, f, std::false_type{});
            f = step(t + 1, g, std::false_type{});
        }
        for (; t + 1 < t_um; t++) f = step(t, f, std::false_type{});
        for (; t + 1 < t1; t++) f = step(t, f, std::true_type{});
        const float pbv = update(f);
        back(f.p_lo, f.p_hi, f.corr, pbv, t & 1);
    }
    if (nsplit == 1) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        float* orow = out + (size_t)qrow * HD + 4 * G;
#pragma unroll
        for (int dt = 0; dt < 16; dt++)
            *reinterpret_cast<float4*>(orow + 16 * dt) =
                make_float4(O[dt][0] * inv, O[dt][1] * inv, O[dt][2] * inv, O[dt][3] * inv);
    } else {
        // Split-KV: this split's partial state (unnormalised O, running max in log2
        // units, L) is written through to the device-coherent level (sc1 stores: the
        // workgroup that combines may run on another XCD), then counted in for this
        // (query block, head).  The workgroup that counts last combines every split
        // in split order -- M = max_s m_s, out = Σ_s O_s 2^(m_s - M) / Σ_s L_s 2^(m_s - M)
        // -- and re-arms the counter for the next call.  No workgroup waits for
        // another.
        constexpr int kSc1 = 16;    // cache policy: sc1
        constexpr int kFastSplits = 4;   // split counts combined with loads issued in bulk
        const int item = head * gridDim.x + blockIdx.x;
        // this query block's 64 rows of split s: O [64][HD] and (m, L) [64]
        auto o_rsrc = [&](int s) {
            return __builtin_amdgcn_make_buffer_rsrc(opart + (((size_t)s * gridDim.y + head) * n_q + q0) * HD, 0,
                                                     QROWS * HD * 4, kRsrcW3);
        };
        auto ml_rsrc = [&](int s) {
            return __builtin_amdgcn_make_buffer_rsrc(mlpart + ((size_t)s * gridDim.y + head) * n_q + q0, 0,
                                                     QROWS * 8, kRsrcW3);
        };
        const int ooff = ((16 * w + qi) * HD + 4 * G) * 4;   // this lane's first 16 bytes in a block
        const int moff = (16 * w + qi) * 8;
        {
            const __amdgpu_buffer_rsrc_t rs = o_rsrc(split);
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
                __builtin_amdgcn_raw_buffer_store_b128(
                    v4u{__float_as_uint(O[dt][0]), __float_as_uint(O[dt][1]), __float_as_uint(O[dt][2]),
                        __float_as_uint(O[dt][3])},
                    rs, ooff + dt * 64, 0, kSc1);
            if (G == 0)
                __builtin_amdgcn_raw_buffer_store_b64(v2u{__float_as_uint(rref), __float_as_uint(L)}, ml_rsrc(split),
                                                      moff, 0, kSc1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(cnt + item, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nsplit - 1;
        __syncthreads();
        if (s_last) {
            auto ml_of = [&](int s) -> float2 {
                const v2u v = __builtin_amdgcn_raw_buffer_load_b64(ml_rsrc(s), moff, 0, kSc1);
                return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
            };
            float o[16][4];
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++) o[dt][r] = 0.f;
            float l = 0.f;
            if (nsplit <= kFastSplits) {
                // All loads of a round are issued before any is used: every split's
                // (m, L) in one round, then the partial O in four rounds of 64 dims,
                // each holding that quarter of every split (5 memory round trips in
                // place of 2·nsplit + 1 dependent ones).  This workgroup's own split
                // is read back like the others (its stores completed at vmcnt(0)
                // above).  The sums run in split order, as in the general path.
                float2 ml[kFastSplits];
#pragma unroll
                for (int s = 0; s < kFastSplits; s++)
                    if (s < nsplit) ml[s] = ml_of(s);
                float Mx = -__builtin_inff();
#pragma unroll
                for (int s = 0; s < kFastSplits; s++)
                    if (s < nsplit) Mx = fmaxf(Mx, ml[s].x);
                float a[kFastSplits];
#pragma unroll
                for (int s = 0; s < kFastSplits; s++)
                    if (s < nsplit) {
                        a[s] = exp2f(ml[s].x - Mx);
                        l = fmaf(a[s], ml[s].y, l);
                    }
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    v4u b[kFastSplits][4];
#pragma unroll
                    for (int s = 0; s < kFastSplits; s++)
                        if (s < nsplit) {
                            const __amdgpu_buffer_rsrc_t rs = o_rsrc(s);
#pragma unroll
                            for (int d = 0; d < 4; d++)
                                b[s][d] = __builtin_amdgcn_raw_buffer_load_b128(rs, ooff + (4 * c + d) * 64, 0, kSc1);
                        }
#pragma unroll
                    for (int s = 0; s < kFastSplits; s++)
                        if (s < nsplit) {
#pragma unroll
                            for (int d = 0; d < 4; d++) {
                                const int dt = 4 * c + d;
                                o[dt][0] = fmaf(a[s], __uint_as_float(b[s][d].x), o[dt][0]);
                                o[dt][1] = fmaf(a[s], __uint_as_float(b[s][d].y), o[dt][1]);
                                o[dt][2] = fmaf(a[s], __uint_as_float(b[s][d].z), o[dt][2]);
                                o[dt][3] = fmaf(a[s], __uint_as_float(b[s][d].w), o[dt][3]);
                            }
                        }
                }
            } else {
                float Mx = -__builtin_inff();
                for (int s = 0; s < nsplit; s++) Mx = fmaxf(Mx, ml_of(s).x);
                for (int s = 0; s < nsplit; s++) {
                    const float2 ml = ml_of(s);
                    const float a = exp2f(ml.x - Mx);
                    const __amdgpu_buffer_rsrc_t rs = o_rsrc(s);
#pragma unroll
                    for (int dt = 0; dt < 16; dt++) {
                        const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rs, ooff + dt * 64, 0, kSc1);
                        o[dt][0] = fmaf(a, __uint_as_float(v.x), o[dt][0]);
                        o[dt][1] = fmaf(a, __uint_as_float(v.y), o[dt][1]);
                        o[dt][2] = fmaf(a, __uint_as_float(v.z), o[dt][2]);
                        o[dt][3] = fmaf(a, __uint_as_float(v.w), o[dt][3]);
                    }
                    l = fmaf(a, ml.y, l);
                }
            }
            float* orow = out + (size_t)qrow * HD + 4 * G;
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
                *reinterpret_cast<float4*>(orow + 16 * dt) =
                    make_float4(l > 0.f ? o[dt][0] / l : 0.f, l > 0.f ? o[dt][1] / l : 0.f,
                                l > 0.f ? o[dt][2] / l : 0.f, l > 0.f ? o[dt][3] / l : 0.f);
            if (tid == 0) __hip_atomic_store(cnt + item, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Staged K/V blocks of every tile of every KV head, for the DMA path: the kernel's
// own staging (same loads, range checks and byte layout), run once per call instead
// of once per query block and split.  Block (vh, t) of kx / vx holds the 16 KB that
// tile t's staging writes to LDS.
__global__ __launch_bounds__(256) void fa_expand_kv_k(const uint32_t* __restrict__ kc,
                                                      const uint32_t* __restrict__ vc,
                                                      unsigned char* __restrict__ kx,
                                                      unsigned char* __restrict__ vx, int n_kv, int n_tile,
                                                      int kv_cap) {
    const int t = blockIdx.x, vh = blockIdx.y, tid = threadIdx.x;
    const size_t blk = ((size_t)vh * n_tile + t) * KU_BYTES;
    if (blockIdx.z == 0) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(kc + (size_t)vh * kv_cap * KDW), 0, n_kv * KDW * 4, kRsrcW3);
        const int off = ((tid & 63) * KDW + 8 * (tid >> 6)) * 4;
        const int sk = (int)((uint32_t)t * (uint32_t)(BNK * KDW * 4));
        const v4u k0 = __builtin_amdgcn_raw_buffer_load_b128(rs, off, sk, 0);
        const v4u k1 = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16, sk, 0);
        put_k_slots(kx + blk, k0, k1, tid);
    } else {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(vc + (size_t)vh * (kv_cap / 8) * HD), 0, (n_kv / 8) * HD * 4, kRsrcW3);
        const int sv = (int)((uint32_t)t * (uint32_t)(BNK / 8 * HD * 4));
        uint32_t vw[8];
#pragma unroll
        for (int g = 0; g < 8; g++)
            vw[g] = __builtin_amdgcn_raw_buffer_load_b32(rs, tid * 4 + (g & 3) * HD * 4, sv + (g >> 2) * 4 * HD * 4, 0);
        put_v_slots(vx + blk, vw, tid);
    }
}

// -------------------------------------------------------------- launchers --

int fa_splits(int n_q, int n_heads, int n_tile, int cus) {
    // workgroups resident per CU: LDS (double-buffered operands) allows two
    const int slots = (cus > 0 ? cus : 256) * 2;
    const int items = (n_q / QROWS) * n_heads;
    int best = 1;
    double best_eff = 0.0;
    for (int s = 1; s <= 8; s++) {
        if (s > 1 && n_tile / s < 8) break;          // keep at least 8 tiles per split
        const long long blocks = (long long)items * s;
        const double eff = (double)blocks / ((double)slots * (double)((blocks + slots - 1) / slots));
        if (eff > best_eff + 0.02) {
            best_eff = eff;
            best = s;
        }
    }
    return best;
}

size_t fa_part_bytes(int n_q, int n_heads, int nsplit) {
    return nsplit > 1 ? (size_t)nsplit * n_heads * n_q * (HD + 2) * sizeof(float) : 0;
}

size_t fa_cnt_bytes(int n_q, int n_heads, int nsplit) {
    return nsplit > 1 ? (size_t)(n_q / QROWS) * n_heads * sizeof(int) : 0;
}

size_t fa_kvx_bytes(int n_heads, int ratio, int n_tile) {
    return (size_t)2 * (size_t)(n_heads / ratio) * (size_t)n_tile * KU_BYTES;
}

hipError_t launch_fa_int4(float* out, const uint32_t* qq, const float* qsc, const uint32_t* kc, const float* ksc,
                          const uint32_t* vc, const float* vsc, int n_q, int n_kv, int off, int n_tile,
                          int n_heads, int ratio, int kv_cap, int nsplit, float* part, int* cnt, void* kvx,
                          hipStream_t st) {
    float* opart = part;
    float2* mlpart = part ? reinterpret_cast<float2*>(part + (size_t)nsplit * n_heads * n_q * HD) : nullptr;
    const dim3 grid(n_q / QROWS, n_heads, nsplit);
    if (!kvx) {
        hipLaunchKernelGGL(fa_int4_k<false>, grid, dim3(NTA), 0, st, qq, qsc, kc, ksc, vc, vsc, out, n_q, n_kv, off,
                           n_tile, ratio, kv_cap, nsplit, opart, mlpart, cnt, nullptr, nullptr);
        return hipGetLastError();
    }
    const int kvh = n_heads / ratio;
    unsigned char* kx = static_cast<unsigned char*>(kvx);
    unsigned char* vx = kx + (size_t)kvh * n_tile * KU_BYTES;
    hipLaunchKernelGGL(fa_expand_kv_k, dim3(n_tile, kvh, 2), dim3(256), 0, st, kc, vc, kx, vx, n_kv, n_tile, kv_cap);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(fa_int4_k<true>, grid, dim3(NTA), 0, st, qq, qsc, kc, ksc, vc, vsc, out, n_q, n_kv, off,
                       n_tile, ratio, kv_cap, nsplit, opart, mlpart, cnt, kx, vx);
    return hipGetLastError();
}

}  // namespace rt4
