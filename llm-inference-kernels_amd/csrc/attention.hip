// Split-K ("FlashDecoding") GQA decode attention over an fp16, INT8
// per-token or INT4 KIVI KV cache, for gfx950.
//
// Math (reference/attention_ref.py:43-80, bindings/extension.cpp:26-83):
//   out[b,h,:] = softmax(scale * q[b,h] . K[b,h/G,0:S]^T) @ V[b,h/G,0:S]
// with the cache addressed at stride kv_buf_len and read over [0, seqlen).
//
// Work decomposition (both kernels below)
//   * One workgroup owns one (batch, kv_head, head_chunk, split): the
//     HPW <= 4 query heads that share a kv head are processed together, so
//     every K/V byte of the split is read from HBM exactly once (the
//     reference re-reads each kv head once per query head,
//     kernels/attention/fused_attention_splitk.cu:84-90).
//   * Each workgroup keeps several online-softmax states (m, l, o) in the
//     log2 domain, merges them through LDS, and writes the split's
//     un-normalised (o, m, l) to the workspace. The last workgroup to finish
//     a (batch, kv_head, head_chunk) merges all splits in split order and
//     writes fp16 out, so a call is one launch and results are deterministic.
//
// Main kernel (decode_attention_mfma_kernel): each wave walks its tiles of
// 32 tokens on v_mfma_f32_16x16x32_f16:
//   QK : A = q (16 rows, row m holds head (m / 4) % HPW), B = 16 tokens'
//        keys (lane = token, 8 consecutive channels per lane group) -> lane
//        group g gets head g % HPW's score of its token and runs that head's
//        online softmax; no cross-group reductions.
//   PV : A = p as an fp16 hi + lo pair (two MFMAs per B operand, through a
//        512-byte per-wave LDS slot; fp16 p alone would cost ~2^-12 |v| of
//        accuracy under a peaked softmax), B = values:
//        lane (g, c) loads the channels 8c..8c+7 of the tokens in k-slots
//        8g..8g+7 (tokens 8g + e; INT4, whose rows are 64 bytes: tokens
//        4e + g, so that each load instruction reads whole lines) and one
//        v_perm_b32 per dword turns them into the B operand of MFMA j, which
//        owns channels 8c + j.
//   INT8/INT4 codes are converted to fp16 exactly in registers; the INT8
//   per-token K scale multiplies the score, the per-token V scale folds into
//   p, the INT4 per-channel K scale folds into q per group (q*s split into an
//   fp16 hi + lo pair in alternate rows of QK's A operand, so the product
//   keeps fp32 precision at one MFMA per k-step; INT4's PV likewise carries
//   both P planes in one MFMA, in alternate lane groups' rows).
// fp16 16-token form (decode_attention_f16h_kernel): the same products over
// 16-token tiles with the next tile's loads in flight (PV on
// v_mfma_f32_16x16x16_f16), for the plans where it measured faster.
// Fallback kernel (decode_attention_valu_kernel): fp32 VALU with 16-lane
// DPP reductions; used for INT4 group sizes that are not multiples of 32.
//
// KV formats (packing is kernels/kv_cache/kv_compress.cuh:25-28 and
// kernels/common/cuda_utils.cuh:85-119 of the reference):
//   F16: k,v [B,Hkv,L,128] fp16
//   I8 : k,v [B,Hkv,L,128] int8, k_scale,v_scale [B,Hkv,L] fp16 (per token)
//   I4 : k,v [B,Hkv,L,64] packed int4 (even channel in the low nibble),
//        k_scale [B,Hkv,n_groups,128] fp16 (per channel, per group of
//        group_size tokens), v_scale [B,Hkv,L] fp16 (per token)
#include <atomic>

#include "device_common.hpp"
#include "llmik_internal.hpp"

namespace llmik {

enum class KvFormat { F16, I8, I4 };

constexpr int kAttnThreads = 256;   // VALU kernel
constexpr int kHeadDim = 128;
constexpr int kTile = 32;   // tokens per wave step of the MFMA kernel
#ifndef LLMIK_ATTN_WGS_PER_CU
#define LLMIK_ATTN_WGS_PER_CU 1
#endif
constexpr int kAttnWgsPerCu = LLMIK_ATTN_WGS_PER_CU;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const uint16_t* q;
    const void* k;
    const void* v;
    const uint16_t* k_scale;
    const uint16_t* v_scale;
    uint16_t* out;
    float* part_o;        // [slots, HPW, 128]
    float* part_ml;       // [slots, HPW, 2]
    uint32_t* counters;   // [B * Hkv * n_hchunks], zero between calls
    int n_heads, n_kv_heads, seqlen, kv_buf_len;
    int group_size, n_groups;
    int n_splits, chunk, n_hchunks, gqa;
    float scale_log2;
};

// Split hand-off. Thread t < HPW * 32 of the workgroup owns head t / 32,
// channels 4 (t % 32) .. + 3 of the workgroup's outputs; the partials and
// the combine move those four values as one 16-byte access (sc1, like the
// 4-byte forms above), and the output as one 8-byte store.
template <int HPW>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_o_rsrc(const AttnParams& p, long slot) {
    return make_buffer_rsrc(p.part_o + slot * HPW * kHeadDim, (uint32_t)(HPW * kHeadDim * sizeof(float)));
}

__device__ __forceinline__ void store_out4_f16(const AttnParams& p, long o, const float v[4], float inv) {
    const uint32_t lo = (uint32_t)f2h_bits(v[0] * inv) | ((uint32_t)f2h_bits(v[1] * inv) << 16);
    const uint32_t hi = (uint32_t)f2h_bits(v[2] * inv) | ((uint32_t)f2h_bits(v[3] * inv) << 16);
    *reinterpret_cast<u32x2*>(p.out + o) = u32x2{lo, hi};
}

// The last split's combine of a (batch, kv head, head chunk) slot group: each
// thread issues the (m, l) and partial-output loads of a batch of KB splits
// together, so a combine of up to KB splits costs one memory round trip;
// rescaling to a common maximum is done in registers. Batch entries past the
// split count re-read the last split and add zero.
template <int KB, int HPW>
__device__ __forceinline__ void combine_splits(const AttnParams& p, int b, int slot_group, int head0, int h,
                                               int d) {
    const long base = (long)slot_group * p.n_splits;
    float gm = -INFINITY, sl = 0.0f;
    float so[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp0 = 0; sp0 < p.n_splits; sp0 += KB) {
        float mv[KB], lv[KB];
        u32x4 ov[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const long slot = base + min(sp0 + u, p.n_splits - 1);
            mv[u] = publish_load(&p.part_ml[(slot * HPW + h) * 2]);
            lv[u] = publish_load(&p.part_ml[(slot * HPW + h) * 2 + 1]);
            ov[u] = publish_load16(part_o_rsrc<HPW>(p, slot), (uint32_t)((h * kHeadDim + d) * sizeof(float)));
        }
        float bm = gm;
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (sp0 + u < p.n_splits) bm = fmaxf(bm, mv[u]);
        if (bm == -INFINITY) continue;
        const float r = (gm == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(gm - bm);
#pragma unroll
        for (int e = 0; e < 4; ++e) so[e] *= r;
        sl *= r;
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const float w = (sp0 + u < p.n_splits && mv[u] != -INFINITY) ? __builtin_amdgcn_exp2f(mv[u] - bm)
                                                                         : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t ob = ov[u][e];
                so[e] = fmaf(__uint_as_float(ob), w, so[e]);
            }
            sl = fmaf(lv[u], w, sl);
        }
        gm = bm;
    }
    const float inv = (sl > 0.0f) ? 1.0f / sl : 0.0f;
    store_out4_f16(p, ((long)b * p.n_heads + head0 + h) * kHeadDim + d, so, inv);
}

// ---------------------------------------------------------------------------
// Shared tail: merge NR partial states held in LDS, then either write the
// output (single split) or publish the split and let the last one combine.
// ---------------------------------------------------------------------------
template <int NR, int HPW, int NT>
__device__ __forceinline__ void finish_split(const AttnParams& p, const float (*s_o)[HPW][kHeadDim],
                                             const float (*s_m)[HPW], const float (*s_l)[HPW],
                                             uint32_t* s_last, int b, int kvh, int hchunk,
                                             int split, int head0) {
    constexpr int kThr = HPW * (kHeadDim / 4);   // threads owning four outputs
    static_assert(NT >= kThr, "the workgroup must cover every output");
    const int tid = threadIdx.x;
    const bool owner = tid < kThr;
    const int h = owner ? tid / (kHeadDim / 4) : 0;
    const int d = owner ? 4 * (tid % (kHeadDim / 4)) : 0;
    const int slot_group = (b * p.n_kv_heads + kvh) * p.n_hchunks + hchunk;
    const long slot = (long)slot_group * p.n_splits + split;
    float wo[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float wm = -INFINITY, wl = 0.0f;
    if (owner) {
        float gm = -INFINITY;
#pragma unroll
        for (int r = 0; r < NR; ++r) gm = fmaxf(gm, s_m[r][h]);
        if (gm != -INFINITY) {
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float w = (s_m[r][h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(s_m[r][h] - gm);
                const f32x4 o4 = *reinterpret_cast<const f32x4*>(&s_o[r][h][d]);
#pragma unroll
                for (int e = 0; e < 4; ++e) wo[e] = fmaf(o4[e], w, wo[e]);
                wl = fmaf(s_l[r][h], w, wl);
            }
        }
        wm = gm;
    }

    if (p.n_splits == 1) {
        if (owner) {
            const float inv = (wl > 0.0f) ? 1.0f / wl : 0.0f;
            store_out4_f16(p, ((long)b * p.n_heads + head0 + h) * kHeadDim + d, wo, inv);
        }
        return;
    }

    if (owner) {
        publish_store16(part_o_rsrc<HPW>(p, slot), (uint32_t)((h * kHeadDim + d) * sizeof(float)),
                        make_u32x4(__float_as_uint(wo[0]), __float_as_uint(wo[1]), __float_as_uint(wo[2]),
                                   __float_as_uint(wo[3])));
        if (d == 0) {
            publish_store(&p.part_ml[(slot * HPW + h) * 2 + 0], wm);
            publish_store(&p.part_ml[(slot * HPW + h) * 2 + 1], wl);
        }
    }
    publish_wait();
    __syncthreads();
    if (tid == 0) *s_last = arrive_last(&p.counters[slot_group], (uint32_t)p.n_splits) ? 1u : 0u;
    __syncthreads();
    if (*s_last == 0u) return;

    // Last split of this slot group: combine all splits, in batches of the
    // split count rounded up to 4, 8 or 16, so that a combine of 4 splits
    // issues 4 loads per value and not 16. The batches run in split order,
    // so the sum is the same bits for every batch size.
    if (owner) {
        if (p.n_splits <= 4) combine_splits<4, HPW>(p, b, slot_group, head0, h, d);
        else if (p.n_splits <= 8) combine_splits<8, HPW>(p, b, slot_group, head0, h, d);
        else combine_splits<16, HPW>(p, b, slot_group, head0, h, d);
    }
    if (tid == 0) p.counters[slot_group] = 0u;   // leave the counter zeroed for the next call
}

// ===========================================================================
// MFMA kernel
// ===========================================================================


__device__ __forceinline__ f32x4 mfma16x16x32(const f16x8 a, const f16x8 b, const f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x8 as_f16x8(const u32x4 v) { return __builtin_bit_cast(f16x8, v); }


// Two biased int8 bytes (value + 128, in bytes 0 and 2 of x, bytes 1 and 3
// zero) -> two exact fp16 values: 0x6400 | u is 1024 + u.
__device__ __forceinline__ uint32_t u8pair_to_f16x2(uint32_t x) {
    const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
    const f16x2 h = as_f16x2(x | 0x64006400u) - bias;
    return __builtin_bit_cast(uint32_t, h);
}

// Four int8 codes of one dword -> fp16 pairs (b0,b1), (b2,b3), exact.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    w ^= 0x80808080u;
    lo = u8pair_to_f16x2(perm_b32(0u, w, 0x0C010C00u));
    hi = u8pair_to_f16x2(perm_b32(0u, w, 0x0C030C02u));
}

// Eight int4 codes of one dword (already xor-biased by 8 per nibble) ->
// fp16 pairs (n0,n4), (n1,n5), (n2,n6), (n3,n7), exact.
__device__ __forceinline__ u32x4 i4x8b_to_f16(uint32_t w) {
    const uint32_t w8 = w >> 8;
    const f16x2 bias = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 bias16 = {(f16)72.0f, (f16)72.0f};
    const f16x2 a = as_f16x2((w & 0x000F000Fu) | 0x64006400u) - bias;
    const f16x2 b = as_f16x2((w & 0x00F000F0u) | 0x64006400u) * sixteenth - bias16;
    const f16x2 c = as_f16x2((w8 & 0x000F000Fu) | 0x64006400u) - bias;
    const f16x2 d = as_f16x2((w8 & 0x00F000F0u) | 0x64006400u) * sixteenth - bias16;
    return make_u32x4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                      __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d));
}

// Order of the channels inside an INT4 K operand: half e of the fp16 octet
// made from one dword holds nibble i4_perm(e) (pairs (0,4), (1,5), (2,6), (3,7)).
__host__ __device__ constexpr int i4_perm(int e) { return (e & 1) ? (e >> 1) + 4 : (e >> 1); }

// Eight fp16 in channel order 0..7 -> the order i4_perm (0, 4, 1, 5, 2, 6, 3, 7).
__device__ __forceinline__ u32x4 i4_pair_order(const u32x4 a) {
    return make_u32x4(perm_b32(a[2], a[0], 0x05040100u), perm_b32(a[2], a[0], 0x07060302u),
                      perm_b32(a[3], a[1], 0x05040100u), perm_b32(a[3], a[1], 0x07060302u));
}

// Per-wave load context of the MFMA kernel: buffer views of one (batch, kv
// head) slab of the cache that end at the wave's last token w1, so a tile
// load past the range returns zeros (those tokens are masked to -inf
// anyway) and needs no clamping; every load is a lane-constant voffset plus
// a uniform soffset (t0 * row bytes), so a tile costs no VALU address work.
// The masks of the code conversions live in VGPRs so that each
// (word & mask) | bias is one three-operand bit op.
struct TileCtx {
    __amdgpu_buffer_rsrc_t rk, rv, rks, rvs, rkg;
    uint32_t koff, voff, soff, kgoff;
    uint32_t m_lo, m_hi, e16, e8;
    uint32_t x_lo, x_hi;   // INT4: exponent bits of 0x6400 pairs xor the nibble sign bits
};

template <KvFormat F>
struct MfmaTile;

// ---- fp16 ------------------------------------------------------------------
// QK operand of k-step ks for lane group g: channels 32*ks + 8*g + (0..7).
template <>
struct MfmaTile<KvFormat::F16> {
    static constexpr float kPScale = 256.0f;   // p <= 1 -> fp16 p*256 has no subnormals above 2^-32
    static constexpr uint32_t kRow = kHeadDim * 2;
    u32x4 k[2][4];
    u32x4 v[8];
    // K: lane (g, c) reads row 16 blk + c, channels 32 ks + 8g; V: rows
    // 8g + e, channels 8c.
    __device__ __forceinline__ void load(const TileCtx& x, int t0) {
        const uint32_t so = (uint32_t)t0 * kRow;
        // Each K instruction reads 64 bytes of every row (half a 128-byte
        // line; the next k-step's instruction reads the rest), so K is loaded
        // without the non-temporal hint and the line waits in L2 for its
        // second half. V instructions read whole rows and keep the hint.
#pragma unroll
        for (int blk = 0; blk < 2; ++blk)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                k[blk][ks] = __builtin_amdgcn_raw_buffer_load_b128(
                    x.rk, (int)x.koff, (int)(so + 16 * kRow * blk + 64 * ks), 0);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = __builtin_amdgcn_raw_buffer_load_b128(x.rv, (int)x.voff, (int)(so + kRow * e), 2);
    }
    __device__ __forceinline__ f16x8 kop(const TileCtx&, int blk, int ks) const { return as_f16x8(k[blk][ks]); }
    // B operand of PV MFMA j: (V[token 8g+2i][8c+j], V[token 8g+2i+1][8c+j]) per dword i.
    __device__ __forceinline__ f16x8 vop(const TileCtx&, int j) const {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        uint32_t d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = v[2 * i][j >> 1];
            const uint32_t hi = v[2 * i + 1][j >> 1];
            d[i] = perm_b32(hi, lo, sel);
        }
        return as_f16x8(make_u32x4(d[0], d[1], d[2], d[3]));
    }
};

// ---- int8 ------------------------------------------------------------------
// QK operand of k-step ks = 2u + h for lane group g: channels 64u + 16g + 8h + (0..7).
template <>
struct MfmaTile<KvFormat::I8> {
    static constexpr float kPScale = 64.0f;    // p * v_scale * 64 <= 516 * 64 < 65504
    static constexpr uint32_t kRow = kHeadDim;
    u32x4 k[2][2];
    u32x2 v[8];
    uint16_t ks[2], vs[2];
    __device__ __forceinline__ void load(const TileCtx& x, int t0) {
        const uint32_t so = (uint32_t)t0 * kRow;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int u = 0; u < 2; ++u)   // half rows: no non-temporal hint (see the fp16 tile)
                k[blk][u] = __builtin_amdgcn_raw_buffer_load_b128(
                    x.rk, (int)x.koff, (int)(so + 16 * kRow * blk + 64 * u), 0);
            ks[blk] = __builtin_amdgcn_raw_buffer_load_b16(x.rks, (int)x.soff, (int)(2 * t0 + 32 * blk), 0);
            vs[blk] = __builtin_amdgcn_raw_buffer_load_b16(x.rvs, (int)x.soff, (int)(2 * t0 + 32 * blk), 0);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                x.rv, (int)x.voff, (int)(so + kRow * e), 2));
    }
    // Four codes of a dword -> exact fp16 pairs: one v_perm_b32 places bytes
    // (b0, b1) (or (b2, b3)) under the 0x64 exponent bytes of x.e8, giving
    // 1024 + u; the bias 1152 = 1024 + 128 is then subtracted.
    __device__ __forceinline__ f16x8 kop(const TileCtx& x, int blk, int ks_) const {
        const u32x4 w = k[blk][ks_ >> 1];
        const f16x2 bias = {(f16)1152.0f, (f16)1152.0f};
        uint32_t d[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t wi = w[(ks_ & 1) * 2 + i] ^ 0x80808080u;
            d[2 * i] = __builtin_bit_cast(uint32_t, as_f16x2(perm_b32(x.e8, wi, 0x07010600u)) - bias);
            d[2 * i + 1] = __builtin_bit_cast(uint32_t, as_f16x2(perm_b32(x.e8, wi, 0x07030602u)) - bias);
        }
        return as_f16x8(make_u32x4(d[0], d[1], d[2], d[3]));
    }
    // B operand of PV MFMA j, biased: (V[8g+2i][8c+j], V[8g+2i+1][8c+j]) as
    // 1152 + code. One permute places the two code bytes under zero bytes;
    // xor 0x6480 6480 sets the 0x64 exponents and flips the code's sign bit
    // (1024 + (code + 128)). The bias is taken out once, at the end, from
    // the sum of P (kVBias).
    static constexpr float kVBias[2] = {1152.0f, 1152.0f};
    static constexpr float kVUnscale[2] = {1.0f, 1.0f};
    __device__ __forceinline__ f16x8 vop(const TileCtx& x, int j) const {
        const int byte = j & 3;
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + byte) << 16) | (uint32_t)byte;
        uint32_t d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = perm_b32(v[2 * i + 1][j >> 2], v[2 * i][j >> 2], sel) ^ 0x64806480u;
        return as_f16x8(make_u32x4(d[0], d[1], d[2], d[3]));
    }
};

// ---- int4 ------------------------------------------------------------------
// QK operand of k-step ks for lane group g: channels 32g + 8ks + i4_perm(e).
template <>
struct MfmaTile<KvFormat::I4> {
    static constexpr float kPScale = 4.0f;     // p * v_scale * 4 <= 9358 * 4 < 65504
    static constexpr uint32_t kRow = kHeadDim / 2;
    u32x4 k[2];
    uint32_t v[8];
    uint16_t vs[2];
    u32x4 ksc[4];   // K scales of the tile's group, channels 32g..32g+31 (L2-resident)
    int grp;        // the tile's scale group (a 32-token tile lies in one group)
    __device__ __forceinline__ void load(const TileCtx& x, int t0, int group_size, int t_last) {
        const uint32_t so = (uint32_t)t0 * kRow;
        grp = min(t0, t_last) / group_size;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ksc[i] = __builtin_amdgcn_raw_buffer_load_b128(x.rkg, (int)x.kgoff,
                                                           (int)((uint32_t)grp * kHeadDim * 2 + 16 * i), 0);
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            k[blk] = __builtin_amdgcn_raw_buffer_load_b128(x.rk, (int)x.koff, (int)(so + 16 * kRow * blk), 2);
            vs[blk] = __builtin_amdgcn_raw_buffer_load_b16(x.rvs, (int)x.soff, (int)(2 * t0 + 32 * blk), 0);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            v[e] = __builtin_amdgcn_raw_buffer_load_b32(x.rv, (int)x.voff, (int)(so + 4 * kRow * e), 2);
    }
    // Eight codes of a dword -> fp16 pairs (n0,n4), (n1,n5), (n2,n6), (n3,n7), exact.
    // (w ^ 0x88888888) & m | 0x6400 6400 == (w & m) ^ x.x_lo / x.x_hi: the
    // masked nibbles, the sign bits flipped and the exponents never overlap.
    __device__ __forceinline__ f16x8 kop(const TileCtx& x, int blk, int ks_) const {
        const uint32_t w = k[blk][ks_];
        const uint32_t w8 = w >> 8;
        const f16x2 bias = {(f16)1032.0f, (f16)1032.0f};
        const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
        const f16x2 bias16 = {(f16)72.0f, (f16)72.0f};
        const f16x2 a = as_f16x2((w & x.m_lo) ^ x.x_lo) - bias;
        const f16x2 b = as_f16x2((w & x.m_hi) ^ x.x_hi) * sixteenth - bias16;
        const f16x2 c = as_f16x2((w8 & x.m_lo) ^ x.x_lo) - bias;
        const f16x2 d = as_f16x2((w8 & x.m_hi) ^ x.x_hi) * sixteenth - bias16;
        return as_f16x8(make_u32x4(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                   __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)));
    }
    // B operand of PV MFMA j, biased: every code enters as the exact fp16
    // 1024 + 16 (code + 8) = 16 code + 1152, its nibble in mantissa bits 4-7.
    // Odd j (channel 8c + j odd) takes the high nibbles in place; even j the
    // low nibbles of the words shifted left by 4 (vop_lo). The bias and the
    // factor 16 are taken out once, at the end, from the sum of P (kVBias,
    // kVUnscale). A low nibble in bits 0-3 (1024 + code + 8) would put ~130x
    // the signal into the fp32 accumulator as bias, against ~9x here.
    static constexpr float kVBias[2] = {1152.0f, 1152.0f};
    static constexpr float kVUnscale[2] = {0.0625f, 0.0625f};
    __device__ __forceinline__ f16x8 vop(const TileCtx& x, int j) const {
        const int byte = j >> 1;
        const uint32_t sel = 0x0C000C00u | ((uint32_t)(4 + byte) << 16) | (uint32_t)byte;
        uint32_t d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = (j & 1) ? v[2 * i] : (v[2 * i] << 4);
            const uint32_t hi = (j & 1) ? v[2 * i + 1] : (v[2 * i + 1] << 4);
            d[i] = (perm_b32(hi, lo, sel) & x.m_hi) ^ x.x_hi;
        }
        return as_f16x8(make_u32x4(d[0], d[1], d[2], d[3]));
    }
};

// NW waves per workgroup. fp16 / INT8: split s takes the sequence's 32-token
// tiles s, s + n_splits, ... and its waves take those round robin, so a
// workgroup's waves finish within a tile of each other. INT4: each wave takes
// a contiguous quarter / eighth of the split, so its K-scale group changes
// only every group_size tokens.
template <KvFormat F, int HPW, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
void decode_attention_mfma_kernel(AttnParams p) {
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / p.n_hchunks;
    const int hchunk = blockIdx.y % p.n_hchunks;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int c = lane & 15;

    const int head0 = kvh * p.gqa + hchunk * HPW;
    // QK's A operand row m holds head (m / 4) % HPW: the four outputs of lane
    // group g (rows 4g..4g+3) are all head g % HPW's scores, so each lane
    // group runs the online softmax of one head (PV keeps row m = head m % HPW).
    const uint16_t* qrow = p.q + ((long)b * p.n_heads + head0 + ((c >> 2) % HPW)) * kHeadDim;

    // Q as the A operand (4 k-steps). INT4: q * k_scale as an fp16 hi + lo
    // pair, hi in the even and lo in the odd rows of each lane group's four,
    // so that one MFMA per k-step yields both (score = row 4g + row 4g + 1).
    f16x8 qa[4];
    f16x8 qp[4];    // INT4 only: q of channels 32g + 8ks + i4_perm(e), the K operand's order
    if constexpr (F == KvFormat::F16) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qa[ks] = as_f16x8(load16(qrow + 32 * ks + 8 * g));
    } else if constexpr (F == KvFormat::I8) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            qa[ks] = as_f16x8(load16(qrow + 64 * (ks >> 1) + 16 * g + 8 * (ks & 1)));
    } else {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qp[ks] = as_f16x8(i4_pair_order(load16(qrow + 32 * g + 8 * ks)));
    }

    f32x4 o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // INT8 / INT4: V enters the PV products biased (MfmaTile::vop); sum_p
    // accumulates the row sums of the same fp16 P operand (one more MFMA
    // against ones, rescaled with o) so that the bias is removed exactly
    // once at the end: o_j = (o_j - kVBias * sum_p) * kVUnscale.
    f32x4 sum_p = {0.0f, 0.0f, 0.0f, 0.0f};
    const f16x8 ones = {(f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f, (f16)1.0f};
    // Online-softmax state of this lane group's head (the same in its 16 lanes).
    float m_run = -INFINITY, l_run = 0.0f;

    // P as an fp16 hi + lo pair (plane 0: fp16(x), plane 1: fp16(x - hi)),
    // so that the PV products carry p to ~2^-22 instead of fp16's 2^-12.
    // fp16 / INT8: two MFMAs per B operand, one per plane. INT4 (kPlaneRows):
    // PV's A row m holds plane (m / 4) & 1 of head m % HPW, so lane groups 0
    // and 2 accumulate the hi products and 1 and 3 the lo products in one
    // MFMA, and the two halves are added once at the end (measured: faster
    // for INT4, whose QK already carries a hi/lo pair; not for fp16 / INT8).
    constexpr bool kPlaneRows = (F == KvFormat::I4);
    __shared__ __attribute__((aligned(16))) uint16_t s_p[NW][2][4][kTile];
    // Each head's rescale factor of the tile, for the PV accumulators, which
    // hold all heads in every lane.
    __shared__ __attribute__((aligned(16))) float s_alpha[NW][4];

    const int t_begin = split * p.chunk;
    const int t_end = min(t_begin + p.chunk, p.seqlen);
    constexpr bool kInterleave = (F != KvFormat::I4);
    constexpr int kWaveStride = kTile;   // INT4: the wave walks its range tile by tile
    // fp16 / INT8: split s takes tiles s, s + n_splits, s + 2 n_splits, ...
    // of the whole sequence and its waves every NW-th of those, so each
    // workgroup's reads spread over its KV head's whole K and V instead of
    // one contiguous quarter (fp16, against contiguous ranges: A16 and B=1
    // 1-3 % faster, S=16384 and B=64 about 1 % slower; INT8 neutral).
    constexpr bool kSplitTiles = kInterleave;
    int w0, w1;
    if constexpr (kSplitTiles) {
        w0 = (split + p.n_splits * wave) * kTile;
        w1 = p.seqlen;
    } else {
        const int per_wave = p.chunk / NW;   // multiple of kTile
        w0 = min(t_begin + wave * per_wave, t_end);
        w1 = min(w0 + per_wave, t_end);
    }
    // Load context of this wave (buffer views end at its last token w1).
    TileCtx x;
    {
        const long slab = (long)(b * p.n_kv_heads + kvh);
        constexpr uint32_t kRow = MfmaTile<F>::kRow;
        const long kv_base = slab * p.kv_buf_len * (long)kRow;
        const uint32_t range = (uint32_t)max(w1, 0) * kRow;
        x.rk = make_buffer_rsrc(static_cast<const char*>(p.k) + kv_base, range);
        x.rv = make_buffer_rsrc(static_cast<const char*>(p.v) + kv_base, range);
        if constexpr (F != KvFormat::F16) {
            x.rvs = make_buffer_rsrc(p.v_scale + slab * p.kv_buf_len, (uint32_t)max(w1, 0) * 2u);
            x.rks = make_buffer_rsrc(F == KvFormat::I8 ? p.k_scale + slab * p.kv_buf_len : p.v_scale,
                                     (uint32_t)max(w1, 0) * 2u);
        } else {
            x.rvs = x.rv;
            x.rks = x.rk;
        }
        x.rkg = (F == KvFormat::I4)
            ? make_buffer_rsrc(p.k_scale + slab * p.n_groups * kHeadDim, (uint32_t)p.n_groups * kHeadDim * 2u)
            : x.rk;
        if constexpr (F == KvFormat::F16) {
            x.koff = (uint32_t)c * kRow + 16u * g;
            x.voff = 8u * g * kRow + 16u * c;
        } else if constexpr (F == KvFormat::I8) {
            x.koff = (uint32_t)c * kRow + 16u * g;
            x.voff = 8u * g * kRow + 8u * c;
        } else {
            x.koff = (uint32_t)c * kRow + 16u * g;
            x.voff = (uint32_t)g * kRow + 4u * c;   // token 4e + g in instruction e
        }
        x.soff = 2u * c;
        x.kgoff = 64u * g;
        x.m_lo = vgpr_const(0x000F000Fu);
        x.m_hi = vgpr_const(0x00F000F0u);
        x.e16 = vgpr_const(0x64006400u);
        x.e8 = vgpr_const(0x64646464u);
        x.x_lo = vgpr_const(0x64086408u);
        x.x_hi = vgpr_const(0x64806480u);
    }
    int cur_group = -1;

    auto step = [&](const MfmaTile<F>& tile, const int t0) {

        // ---- scores for the tile's two 16-token blocks ----
        float s[2];
        if constexpr (F == KvFormat::I4) {
            if (tile.grp != cur_group) {   // wave-uniform; the scales came with the tile
                cur_group = tile.grp;
                // q * s as an fp16 hi + lo pair: an fp16 multiply rounds the
                // exact product once (hi), and an fp16 fma rounds the exact
                // q * s - hi once (lo) -- two packed ops per channel pair.
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const f16x8 sc = as_f16x8(i4_pair_order(tile.ksc[ks]));
                    const f16x8 hi = qp[ks] * sc;
                    const f16x8 lo = __builtin_elementwise_fma(qp[ks], sc, -hi);
                    qa[ks] = (c & 1) ? lo : hi;
                }
            }
        }
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const f16x8 kb = tile.kop(x, blk, ks);
                acc = mfma16x16x32(qa[ks], kb, acc);
            }
            const bool valid = (t0 + 16 * blk + c) < w1;
            float sc = p.scale_log2;
            if constexpr (F == KvFormat::I8) sc *= h2f(tile.ks[blk]);
            const float dot = (F == KvFormat::I4) ? acc[0] + acc[1] : acc[0];
            s[blk] = valid ? dot * sc : -INFINITY;
        }

        // ---- online softmax of lane group g's head over the 32 tokens ----
        const float tmax = row16_max(fmaxf(s[0], s[1]));
        const float mn = fmaxf(m_run, tmax);
        const float msafe = (mn == -INFINITY) ? 0.0f : mn;
        const float alpha = __builtin_amdgcn_exp2f(m_run - msafe);
        const bool rescale = __builtin_amdgcn_ballot_w64(mn != m_run) != 0;   // wave-uniform
        m_run = mn;
        const float pr0 = __builtin_amdgcn_exp2f(s[0] - msafe);
        const float pr1 = __builtin_amdgcn_exp2f(s[1] - msafe);
        l_run = fmaf(l_run, alpha, pr0 + pr1);

        // ---- p and alpha -> LDS (lane group g writes head g) -> A operand ----
        if (g < HPW) {
            float f0 = MfmaTile<F>::kPScale, f1 = MfmaTile<F>::kPScale;
            if constexpr (F != KvFormat::F16) {
                f0 *= h2f(tile.vs[0]);
                f1 *= h2f(tile.vs[1]);
            }
            // x - fp16(x) is exact in fp32; rounding it to fp16 leaves a
            // relative error of 2^-11 of a term that is itself <= 2^-11 x.
            const float x0 = pr0 * f0, x1 = pr1 * f1;
            const uint16_t h0 = f2h_bits(x0), h1 = f2h_bits(x1);
            // INT4: PV's k-slot 8 kq + e holds token 4 e + kq (each V load
            // instruction then reads four adjacent 64-byte rows, whole lines).
            const int sl0 = (F == KvFormat::I4) ? 8 * (c & 3) + (c >> 2) : c;
            const int sl1 = (F == KvFormat::I4) ? sl0 + 4 : 16 + c;
            s_p[wave][0][g][sl0] = h0;
            s_p[wave][0][g][sl1] = h1;
            s_p[wave][1][g][sl0] = f2h_bits(x0 - h2f(h0));
            s_p[wave][1][g][sl1] = f2h_bits(x1 - h2f(h1));
            if (c == 0) s_alpha[wave][g] = alpha;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const f16x8 pa = as_f16x8(load16(&s_p[wave][kPlaneRows ? (c >> 2) & 1 : 0][c % HPW][8 * g]));
        const f16x8 pl = kPlaneRows ? pa : as_f16x8(load16(&s_p[wave][1][c % HPW][8 * g]));
        if (rescale) {
            // PV row 4g + i is head i % HPW (PV's A row m = head m % HPW).
            const f32x4 al = *reinterpret_cast<const f32x4*>(&s_alpha[wave][0]);
            float a4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a4[i] = al[i % HPW];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[j][i] *= a4[i];
            if constexpr (F != KvFormat::F16) {
#pragma unroll
                for (int i = 0; i < 4; ++i) sum_p[i] *= a4[i];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();

        // ---- O += P V (hi and lo parts of P against the same B operand) ----
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const f16x8 vb = tile.vop(x, j);
            o[j] = mfma16x16x32(pa, vb, o[j]);
            if constexpr (!kPlaneRows) o[j] = mfma16x16x32(pl, vb, o[j]);
        }
        if constexpr (F != KvFormat::F16) {
            sum_p = mfma16x16x32(pa, ones, sum_p);
            if constexpr (!kPlaneRows) sum_p = mfma16x16x32(pl, ones, sum_p);
        }
    };

    auto load_tile = [&](MfmaTile<F>& t, int t0) {
        if constexpr (F == KvFormat::I4) t.load(x, t0, p.group_size, w1 - 1);
        else t.load(x, t0);
    };
    // The scheduling barriers keep each tile's V loads next to its K loads
    // (the scheduler would otherwise sink them below the QK products, which
    // costs a second memory round trip per tile).
    if constexpr (F != KvFormat::I4) {
        // One 16 / 8 KiB fp16 / INT8 tile per wave in flight already keeps
        // 32 / 16 MiB of loads queued chip-wide; a second one only lengthens
        // the queue (measured slower for both).
        //
        // INT8 with splits: KV head h starts its walk h / Hkv of the way into
        // the sequence and wraps (tile t reads tile (t + rot) mod n_tiles),
        // so the heads of a batch row do not all read the same relative
        // position of their K and V at once. The rotation depends on the
        // head alone, so a batch permutation still permutes the outputs bit
        // for bit. Against the unrotated walk on four boxes (us): B=4
        // S=4096 11.6-12.0 -> 10.6 on every box, A8 15.5-16.1 -> 15.4-15.7,
        // B=16 26.2-29.2 -> 26.1-28.9, B=8 S=1024 +1 %, and B=8 S=16384
        // either way with the box (49-59 -> 46.8, 51.8 -> 55.0); without
        // splits (B=64) it was 2.5 % slower, so unsplit plans keep the plain
        // walk.
        // fp16 is not rotated: B=8 S=8192 53-63 -> 46-49 us, but the A16
        // headline 25.1-25.3 -> 25.5-28.0 and B=64 +1.3 %.
        const int n_rt = (w1 + kTile - 1) / kTile;
        const int rot = (F == KvFormat::I8 && p.n_splits > 1)
            ? (int)((long)kvh * n_rt / p.n_kv_heads) * kTile : 0;
        const int n_tok = n_rt * kTile;
        for (int t0 = w0; t0 < w1; t0 += p.n_splits * NW * kTile) {
            MfmaTile<F> tile;
            int tp = t0 + rot;
            if (tp >= n_tok) tp -= n_tok;
            load_tile(tile, tp);
            __builtin_amdgcn_sched_barrier(0);
            step(tile, tp);
        }
    } else if (w0 < w1) {
        // INT4 tiles are 4 KiB per wave: the next tile's loads are issued
        // before the current tile's arithmetic. The prefetch is
        // unconditional (past the range it reads zeros through the buffer
        // bound): a conditional one would make the compiler's wait count
        // assume it absent and wait for every outstanding load.
        MfmaTile<F> ta, tb;
        int t0 = w0;
        load_tile(ta, t0);
        while (true) {
            load_tile(tb, t0 + kWaveStride);
            __builtin_amdgcn_sched_barrier(0);
            step(ta, t0);
            t0 += kWaveStride;
            if (t0 >= w1) break;
            load_tile(ta, t0 + kWaveStride);
            __builtin_amdgcn_sched_barrier(0);
            step(tb, t0);
            t0 += kWaveStride;
            if (t0 >= w1) break;
        }
    }

    // ---- merge the wave states through LDS ----
    const float l_tot = row16_sum(l_run);   // lane group g: head g's denominator

    __shared__ __attribute__((aligned(16))) float s_o[NW][HPW][kHeadDim];
    __shared__ float s_m[NW][HPW];
    __shared__ float s_l[NW][HPW];
    __shared__ uint32_t s_last;
    constexpr float kInvP = 1.0f / MfmaTile<F>::kPScale;
    if constexpr (kPlaneRows) {   // hi + lo planes: lane group g's PV rows plus lane group g ^ 1's
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[j][i] += __shfl_xor(o[j][i], 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) sum_p[i] += __shfl_xor(sum_p[i], 16);
    }
    if constexpr (F != KvFormat::F16) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[j][i] = (o[j][i] - MfmaTile<F>::kVBias[j & 1] * sum_p[i]) * MfmaTile<F>::kVUnscale[j & 1];
    }
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < HPW; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) s_o[wave][i][8 * c + j] = o[j][i] * kInvP;
    }
    if (c == 0 && g < HPW) {
        s_m[wave][g] = m_run;
        s_l[wave][g] = l_tot;
    }
    __syncthreads();
    finish_split<NW, HPW, NW * kWave>(p, s_o, s_m, s_l, &s_last, b, kvh, hchunk, split, head0);
}

// ===========================================================================
// fp16, 16-token tiles with the next tile in flight
// ===========================================================================
// The kernel above issues a whole 16 KiB fp16 tile per wave and waits for
// it; here a wave walks 16-token tiles (4 KiB of K, 4 KiB of V), the split's
// tiles interleaved as above at 16-token granularity (split s, wave w reads
// tiles s + n_splits * (w + NW * i)), with the next tile's loads issued
// before the current tile's arithmetic: the same 16 KiB per wave stays in
// flight, in two staggered halves, and a wave's reads end in 8 KiB steps
// instead of 16 KiB ones, which evens out when the waves of the grid finish.
// QK is one 16-token block; PV runs v_mfma_f32_16x16x16_f16 over the tile's
// 16 tokens (hi and lo P planes against the same B operand).
// launch_attention picks it for fp16 where it measured faster (see
// use_f16_half_tiles).
constexpr int kHalfTile = 16;

struct F16HalfTile {
    static constexpr uint32_t kRow = kHeadDim * 2;
    u32x4 k[4];   // lane (g, c): token c, channels 32 ks + 8 g
    u32x4 v[4];   // lane (g, c): token 4 g + e, channels 8 c
    // Cache policy (aux bits: 1 = sc0, 2 = nt): K non-temporal, V sc0 and
    // non-temporal. Against K cacheable and V non-temporal (the 32-token
    // tile's policy, which stays faster there), on three boxes (us): A16
    // 24.8-25.2 -> 23.2-24.3 (12 reps on one box all at 24.1-24.3; a second
    // box half of 8 reps at 23.2-23.5, half at 25.4-26.5), B=16 S=4096
    // 43.9-44.0 -> 41.4-41.5, B=8 S=8192 49.5-53.9 -> 43.0-45.6, B=8 S=2048
    // 14.9 -> 14.7, but B=4 S=4096 15.2-15.5 -> 15.4-16.3. K non-temporal
    // with V non-temporal, or sc0 on both, fell into a ~30 us mode on 7 of
    // 12 A16 reps on one box; this pair did not.
    __device__ __forceinline__ void load(const TileCtx& x, int t0) {
        const uint32_t so = (uint32_t)t0 * kRow;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            k[ks] = __builtin_amdgcn_raw_buffer_load_b128(x.rk, (int)x.koff, (int)(so + 64 * ks), 2);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[e] = __builtin_amdgcn_raw_buffer_load_b128(x.rv, (int)x.voff, (int)(so + kRow * e), 3);
    }
    // B operand of PV MFMA j (channels 8 c + j): V[4 g + e][8 c + j], e = 0..3.
    __device__ __forceinline__ f16x4 vop(int j) const {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t d0 = perm_b32(v[1][j >> 1], v[0][j >> 1], sel);
        const uint32_t d1 = perm_b32(v[3][j >> 1], v[2][j >> 1], sel);
        return __builtin_bit_cast(f16x4, u32x2{d0, d1});
    }
};

template <int HPW, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(2)))
void decode_attention_f16h_kernel(AttnParams p) {
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / p.n_hchunks;
    const int hchunk = blockIdx.y % p.n_hchunks;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int head0 = kvh * p.gqa + hchunk * HPW;
    const uint16_t* qrow = p.q + ((long)b * p.n_heads + head0 + ((c >> 2) % HPW)) * kHeadDim;
    f16x8 qa[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qa[ks] = as_f16x8(load16(qrow + 32 * ks + 8 * g));
    f32x4 o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;
    __shared__ __attribute__((aligned(16))) uint16_t s_p[NW][2][4][kHalfTile];
    __shared__ __attribute__((aligned(16))) float s_alpha[NW][4];

    const int w0 = (split + p.n_splits * wave) * kHalfTile;
    const int w1 = p.seqlen;
    const int stride = p.n_splits * NW * kHalfTile;
    TileCtx x;
    {
        const long slab = (long)(b * p.n_kv_heads + kvh);
        constexpr uint32_t kRow = F16HalfTile::kRow;
        const long kv_base = slab * p.kv_buf_len * (long)kRow;
        const uint32_t range = (uint32_t)max(w1, 0) * kRow;
        x.rk = make_buffer_rsrc(static_cast<const char*>(p.k) + kv_base, range);
        x.rv = make_buffer_rsrc(static_cast<const char*>(p.v) + kv_base, range);
        x.koff = (uint32_t)c * kRow + 16u * g;
        x.voff = 4u * g * kRow + 16u * c;
    }

    auto step = [&](const F16HalfTile& tile, const int t0) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) acc = mfma16x16x32(qa[ks], as_f16x8(tile.k[ks]), acc);
        const float s = (t0 + c) < w1 ? acc[0] * p.scale_log2 : -INFINITY;
        const float tmax = row16_max(s);
        const float mn = fmaxf(m_run, tmax);
        const float msafe = (mn == -INFINITY) ? 0.0f : mn;
        const float alpha = __builtin_amdgcn_exp2f(m_run - msafe);
        const bool rescale = __builtin_amdgcn_ballot_w64(mn != m_run) != 0;
        m_run = mn;
        const float pr = __builtin_amdgcn_exp2f(s - msafe);
        l_run = fmaf(l_run, alpha, pr);
        if (g < HPW) {
            const float xv = pr * MfmaTile<KvFormat::F16>::kPScale;
            const uint16_t h = f2h_bits(xv);
            s_p[wave][0][g][c] = h;
            s_p[wave][1][g][c] = f2h_bits(xv - h2f(h));
            if (c == 0) s_alpha[wave][g] = alpha;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // A operand of PV: row c (head c % HPW), tokens 4 g .. 4 g + 3.
        const f16x4 pa = __builtin_bit_cast(f16x4, *reinterpret_cast<const u32x2*>(&s_p[wave][0][c % HPW][4 * g]));
        const f16x4 pl = __builtin_bit_cast(f16x4, *reinterpret_cast<const u32x2*>(&s_p[wave][1][c % HPW][4 * g]));
        if (rescale) {
            const f32x4 al = *reinterpret_cast<const f32x4*>(&s_alpha[wave][0]);
            float a4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a4[i] = al[i % HPW];
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[j][i] *= a4[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const f16x4 vb = tile.vop(j);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vb, o[j], 0, 0, 0);
            o[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vb, o[j], 0, 0, 0);
        }
    };

    if (w0 < w1) {
        // The prefetch past the range reads zeros through the buffer bound;
        // it is unconditional so that the wait counts stay exact.
        F16HalfTile ta, tb;
        int t0 = w0;
        ta.load(x, t0);
        while (true) {
            tb.load(x, t0 + stride);
            __builtin_amdgcn_sched_barrier(0);
            step(ta, t0);
            t0 += stride;
            if (t0 >= w1) break;
            ta.load(x, t0 + stride);
            __builtin_amdgcn_sched_barrier(0);
            step(tb, t0);
            t0 += stride;
            if (t0 >= w1) break;
        }
    }

    const float l_tot = row16_sum(l_run);
    __shared__ __attribute__((aligned(16))) float s_o[NW][HPW][kHeadDim];
    __shared__ float s_m[NW][HPW];
    __shared__ float s_l[NW][HPW];
    __shared__ uint32_t s_last;
    constexpr float kInvP = 1.0f / MfmaTile<KvFormat::F16>::kPScale;
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < HPW; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) s_o[wave][i][8 * c + j] = o[j][i] * kInvP;
    }
    if (c == 0 && g < HPW) {
        s_m[wave][g] = m_run;
        s_l[wave][g] = l_tot;
    }
    __syncthreads();
    finish_split<NW, HPW, NW * kWave>(p, s_o, s_m, s_l, &s_last, b, kvh, hchunk, split, head0);
}

// ===========================================================================
// VALU fallback kernel
// ===========================================================================

constexpr int kRows = kAttnThreads / 16;   // 16 token rows per workgroup
constexpr int kUnroll = 4;                 // tokens per row per step
constexpr int kStepTokens = kRows * kUnroll;

template <KvFormat F>
struct KvRow;

// Per-lane view of one token row: 8 fp32 channels of K and of V.
template <>
struct KvRow<KvFormat::F16> {
    u32x4 kraw, vraw;
    __device__ __forceinline__ void load(const AttnParams& p, long row_base, int t, int c) {
        const long off = (row_base + t) * kHeadDim + 8 * c;
        kraw = load16(static_cast<const uint16_t*>(p.k) + off);
        vraw = load16(static_cast<const uint16_t*>(p.v) + off);
    }
    __device__ __forceinline__ void k_f32(float kf[8]) const { f16x8_to_f32(kraw, kf); }
    __device__ __forceinline__ void v_f32(float vf[8]) const { f16x8_to_f32(vraw, vf); }
    __device__ __forceinline__ float k_token_scale() const { return 1.0f; }
    __device__ __forceinline__ float v_token_scale() const { return 1.0f; }
};

template <>
struct KvRow<KvFormat::I8> {
    u32x2 kraw, vraw;
    uint16_t ks, vs;
    __device__ __forceinline__ void load(const AttnParams& p, long row_base, int t, int c) {
        const long off = (row_base + t) * kHeadDim + 8 * c;
        kraw = load8(static_cast<const int8_t*>(p.k) + off);
        vraw = load8(static_cast<const int8_t*>(p.v) + off);
        ks = p.k_scale[row_base + t];
        vs = p.v_scale[row_base + t];
    }
    __device__ __forceinline__ void k_f32(float kf[8]) const { i8x8_to_f32(kraw, kf); }
    __device__ __forceinline__ void v_f32(float vf[8]) const { i8x8_to_f32(vraw, vf); }
    __device__ __forceinline__ float k_token_scale() const { return h2f(ks); }
    __device__ __forceinline__ float v_token_scale() const { return h2f(vs); }
};

template <>
struct KvRow<KvFormat::I4> {
    uint32_t kraw, vraw;
    uint16_t vs;
    __device__ __forceinline__ void load(const AttnParams& p, long row_base, int t, int c) {
        const long off = (row_base + t) * (kHeadDim / 2) + 4 * c;
        kraw = load4(static_cast<const int8_t*>(p.k) + off);
        vraw = load4(static_cast<const int8_t*>(p.v) + off);
        vs = p.v_scale[row_base + t];
    }
    __device__ __forceinline__ void k_f32(float kf[8]) const { i4x8_to_f32(kraw, kf); }
    __device__ __forceinline__ void v_f32(float vf[8]) const { i4x8_to_f32(vraw, vf); }
    __device__ __forceinline__ float k_token_scale() const { return 1.0f; }
    __device__ __forceinline__ float v_token_scale() const { return h2f(vs); }
};

// 16 rows of 16 lanes: lane c of a row owns channels 8c..8c+7 of one token;
// row r walks the split's tokens r, r+16, ... four at a time; dot products
// are reduced inside the DPP row and each row keeps its own softmax state.
template <KvFormat F, int HPW>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_valu_kernel(AttnParams p) {
    const int split = blockIdx.x;
    const int kvh = blockIdx.y / p.n_hchunks;
    const int hchunk = blockIdx.y % p.n_hchunks;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;
    const int row = tid >> 4;
    const int c = tid & 15;

    const int head0 = kvh * p.gqa + hchunk * HPW;
    const long row_base = (long)(b * p.n_kv_heads + kvh) * p.kv_buf_len;

    // q pre-scaled by softmax_scale * log2(e): scores come out in log2 units.
    float q[HPW][8];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        const u32x4 raw = load16(p.q + ((long)b * p.n_heads + head0 + h) * kHeadDim + 8 * c);
        f16x8_to_f32(raw, q[h]);
#pragma unroll
        for (int e = 0; e < 8; ++e) q[h][e] *= p.scale_log2;
    }

    float m[HPW], l[HPW], o[HPW][8];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
    }

    const int t_begin = split * p.chunk;
    const int t_end = min(t_begin + p.chunk, p.seqlen);

    int cur_group = -1;
    float kscale[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) kscale[e] = 1.0f;
    const uint16_t* ks_base =
        p.k_scale + (long)(b * p.n_kv_heads + kvh) * p.n_groups * kHeadDim + 8 * c;

    for (int t0 = t_begin; t0 < t_end; t0 += kStepTokens) {
        KvRow<F> kv[kUnroll];
        int tok[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            tok[u] = t0 + row + kRows * u;
            const int tl = min(tok[u], t_end - 1);   // keep loads in bounds
            kv[u].load(p, row_base, tl, c);
        }

        float s[kUnroll][HPW];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            float kf[8];
            kv[u].k_f32(kf);
            if constexpr (F == KvFormat::I4) {
                const int gi = min(tok[u], t_end - 1) / p.group_size;
                if (gi != cur_group) {
                    cur_group = gi;
                    float tmp[8];
                    f16x8_to_f32(load16(ks_base + (long)gi * kHeadDim), tmp);
#pragma unroll
                    for (int e = 0; e < 8; ++e) kscale[e] = tmp[e];
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) kf[e] *= kscale[e];
            }
            const float kts = kv[u].k_token_scale();
#pragma unroll
            for (int h = 0; h < HPW; ++h) {
                float acc = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc = fmaf(q[h][e], kf[e], acc);
                acc = row16_sum(acc);
                s[u][h] = (tok[u] < t_end) ? acc * kts : -INFINITY;
            }
        }

#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            float mn = m[h];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) mn = fmaxf(mn, s[u][h]);
            const float msafe = (mn == -INFINITY) ? 0.0f : mn;
            const float alpha = __builtin_amdgcn_exp2f(m[h] - msafe);
            l[h] *= alpha;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[h][e] *= alpha;
            m[h] = mn;
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) s[u][h] = __builtin_amdgcn_exp2f(s[u][h] - msafe);
        }

#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            float vf[8];
            kv[u].v_f32(vf);
            const float vts = kv[u].v_token_scale();
#pragma unroll
            for (int h = 0; h < HPW; ++h) {
                l[h] += s[u][h];
                const float pv = s[u][h] * vts;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[h][e] = fmaf(pv, vf[e], o[h][e]);
            }
        }
    }

    __shared__ __attribute__((aligned(16))) float s_o[kRows][HPW][kHeadDim];
    __shared__ float s_m[kRows][HPW];
    __shared__ float s_l[kRows][HPW];
    __shared__ uint32_t s_last;
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[row][h][8 * c + e] = o[h][e];
        if (c == 0) {
            s_m[row][h] = m[h];
            s_l[row][h] = l[h];
        }
    }
    __syncthreads();
    finish_split<kRows, HPW, kAttnThreads>(p, s_o, s_m, s_l, &s_last, b, kvh, hchunk, split, head0);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

int heads_per_wg(int gqa) {
    if (gqa % 4 == 0) return 4;
    if (gqa % 2 == 0) return 2;
    return 1;
}

}  // namespace

AttnPlan plan_attention(int batch, int n_heads, int n_kv_heads, int seqlen) {
    AttnPlan pl{};
    const int gqa = n_heads / n_kv_heads;
    pl.hpw = heads_per_wg(gqa);
    pl.n_hchunks = gqa / pl.hpw;
    const long base_wgs = (long)batch * n_kv_heads * pl.n_hchunks;
    const int cus = device_cu_count();
    // Aim for kAttnWgsPerCu workgroups per CU. Calls that must split the
    // sequence to fill the chip use 8-wave workgroups (more loads in flight
    // per CU); otherwise 4 waves. Every split
    // gets at least one 32-token tile per wave.
    // A short sequence that 8-wave splits (one 256-token step each) cannot
    // spread over the chip runs 4-wave splits instead, as long as that keeps
    // the combine to at most 8 partials: at B=1, S=1024 the 8 splits took
    // 6.9 us against 9.0 us for 4; at B=1, S=4096 32 splits took 12.6 us
    // against 10.4 us for 16 (the combine grows with the split count).
    const long target = (long)kAttnWgsPerCu * cus;
    const long splits8 = ((long)seqlen + 8 * kTile - 1) / (8 * kTile);
    const bool short_seq = base_wgs * splits8 < target && 2 * splits8 <= 8;
    pl.waves = (base_wgs < target && !short_seq) ? 8 : 4;
    // Splits that would give each of 8 waves a single 32-token tile run as
    // 4-wave workgroups at twice the split count (two per CU), as long as the
    // combine stays at <= 8 partials: B=8, S=1024 11.36-11.40 -> 10.94-11.03
    // us; with more partials (B=4, S=1024; B=1, S=4096) it was slower.
    const bool thin = pl.waves == 8 && (long)seqlen * base_wgs <= target * 8 * kTile &&
                      2 * ((target + base_wgs - 1) / base_wgs) <= 8;
    if (thin) pl.waves = 4;
    const int step = kTile * pl.waves;
    long want = ((thin ? 2 : 1) * target + base_wgs - 1) / base_wgs;
    const long max_useful = (seqlen + step - 1) / step;
    if (want > max_useful) want = max_useful;
    if (want > kMaxAttnSplits) want = kMaxAttnSplits;
    if (base_wgs > kMaxCounters) want = 1;   // enough workgroups without splitting
    if (want < 1) want = 1;
    int chunk = (int)((seqlen + want - 1) / want);
    chunk = ((chunk + step - 1) / step) * step;
    if (chunk < step) chunk = step;
    pl.chunk = chunk;
    pl.n_splits = seqlen > 0 ? (seqlen + chunk - 1) / chunk : 1;
    pl.n_slot_groups = base_wgs;
    const size_t slots = (size_t)base_wgs * pl.n_splits * pl.hpw;
    const size_t ml = align_up(slots * 2 * sizeof(float), 256);
    const size_t po = align_up(slots * kHeadDim * sizeof(float), 256);
    pl.workspace_bytes = (pl.n_splits > 1) ? kCounterBytes + ml + po : 0;
    pl.off_ml = kCounterBytes;
    pl.off_o = kCounterBytes + ml;
    return pl;
}

// fp16 16-token tiles (decode_attention_f16h_kernel, with its cache policy)
// against 32-token ones, forced through the override, two boxes, four
// interleaved reps each (median us, 32 -> 16): B=8 S=4096 25.69 -> 24.65,
// B=16 S=4096 45.34 -> 41.79, B=32 S=1024 23.28 -> 21.51, B=16 S=1024 15.04
// -> 14.08, B=32 S=2048 41.70 -> 39.42, B=32 S=4096 79.92 -> 75.89, B=16
// S=8192 82.25 -> 78.56, B=8 S=16384 83.17 -> 79.82, B=8 S=2048 15.58 ->
// 14.89, B=64 S=4096 155.03 -> 150.79, B=64 S=8192 308.86 -> 300.36, B=4
// S=4096 15.96 -> 15.57, B=4 S=8192 26.61 -> 26.21, B=8 S=1024 10.26-10.37
// -> 10.06-10.22; slower where the grid does not fill the chip in whole
// rounds (B=12 S=4096, 288 workgroups, 46.60 -> 50.40; B=24 S=4096, 384,
// 73.16 -> 73.94; B=48 S=2048, 384, 69.07 -> 70.09), with fewer than 32
// slabs (B=1 S=4096 9.29 -> 9.75, B=2 S=16384 28.08 -> 29.87) and with one
// tile per 8-wave wave (B=4 S=2048 10.51 -> 10.85); even at B=8 S=32768
// (163.78 -> 163.88). The rule: at least 32 (batch, kv head, head chunk)
// slabs, a workgroup count that is a multiple of the CU count, and at least
// two 32-token tiles per wave unless the workgroups have 4 waves. It takes
// the faster form at 24 of these 26 shapes (the earlier rule, 2-8 tiles per
// wave, at 16). The override (llmik_attention_set_plan_override) forces
// either.
namespace {
std::atomic<int> g_f16_tiles{-1};   // -1: the rule, 0: 32-token tiles, 1: 16-token tiles
}  // namespace

void set_attention_plan_override(int f16_half_tiles) {
    g_f16_tiles.store(f16_half_tiles < 0 ? -1 : (f16_half_tiles ? 1 : 0), std::memory_order_relaxed);
}

static bool use_f16_half_tiles(const AttnPlan& pl, int seqlen) {
    const int mode = g_f16_tiles.load(std::memory_order_relaxed);
    if (mode >= 0) return mode == 1;
    const long tiles = (seqlen + kTile - 1) / kTile;
    const long per_wave = (tiles + (long)pl.n_splits * pl.waves - 1) / ((long)pl.n_splits * pl.waves);
    const long wgs = (long)pl.n_slot_groups * pl.n_splits;
    return pl.n_slot_groups >= 32 && wgs % device_cu_count() == 0 && (per_wave >= 2 || pl.waves == 4);
}

template <KvFormat F, int HPW>
static void launch_kernel(const AttnParams& p, dim3 grid, bool mfma, int waves, bool half, hipStream_t stream) {
    if (F == KvFormat::F16 && mfma && half) {
        if (waves == 8)
            hipLaunchKernelGGL((decode_attention_f16h_kernel<HPW, 8>), grid, dim3(8 * kWave), 0, stream, p);
        else
            hipLaunchKernelGGL((decode_attention_f16h_kernel<HPW, 4>), grid, dim3(4 * kWave), 0, stream, p);
        return;
    }
    if (mfma && waves == 8) {
        hipLaunchKernelGGL((decode_attention_mfma_kernel<F, HPW, 8>), grid, dim3(8 * kWave), 0,
                           stream, p);
    } else if (mfma) {
        hipLaunchKernelGGL((decode_attention_mfma_kernel<F, HPW, 4>), grid, dim3(4 * kWave), 0,
                           stream, p);
    } else {
        hipLaunchKernelGGL((decode_attention_valu_kernel<F, HPW>), grid, dim3(kAttnThreads), 0,
                           stream, p);
    }
}

template <KvFormat F>
static int launch_attention(const AttnLaunch& a, hipStream_t stream) {
    const AttnPlan pl = plan_attention(a.batch, a.n_heads, a.n_kv_heads, a.seqlen);
    if (pl.n_splits > 1 && a.workspace_bytes < pl.workspace_bytes) {
        return set_error(LLMIK_ERR_WORKSPACE, "workspace too small for this attention call");
    }
    AttnParams p{};
    p.q = static_cast<const uint16_t*>(a.q);
    p.k = a.k;
    p.v = a.v;
    p.k_scale = static_cast<const uint16_t*>(a.k_scale);
    p.v_scale = static_cast<const uint16_t*>(a.v_scale);
    p.out = static_cast<uint16_t*>(a.out);
    char* ws = static_cast<char*>(a.workspace);
    p.counters = reinterpret_cast<uint32_t*>(ws);
    p.part_ml = ws ? reinterpret_cast<float*>(ws + pl.off_ml) : nullptr;
    p.part_o = ws ? reinterpret_cast<float*>(ws + pl.off_o) : nullptr;
    p.n_heads = a.n_heads;
    p.n_kv_heads = a.n_kv_heads;
    p.seqlen = a.seqlen;
    p.kv_buf_len = a.kv_buf_len;
    p.group_size = a.group_size > 0 ? a.group_size : 1;
    p.n_groups = a.n_groups;
    p.n_splits = pl.n_splits;
    p.chunk = pl.chunk;
    p.n_hchunks = pl.n_hchunks;
    p.gqa = a.n_heads / a.n_kv_heads;
    p.scale_log2 = a.softmax_scale * kLog2e;

    // The MFMA path keeps each 32-token tile inside one INT4 K-scale group,
    // and addresses a (batch, kv head) slab with 32-bit buffer offsets.
    const long row_bytes = (F == KvFormat::F16) ? 2 * kHeadDim : (F == KvFormat::I8 ? kHeadDim : kHeadDim / 2);
    const bool mfma = ((F != KvFormat::I4) || (p.group_size % kTile == 0)) &&
                      (long)a.kv_buf_len * row_bytes < (1L << 32);
    const bool half = (F == KvFormat::F16) && mfma && use_f16_half_tiles(pl, a.seqlen);
    dim3 grid(pl.n_splits, a.n_kv_heads * pl.n_hchunks, a.batch);
    switch (pl.hpw) {
        case 4: launch_kernel<F, 4>(p, grid, mfma, pl.waves, half, stream); break;
        case 2: launch_kernel<F, 2>(p, grid, mfma, pl.waves, half, stream); break;
        default: launch_kernel<F, 1>(p, grid, mfma, pl.waves, half, stream); break;
    }
    return check_launch();
}

int launch_attention_f16(const AttnLaunch& a, hipStream_t s) { return launch_attention<KvFormat::F16>(a, s); }
int launch_attention_i8(const AttnLaunch& a, hipStream_t s) { return launch_attention<KvFormat::I8>(a, s); }
int launch_attention_i4(const AttnLaunch& a, hipStream_t s) { return launch_attention<KvFormat::I4>(a, s); }

}  // namespace llmik
