// Quantize-on-append KV-cache writers for gfx950, bit-exact with
// reference/kv_cache_ref.py applied to x.float():
//   scale = max(absmax / qmax, 1e-8)            (fp32, IEEE division)
//   q     = clamp(round_half_even(x / scale), -qmax, qmax)
//   scale stored as fp16 (round to nearest even)
// (kv_cache_ref.py:46-62 per token, :73-112 per channel groupwise.)
// Non-finite inputs follow torch: amax propagates NaN (kv_cache_ref.py:59-61)
// and clamp keeps it, so a row (or group channel) holding a NaN stores scale
// NaN and codes 0; one holding +-inf stores scale +inf, and every quotient is
// then 0 (finite / inf) or NaN (inf / inf), whose int8 conversion is 0.
// The reference CUDA writers multiply by an approximate reciprocal under
// fast-math (kernels/kv_cache/kv_compress.cu:50-58,128-129,200-201) and are
// only within +-1 code of the oracle; these kernels divide exactly.
//
// Layouts (one "row" per (batch, kv_head) pair):
//   x     [rows, src_len, 128] fp16; tokens [0, n_tok) of each row are read
//   int8  [rows, dst_len, 128] int8, scale [rows, dst_len] fp16
//   int4  [rows, dst_len, 64] packed (channel 2i -> low nibble of byte i),
//         scale as above
//   K groupwise int4: scale [rows, dst_groups, 128] fp16
// Token t of a row is written to cache position dst_off + t (K groupwise:
// dst_off is a multiple of group_size and group g goes to scale slot
// dst_off / group_size + g). The out-of-place ops are the identity map
// src_len = dst_len = n_tok, dst_off = 0.
#include <type_traits>

#include "device_common.hpp"
#include "llmik_internal.hpp"

namespace llmik {

constexpr int kWriterThreads = 256;   // 32 token groups of 8 lanes, or 16 rows of 16 lanes

// Token indexing of the writers: `flat` runs over the n_tok tokens of every
// (batch, kv_head) row; src / dst give the token's position in x and in the
// destination cache.
struct TokenMap {
    uint32_t n_tok;     // tokens per (batch, kv_head) row to quantise
    uint32_t src_len;   // token stride of x
    uint32_t dst_len;   // token stride of the destination cache
    uint32_t dst_off;   // cache position of token 0
    __device__ __forceinline__ long src(uint32_t flat) const {
        const uint32_t r = flat / n_tok;
        return (long)r * src_len + (flat - r * n_tok);
    }
    __device__ __forceinline__ long dst(uint32_t flat) const {
        const uint32_t r = flat / n_tok;
        return (long)r * dst_len + dst_off + (flat - r * n_tok);
    }
};

// Per token: 8 lanes per token; lane c of an 8-lane group owns channels
// 8c..8c+7 and 64+8c..64+8c+7, so each load instruction reads the first or
// the second half of its tokens' rows, contiguous. The per-token work (the
// 8-lane DPP max, the scale's division, the reciprocal, the addresses) is
// shared by 16 values per lane. The absmax runs on the fp16 bit patterns
// (sign masked, packed unsigned max), the same order as the fp32 magnitudes
// (NaN above +inf). A workgroup covers 32 groups x kTokensPerRow8
// consecutive tokens. Against 16 lanes per token with 8 values each (two
// tokens per lane group), same bits, on one box (us): INT8 B=8 S=4096 18.87
// -> 18.50, INT4 V 17.79 -> 16.25, INT8 / INT4 V B=64 131.8 / 120.7 ->
// 125.5 / 110.2, S=1000 6.62 / 6.48 -> 6.27 / 5.95; two tokens per group
// (64 per workgroup) was slower for INT8 (20.4) and at small shapes.
constexpr int kTokensPerRow8 = 1;

__device__ __forceinline__ uint32_t row8_umax(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppQuadXor1, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppQuadXor2, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppRowHalfMirror, 0xF, 0xF, true));
    return v;
}

template <int QMAX, bool PACK4, bool MAPPED>
__global__ __launch_bounds__(kWriterThreads) void quantize_per_token_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, uint16_t* __restrict__ scale,
    long rows, TokenMap map) {
    constexpr int kGroups = kWriterThreads / 8;
    const long blk = (long)blockIdx.x * (kGroups * kTokensPerRow8);
    const int grp = threadIdx.x >> 3;
    const int c = threadIdx.x & 7;
    u32x4 raw[kTokensPerRow8][2];
#pragma unroll
    for (int i = 0; i < kTokensPerRow8; ++i) {
        // Tokens past the end take part in the DPP reduction on a clamped,
        // in-bounds token but store nothing.
        const long flat = min(blk + kGroups * i + grp, rows - 1);
        const long src = MAPPED ? map.src((uint32_t)flat) : flat;
        raw[i][0] = stream16(x + src * 128 + 8 * c);
        raw[i][1] = stream16(x + src * 128 + 64 + 8 * c);
    }
#pragma unroll
    for (int i = 0; i < kTokensPerRow8; ++i) {
        const long flat = blk + kGroups * i + grp;
        // |x| of the 16 fp16 values as bit patterns, packed max per half.
        uint32_t m = 0u;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t a = raw[i][h][d] & 0x7FFF7FFFu;
                m = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(
                        __builtin_bit_cast(u16x2, m), __builtin_bit_cast(u16x2, a)));
            }
        const uint32_t m16 = max(m & 0xFFFFu, m >> 16);
        const uint32_t amax16 = row8_umax(m16);
        const float amax = h2f((uint16_t)amax16);   // exact; NaN stays NaN, inf stays inf
        const float sc = sym_scale(__float_as_uint(amax), (float)QMAX);
        const float rcp = recip_approx(sc);
        float xf[16];
        f16x8_to_f32(raw[i][0], xf);
        f16x8_to_f32(raw[i][1], xf + 8);
        int code[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) code[e] = sym_code(xf[e], sc, rcp, QMAX);
        if (flat < rows) {
            const long row = MAPPED ? map.dst((uint32_t)flat) : flat;
            if constexpr (PACK4) {
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    w0 |= (uint32_t)(code[e] & 0xF) << (4 * e);
                    w1 |= (uint32_t)(code[8 + e] & 0xF) << (4 * e);
                }
                __builtin_nontemporal_store(w0, reinterpret_cast<uint32_t*>(q + row * 64 + 4 * c));
                __builtin_nontemporal_store(w1, reinterpret_cast<uint32_t*>(q + row * 64 + 32 + 4 * c));
            } else {
                uint32_t w[4];
#pragma unroll
                for (int d = 0; d < 4; ++d)
                    w[d] = (uint32_t)(code[4 * d] & 0xFF) | ((uint32_t)(code[4 * d + 1] & 0xFF) << 8) |
                           ((uint32_t)(code[4 * d + 2] & 0xFF) << 16) | ((uint32_t)(code[4 * d + 3] & 0xFF) << 24);
                __builtin_nontemporal_store(u32x2{w[0], w[1]}, reinterpret_cast<u32x2*>(q + row * 128 + 8 * c));
                __builtin_nontemporal_store(u32x2{w[2], w[3]}, reinterpret_cast<u32x2*>(q + row * 128 + 64 + 8 * c));
            }
            if (c == 0) scale[row] = f2h_bits(sc);
        }
    }
}

// K per channel, group-wise: one workgroup per (batch, kv_head, group). 16
// rows of 16 lanes: row r holds the group's tokens r, r+16, ... (at most
// TPR of them, group_size <= 16 * TPR) in registers; lane c owns channels
// 8c..8c+7. The per-channel absmax is merged across rows in LDS, then the
// codes are formed from the registers: the input is read once.
template <int TPR>
__global__ __launch_bounds__(kWriterThreads) void quantize_k_groupwise_int4_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, uint16_t* __restrict__ scale,
    int group_size, TokenMap map, int dst_groups) {
    const int seqlen = (int)map.n_tok;
    const int g = blockIdx.x;
    const long bh = blockIdx.y;   // batch * n_kv_heads + kv_head
    const int row = threadIdx.x >> 4;
    const int c = threadIdx.x & 15;
    const int t_start = g * group_size;
    const int t_end = min(t_start + group_size, seqlen);
    const long base = bh * map.src_len;                     // x row of token 0
    const long qbase = bh * map.dst_len + map.dst_off;      // cache row of token 0
    const long sslot = bh * dst_groups + map.dst_off / group_size + g;

    u32x4 raw[TPR];
#pragma unroll
    for (int i = 0; i < TPR; ++i) {
        const int t = min(t_start + row + 16 * i, t_end - 1);   // in bounds; duplicates do not move the max
        raw[i] = stream16(x + (base + t) * 128 + 8 * c);
    }
    uint32_t amax[8];   // NaN-propagating absmax per channel, as bits
#pragma unroll
    for (int e = 0; e < 8; ++e) amax[e] = 0u;
#pragma unroll
    for (int i = 0; i < TPR; ++i) {
        float xf[8];
        f16x8_to_f32(raw[i], xf);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax[e] = max(amax[e], abs_bits(xf[e]));
    }

    __shared__ uint32_t s_max[16][128];
    __shared__ float s_scale[128];
#pragma unroll
    for (int e = 0; e < 8; ++e) s_max[row][8 * c + e] = amax[e];
    __syncthreads();
    if (threadIdx.x < 128) {
        uint32_t m = 0u;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = max(m, s_max[r][threadIdx.x]);
        const float sc = sym_scale(m, 7.0f);
        s_scale[threadIdx.x] = sc;
        scale[sslot * 128 + threadIdx.x] = f2h_bits(sc);
    }
    __syncthreads();

    float sv[8], rcp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        sv[e] = s_scale[8 * c + e];
        rcp[e] = recip_approx(sv[e]);
    }
#pragma unroll
    for (int i = 0; i < TPR; ++i) {
        const int t = t_start + row + 16 * i;
        float xf[8];
        f16x8_to_f32(raw[i], xf);
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= (uint32_t)(sym_code(xf[e], sv[e], rcp[e], 7) & 0xF) << (4 * e);
        if (t < t_end)
            __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(q + (qbase + t) * 64 + 4 * c));
    }
}

// Group sizes beyond 16 * 8 tokens: the group is walked twice (max, then
// codes); the second pass re-reads it from the caches.
__global__ __launch_bounds__(kWriterThreads) void quantize_k_groupwise_int4_large_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, uint16_t* __restrict__ scale,
    int group_size, TokenMap map, int dst_groups) {
    const int seqlen = (int)map.n_tok;
    const int g = blockIdx.x;
    const long bh = blockIdx.y;
    const int row = threadIdx.x >> 4;
    const int c = threadIdx.x & 15;
    const int t_start = g * group_size;
    const int t_end = min(t_start + group_size, seqlen);
    const long base = bh * map.src_len;                     // x row of token 0
    const long qbase = bh * map.dst_len + map.dst_off;      // cache row of token 0
    const long sslot = bh * dst_groups + map.dst_off / group_size + g;

    uint32_t amax[8];   // NaN-propagating absmax per channel, as bits
#pragma unroll
    for (int e = 0; e < 8; ++e) amax[e] = 0u;
    for (int t = t_start + row; t < t_end; t += 16) {
        float xf[8];
        f16x8_to_f32(load16(x + (base + t) * 128 + 8 * c), xf);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax[e] = max(amax[e], abs_bits(xf[e]));
    }

    __shared__ uint32_t s_max[16][128];
    __shared__ float s_scale[128];
#pragma unroll
    for (int e = 0; e < 8; ++e) s_max[row][8 * c + e] = amax[e];
    __syncthreads();
    if (threadIdx.x < 128) {
        uint32_t m = 0u;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = max(m, s_max[r][threadIdx.x]);
        const float sc = sym_scale(m, 7.0f);
        s_scale[threadIdx.x] = sc;
        scale[sslot * 128 + threadIdx.x] = f2h_bits(sc);
    }
    __syncthreads();

    float sv[8], rcp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        sv[e] = s_scale[8 * c + e];
        rcp[e] = recip_approx(sv[e]);
    }
    for (int t = t_start + row; t < t_end; t += 16) {
        float xf[8];
        f16x8_to_f32(load16(x + (base + t) * 128 + 8 * c), xf);
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= (uint32_t)(sym_code(xf[e], sv[e], rcp[e], 7) & 0xF) << (4 * e);
        *reinterpret_cast<uint32_t*>(q + (qbase + t) * 64 + 4 * c) = w;
    }
}

int launch_quantize_per_token(const void* x, void* q, void* scale, int rows, int n_tok,
                              int src_len, int dst_len, int dst_off, int qmax, bool pack4,
                              hipStream_t stream) {
    const long total = (long)rows * n_tok;
    if (total == 0) return LLMIK_OK;
    if (total > 0x7FFFFFFFL) return set_error(LLMIK_ERR_UNSUPPORTED, "too many tokens");
    const long rows_per_wg = (kWriterThreads / 8) * kTokensPerRow8;
    const long grid = (total + rows_per_wg - 1) / rows_per_wg;
    const TokenMap map{(uint32_t)n_tok, (uint32_t)src_len, (uint32_t)dst_len, (uint32_t)dst_off};
    auto xp = static_cast<const uint16_t*>(x);
    auto qp = static_cast<int8_t*>(q);
    auto sp = static_cast<uint16_t*>(scale);
    const bool mapped = !(src_len == n_tok && dst_len == n_tok && dst_off == 0);
    const dim3 g((unsigned)grid), b(kWriterThreads);
    if (qmax == 127 && !pack4) {
        if (mapped) hipLaunchKernelGGL((quantize_per_token_kernel<127, false, true>), g, b, 0, stream, xp, qp, sp, total, map);
        else hipLaunchKernelGGL((quantize_per_token_kernel<127, false, false>), g, b, 0, stream, xp, qp, sp, total, map);
    } else if (qmax == 7 && pack4) {
        if (mapped) hipLaunchKernelGGL((quantize_per_token_kernel<7, true, true>), g, b, 0, stream, xp, qp, sp, total, map);
        else hipLaunchKernelGGL((quantize_per_token_kernel<7, true, false>), g, b, 0, stream, xp, qp, sp, total, map);
    } else {
        return set_error(LLMIK_ERR_UNSUPPORTED, "unsupported per-token quantiser variant");
    }
    return check_launch();
}

int launch_quantize_k_groupwise_int4(const void* x, void* q, void* scale, int rows, int n_tok,
                                     int src_len, int dst_len, int dst_off, int dst_groups,
                                     int group_size, hipStream_t stream) {
    if (n_tok == 0 || rows == 0) return LLMIK_OK;
    if (rows > 65535) return set_error(LLMIK_ERR_UNSUPPORTED, "batch * n_kv_heads exceeds 65535");
    const int n_groups = (n_tok + group_size - 1) / group_size;
    const dim3 grid(n_groups, (unsigned)rows), blk(kWriterThreads);
    const TokenMap map{(uint32_t)n_tok, (uint32_t)src_len, (uint32_t)dst_len, (uint32_t)dst_off};
    auto xp = static_cast<const uint16_t*>(x);
    auto qp = static_cast<int8_t*>(q);
    auto sp = static_cast<uint16_t*>(scale);
    if (group_size <= 16)
        hipLaunchKernelGGL(quantize_k_groupwise_int4_kernel<1>, grid, blk, 0, stream, xp, qp, sp, group_size, map, dst_groups);
    else if (group_size <= 32)
        hipLaunchKernelGGL(quantize_k_groupwise_int4_kernel<2>, grid, blk, 0, stream, xp, qp, sp, group_size, map, dst_groups);
    else if (group_size <= 64)
        hipLaunchKernelGGL(quantize_k_groupwise_int4_kernel<4>, grid, blk, 0, stream, xp, qp, sp, group_size, map, dst_groups);
    else if (group_size <= 128)
        hipLaunchKernelGGL(quantize_k_groupwise_int4_kernel<8>, grid, blk, 0, stream, xp, qp, sp, group_size, map, dst_groups);
    else
        hipLaunchKernelGGL(quantize_k_groupwise_int4_large_kernel, grid, blk, 0, stream, xp, qp, sp, group_size, map, dst_groups);
    return check_launch();
}

// One decode-step token appended to a KIVI INT4 cache in one launch, per
// (batch, kv_head) row (one workgroup each; the three launches of the
// general path, integration/kv_int4_cache.py:104-144 restated in place):
//   * V: the token quantised per token into v_q / v_scale at position pos;
//   * K: the token written after the open group's r fp16 tokens (k_open),
//     and the open group (tokens pos - r .. pos) re-quantised per channel
//     into its codes and its scale slot (pos - r) / group_size.
// The arithmetic is the per-token and group-wise writers' above, so the
// stored codes and scales are the same bits. group_size <= 16 * TPR.
template <int TPR>
__global__ __launch_bounds__(kWriterThreads) void kivi_append_token_kernel(
    const uint16_t* __restrict__ k_in, long k_stride, const uint16_t* __restrict__ v_in, long v_stride,
    uint16_t* __restrict__ k_open, int8_t* __restrict__ k_q, uint16_t* __restrict__ k_scale,
    int8_t* __restrict__ v_q, uint16_t* __restrict__ v_scale, int r, int pos, int group_size,
    int max_len, int n_groups) {
    const long bh = blockIdx.x;
    const int row = threadIdx.x >> 4;
    const int c = threadIdx.x & 15;
    const uint16_t* kin = k_in + bh * k_stride + 8 * c;
    uint16_t* kopen = k_open + bh * (long)group_size * 128 + 8 * c;

    // ---- K: tokens 0..r of the open group (r from k_in, the rest from k_open)
    const u32x4 knew = load16(kin);
    u32x4 raw[TPR];
#pragma unroll
    for (int i = 0; i < TPR; ++i) {
        const int t = min(row + 16 * i, r);   // past the group: a duplicate, which does not move the max
        raw[i] = (t == r) ? knew : load16(kopen + (long)t * 128);
    }
    if (row == (r & 15)) *reinterpret_cast<u32x4*>(kopen + (long)r * 128) = knew;

    uint32_t amax[8];   // NaN-propagating absmax per channel, as bits
#pragma unroll
    for (int e = 0; e < 8; ++e) amax[e] = 0u;
#pragma unroll
    for (int i = 0; i < TPR; ++i) {
        float xf[8];
        f16x8_to_f32(raw[i], xf);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax[e] = max(amax[e], abs_bits(xf[e]));
    }
    __shared__ uint32_t s_max[16][128];
    __shared__ float s_scale[128];
#pragma unroll
    for (int e = 0; e < 8; ++e) s_max[row][8 * c + e] = amax[e];
    __syncthreads();
    const int start = pos - r;
    if (threadIdx.x < 128) {
        uint32_t m = 0u;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) m = max(m, s_max[rr][threadIdx.x]);
        const float sc = sym_scale(m, 7.0f);
        s_scale[threadIdx.x] = sc;
        k_scale[(bh * n_groups + start / group_size) * 128 + threadIdx.x] = f2h_bits(sc);
    }
    __syncthreads();
    float sv[8], rcp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        sv[e] = s_scale[8 * c + e];
        rcp[e] = recip_approx(sv[e]);
    }
#pragma unroll
    for (int i = 0; i < TPR; ++i) {
        const int t = row + 16 * i;
        float xf[8];
        f16x8_to_f32(raw[i], xf);
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= (uint32_t)(sym_code(xf[e], sv[e], rcp[e], 7) & 0xF) << (4 * e);
        if (t <= r) *reinterpret_cast<uint32_t*>(k_q + (bh * max_len + start + t) * 64 + 4 * c) = w;
    }

    // ---- V: the token per token (row 0's 16 lanes)
    if (row == 0) {
        float xf[8];
        f16x8_to_f32(load16(v_in + bh * v_stride + 8 * c), xf);
        uint32_t amax1 = 0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax1 = max(amax1, abs_bits(xf[e]));
        amax1 = row16_umax(amax1);
        const float sc = sym_scale(amax1, 7.0f);
        const float rc = recip_approx(sc);
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= (uint32_t)(sym_code(xf[e], sc, rc, 7) & 0xF) << (4 * e);
        *reinterpret_cast<uint32_t*>(v_q + (bh * max_len + pos) * 64 + 4 * c) = w;
        if (c == 0) v_scale[bh * max_len + pos] = f2h_bits(sc);
    }
}

int launch_kivi_append_token(const void* k, long k_stride, const void* v, long v_stride, void* k_open,
                             void* k_q, void* k_scale, void* v_q, void* v_scale, int rows, int r,
                             int pos, int group_size, int max_len, int n_groups, hipStream_t stream) {
    if (rows == 0) return LLMIK_OK;
    const int tpr = (group_size + 15) / 16;
    auto go = [&](auto tag) {
        constexpr int T = decltype(tag)::value;
        hipLaunchKernelGGL((kivi_append_token_kernel<T>), dim3(rows), dim3(kWriterThreads), 0, stream,
                           static_cast<const uint16_t*>(k), k_stride, static_cast<const uint16_t*>(v),
                           v_stride, static_cast<uint16_t*>(k_open), static_cast<int8_t*>(k_q),
                           static_cast<uint16_t*>(k_scale), static_cast<int8_t*>(v_q),
                           static_cast<uint16_t*>(v_scale), r, pos, group_size, max_len, n_groups);
    };
    if (tpr <= 1) go(std::integral_constant<int, 1>{});
    else if (tpr <= 2) go(std::integral_constant<int, 2>{});
    else if (tpr <= 4) go(std::integral_constant<int, 4>{});
    else go(std::integral_constant<int, 8>{});
    return check_launch();
}

}  // namespace llmik
