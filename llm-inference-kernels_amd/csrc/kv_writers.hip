// Quantize-on-append KV-cache writers for gfx950, bit-exact with
// reference/kv_cache_ref.py applied to x.float():
//   scale = max(absmax / qmax, 1e-8)            (fp32, IEEE division)
//   q     = clamp(round_half_even(x / scale), -qmax, qmax)
//   scale stored as fp16 (round to nearest even)
// (kv_cache_ref.py:46-62 per token, :73-112 per channel groupwise.)
// The reference CUDA writers multiply by an approximate reciprocal under
// fast-math (kernels/kv_cache/kv_compress.cu:50-58,128-129,200-201) and are
// only within +-1 code of the oracle; these kernels divide exactly.
//
// Layouts:
//   x     [rows, 128] fp16 (rows = batch * n_kv_heads * seqlen)
//   int8  [rows, 128] int8, scale [rows] fp16
//   int4  [rows, 64] packed (channel 2i -> low nibble of byte i), scale as above
//   K groupwise int4: scale [batch, n_kv_heads, n_groups, 128] fp16
#include "device_common.hpp"
#include "llmik_internal.hpp"

namespace llmik {

constexpr int kWriterThreads = 256;   // 16 token rows of 16 lanes

// One DPP row (16 lanes) per token: lane c owns channels 8c..8c+7.
template <int QMAX, bool PACK4>
__global__ __launch_bounds__(kWriterThreads) void quantize_per_token_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, uint16_t* __restrict__ scale,
    long rows) {
    const long row = (long)blockIdx.x * (kWriterThreads / 16) + (threadIdx.x >> 4);
    const int c = threadIdx.x & 15;
    // Rows past the end still take part in the DPP reduction (on a clamped,
    // in-bounds row) but store nothing.
    const long r = row < rows ? row : rows - 1;

    float xf[8];
    f16x8_to_f32(load16(x + r * 128 + 8 * c), xf);
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(xf[e]));
    amax = row16_max(amax);

    const float s = fmaxf(amax / (float)QMAX, 1.0e-8f);
    const float rcp = 1.0f / s;
    int code[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float v = quant_round(xf[e], s, rcp);
        v = fminf(fmaxf(v, -(float)QMAX), (float)QMAX);
        code[e] = (int)v;
    }
    if (row >= rows) return;

    if constexpr (PACK4) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= (uint32_t)(code[e] & 0xF) << (4 * e);
        *reinterpret_cast<uint32_t*>(q + row * 64 + 4 * c) = w;
    } else {
        u32x2 w;
        w[0] = (uint32_t)(code[0] & 0xFF) | ((uint32_t)(code[1] & 0xFF) << 8) |
               ((uint32_t)(code[2] & 0xFF) << 16) | ((uint32_t)(code[3] & 0xFF) << 24);
        w[1] = (uint32_t)(code[4] & 0xFF) | ((uint32_t)(code[5] & 0xFF) << 8) |
               ((uint32_t)(code[6] & 0xFF) << 16) | ((uint32_t)(code[7] & 0xFF) << 24);
        *reinterpret_cast<u32x2*>(q + row * 128 + 8 * c) = w;
    }
    if (c == 0) scale[row] = f2h_bits(s);
}

// One workgroup per (batch, kv_head, group). 16 rows of 16 lanes: row r
// walks the group's tokens r, r+16, ...; lane c owns channels 8c..8c+7.
// Pass 1 takes the per-channel absmax (rows merged in LDS), pass 2
// re-reads the (cache-resident) group and writes packed codes.
__global__ __launch_bounds__(kWriterThreads) void quantize_k_groupwise_int4_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q, uint16_t* __restrict__ scale,
    int seqlen, int group_size, int n_groups) {
    const int g = blockIdx.x;
    const long bh = blockIdx.y;   // batch * n_kv_heads + kv_head
    const int row = threadIdx.x >> 4;
    const int c = threadIdx.x & 15;
    const int t_start = g * group_size;
    const int t_end = min(t_start + group_size, seqlen);
    const long base = bh * seqlen;

    float amax[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) amax[e] = 0.0f;
    for (int t = t_start + row; t < t_end; t += 16) {
        float xf[8];
        f16x8_to_f32(load16(x + (base + t) * 128 + 8 * c), xf);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax[e] = fmaxf(amax[e], fabsf(xf[e]));
    }

    __shared__ float s_max[16][128];
    __shared__ float s_scale[128];
#pragma unroll
    for (int e = 0; e < 8; ++e) s_max[row][8 * c + e] = amax[e];
    __syncthreads();
    if (threadIdx.x < 128) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, s_max[r][threadIdx.x]);
        const float s = fmaxf(m / 7.0f, 1.0e-8f);
        s_scale[threadIdx.x] = s;
        scale[(bh * n_groups + g) * 128 + threadIdx.x] = f2h_bits(s);
    }
    __syncthreads();

    float s[8], rcp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        s[e] = s_scale[8 * c + e];
        rcp[e] = 1.0f / s[e];
    }
    for (int t = t_start + row; t < t_end; t += 16) {
        float xf[8];
        f16x8_to_f32(load16(x + (base + t) * 128 + 8 * c), xf);
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = quant_round(xf[e], s[e], rcp[e]);
            v = fminf(fmaxf(v, -7.0f), 7.0f);
            w |= (uint32_t)((int)v & 0xF) << (4 * e);
        }
        *reinterpret_cast<uint32_t*>(q + (base + t) * 64 + 4 * c) = w;
    }
}

int launch_quantize_per_token(const void* x, void* q, void* scale, long rows, int qmax,
                              bool pack4, hipStream_t stream) {
    if (rows == 0) return LLMIK_OK;
    const long rows_per_wg = kWriterThreads / 16;
    const long grid = (rows + rows_per_wg - 1) / rows_per_wg;
    if (grid > 0x7FFFFFFFL) return set_error(LLMIK_ERR_UNSUPPORTED, "too many token rows");
    auto xp = static_cast<const uint16_t*>(x);
    auto qp = static_cast<int8_t*>(q);
    auto sp = static_cast<uint16_t*>(scale);
    if (qmax == 127 && !pack4) {
        hipLaunchKernelGGL((quantize_per_token_kernel<127, false>), dim3((unsigned)grid),
                           dim3(kWriterThreads), 0, stream, xp, qp, sp, rows);
    } else if (qmax == 7 && pack4) {
        hipLaunchKernelGGL((quantize_per_token_kernel<7, true>), dim3((unsigned)grid),
                           dim3(kWriterThreads), 0, stream, xp, qp, sp, rows);
    } else {
        return set_error(LLMIK_ERR_UNSUPPORTED, "unsupported per-token quantiser variant");
    }
    return check_launch();
}

int launch_quantize_k_groupwise_int4(const void* x, void* q, void* scale, int batch,
                                     int n_kv_heads, int seqlen, int group_size,
                                     hipStream_t stream) {
    if (seqlen == 0 || batch == 0 || n_kv_heads == 0) return LLMIK_OK;
    const int n_groups = (seqlen + group_size - 1) / group_size;
    const long bh = (long)batch * n_kv_heads;
    if (bh > 65535L) return set_error(LLMIK_ERR_UNSUPPORTED, "batch * n_kv_heads exceeds 65535");
    hipLaunchKernelGGL(quantize_k_groupwise_int4_kernel, dim3(n_groups, (unsigned)bh),
                       dim3(kWriterThreads), 0, stream, static_cast<const uint16_t*>(x),
                       static_cast<int8_t*>(q), static_cast<uint16_t*>(scale), seqlen,
                       group_size, n_groups);
    return check_launch();
}

}  // namespace llmik
