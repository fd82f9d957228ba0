// Symmetric INT4 group-wise weight quantisation and INT4 packing along K,
// on the GPU, bit-exact to the reference's host-side torch path
// (reference/quant_matmul_ref.py:39-88 and :140-165, called by
// integration/w4a16_patch.py:78-84 and tests/test_quant.py:265-267):
//
//   scale[g, n] = max(absmax_{k in group g} |W[k, n]| / 7, 1e-8)  in W's dtype
//   q[k, n]     = clamp(rint(fp32(W[k, n]) / fp32(scale[k / g, n])), -7, 7)
//   packed[kp, n] bits 4i..4i+3 = q[8 kp + i, n] (two's complement nibble)
//
// dtype semantics, as torch evaluates them:
//   * fp16 W: absmax / 7 is an fp32 quotient rounded to fp16, and the 1e-8
//     floor is fp16(1e-8) = 0; fp32 W: fp32 quotient, floor 1e-8f;
//   * the code is rint of the IEEE fp32 quotient (correctly rounded; formed
//     as x * (1 / s) with the true division near half-integers, quant_round),
//     rint is round-half-to-even, and a NaN quotient (0 / 0 of an all-zero
//     fp16 group) becomes code 0;
//   * a short last group (K % g != 0) uses only its real rows: the
//     reference's zero padding never raises an absmax.
// With group_size % 8 == 0 (up to 1024) and K % 8 == 0 one workgroup codes
// one group of 64 columns in a single pass (quantize_w4_tile_kernel);
// otherwise one thread owns one (group, column): a first pass over the
// group's rows takes the absmax, a second (L2-hot) pass writes the codes.
#include <type_traits>

#include "device_common.hpp"
#include "llmik_internal.hpp"

namespace llmik {

constexpr int kQuantThreads = 256;

template <bool F16>
__device__ __forceinline__ float w_at(const void* W, long idx) {
    if constexpr (F16) return h2f(static_cast<const uint16_t*>(W)[idx]);
    else return static_cast<const float*>(W)[idx];
}

template <bool F16>
__global__ __launch_bounds__(kQuantThreads) void quantize_w4_kernel(
    const void* __restrict__ W, int K, int N, int group_size, int8_t* __restrict__ q,
    uint32_t* __restrict__ packed, void* __restrict__ scale, uint16_t* __restrict__ scale_f16) {
    const int n = blockIdx.x * kQuantThreads + threadIdx.x;
    const int g = blockIdx.y;
    if (n >= N) return;
    const int k0 = g * group_size;
    const int k1 = min(k0 + group_size, K);

    float amax = 0.0f;
    bool nan = false;
    for (int k = k0; k < k1; ++k) {
        const float x = w_at<F16>(W, (long)k * N + n);
        nan |= (x != x);
        amax = fmaxf(amax, fabsf(x));
    }
    if (nan) amax = __builtin_nanf("");   // torch's amax propagates NaN

    float s;
    uint16_t s16;
    if constexpr (F16) {
        // fp16 / 7: fp32 quotient rounded to fp16; clamp(min=fp16(1e-8) = 0).
        s16 = f2h_bits(amax / 7.0f);
        s = h2f(s16);
        if (s < 0.0f) { s = 0.0f; s16 = 0; }
        if (scale) static_cast<uint16_t*>(scale)[(long)g * N + n] = s16;
    } else {
        s = amax / 7.0f;
        if (s < 1e-8f) s = 1e-8f;   // NaN stays NaN, as clamp keeps it
        s16 = f2h_bits(s);
        if (scale) static_cast<float*>(scale)[(long)g * N + n] = s;
    }
    if (scale_f16) scale_f16[(long)g * N + n] = s16;

    uint32_t word = 0;
    const float r = recip_approx(s);
    for (int k = k0; k < k1; ++k) {
        const float x = w_at<F16>(W, (long)k * N + n);
        float c = quant_round(x, s, r);
        if (c != c) c = 0.0f;   // a NaN quotient (0 / 0, or a NaN weight or scale) -> code 0
        c = fminf(fmaxf(c, -7.0f), 7.0f);
        const int code = (int)c;
        if (q) q[(long)k * N + n] = (int8_t)code;
        if (packed) {
            word |= ((uint32_t)code & 0xFu) << (4 * (k & 7));
            if ((k & 7) == 7) {
                packed[(long)(k >> 3) * N + n] = word;
                word = 0;
            }
        }
    }
}

// One pass for group_size % 8 == 0 and K % 8 == 0: a workgroup of 16
// waves owns one scale group of 64 columns. Lane c is column n0 + c (so
// every load and store instruction is 64 consecutive elements), and wave s
// holds the 8-row slabs s, s + 16, ... of the group (SP of them) in
// registers. The column absmax meets through LDS; every thread then codes
// its slabs and writes one packed word (and the int8 codes) per slab.
constexpr int kTileWaves = 16;

template <bool F16, int SP>
__global__ __launch_bounds__(kTileWaves * kWave) void quantize_w4_tile_kernel(
    const void* __restrict__ W, int K, int N, int group_size, int8_t* __restrict__ q,
    uint32_t* __restrict__ packed, void* __restrict__ scale, uint16_t* __restrict__ scale_f16) {
    __shared__ float s_max[kTileWaves][kWave];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = blockIdx.x * kWave + lane;
    const int g = blockIdx.y;
    const int k0 = g * group_size;
    const int k1 = min(k0 + group_size, K);
    const int nslab = (k1 - k0) / 8;
    const bool col_ok = n < N;

    float x[SP][8];
    float amax = 0.0f;
    bool nan = false;
#pragma unroll
    for (int j = 0; j < SP; ++j) {
        const int sl = wave + kTileWaves * j;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[j][i] = (col_ok && sl < nslab) ? w_at<F16>(W, (long)(k0 + 8 * sl + i) * N + n) : 0.0f;
            nan |= (x[j][i] != x[j][i]);
            amax = fmaxf(amax, fabsf(x[j][i]));
        }
    }
    s_max[wave][lane] = nan ? __builtin_nanf("") : amax;
    __syncthreads();
    amax = 0.0f;
    nan = false;
#pragma unroll
    for (int w = 0; w < kTileWaves; ++w) {
        const float v = s_max[w][lane];
        nan |= (v != v);
        amax = fmaxf(amax, v);
    }
    if (nan) amax = __builtin_nanf("");   // torch's amax propagates NaN
    if (!col_ok) return;

    float s;
    uint16_t s16;
    if constexpr (F16) {
        s16 = f2h_bits(amax / 7.0f);   // fp32 quotient rounded to fp16; the fp16 floor is 0
        s = h2f(s16);
    } else {
        s = amax / 7.0f;
        if (s < 1e-8f) s = 1e-8f;      // NaN stays NaN, as clamp keeps it
        s16 = f2h_bits(s);
    }
    if (wave == 0) {
        if (scale) {
            if constexpr (F16) static_cast<uint16_t*>(scale)[(long)g * N + n] = s16;
            else static_cast<float*>(scale)[(long)g * N + n] = s;
        }
        if (scale_f16) scale_f16[(long)g * N + n] = s16;
    }
    const float r = recip_approx(s);
#pragma unroll
    for (int j = 0; j < SP; ++j) {
        const int sl = wave + kTileWaves * j;
        if (sl >= nslab) break;
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float c = quant_round(x[j][i], s, r);
            if (c != c) c = 0.0f;   // a NaN quotient -> code 0
            c = fminf(fmaxf(c, -7.0f), 7.0f);
            const int code = (int)c;
            if (q) q[(long)(k0 + 8 * sl + i) * N + n] = (int8_t)code;
            word |= ((uint32_t)code & 0xFu) << (4 * i);
        }
        if (packed) packed[(long)(k0 / 8 + sl) * N + n] = word;
    }
}

__global__ __launch_bounds__(kQuantThreads) void pack_int4_kernel(const int8_t* __restrict__ q,
                                                                  int N, long total,
                                                                  uint32_t* __restrict__ packed) {
    const long i = (long)blockIdx.x * kQuantThreads + threadIdx.x;   // over [K/8, N]
    if (i >= total) return;
    const long kp = i / N;
    const int n = (int)(i % N);
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        word |= ((uint32_t)(int)q[(8 * kp + j) * N + n] & 0xFu) << (4 * j);
    packed[i] = word;
}

int launch_quantize_weights_int4(const void* W, bool w_fp16, int K, int N, int group_size, void* q,
                                 void* packed, void* scale, void* scale_f16, hipStream_t stream) {
    if (K == 0 || N == 0) return LLMIK_OK;
    const int n_groups = (K + group_size - 1) / group_size;
    if (n_groups > 65535) return set_error(LLMIK_ERR_UNSUPPORTED, "too many scale groups (> 65535)");
    if (group_size % 8 == 0 && K % 8 == 0 && group_size <= 8 * kTileWaves * 8) {
        const int slabs = group_size / 8;
        const int sp = (slabs + kTileWaves - 1) / kTileWaves;   // 1, 2, 4 or 8 (group <= 1024)
        const dim3 grid((N + kWave - 1) / kWave, n_groups), blk(kTileWaves * kWave);
        auto go = [&](auto f16_tag, auto sp_tag) {
            constexpr bool F = decltype(f16_tag)::value;
            constexpr int P = decltype(sp_tag)::value;
            hipLaunchKernelGGL((quantize_w4_tile_kernel<F, P>), grid, blk, 0, stream, W, K, N, group_size,
                               static_cast<int8_t*>(q), static_cast<uint32_t*>(packed), scale,
                               static_cast<uint16_t*>(scale_f16));
        };
        auto by_sp = [&](auto f16_tag) {
            if (sp <= 1) go(f16_tag, std::integral_constant<int, 1>{});
            else if (sp <= 2) go(f16_tag, std::integral_constant<int, 2>{});
            else if (sp <= 4) go(f16_tag, std::integral_constant<int, 4>{});
            else go(f16_tag, std::integral_constant<int, 8>{});
        };
        if (w_fp16) by_sp(std::true_type{});
        else by_sp(std::false_type{});
        return check_launch();
    }
    const dim3 grid((N + kQuantThreads - 1) / kQuantThreads, n_groups);
    if (w_fp16) {
        hipLaunchKernelGGL(quantize_w4_kernel<true>, grid, dim3(kQuantThreads), 0, stream, W, K, N,
                           group_size, static_cast<int8_t*>(q), static_cast<uint32_t*>(packed),
                           scale, static_cast<uint16_t*>(scale_f16));
    } else {
        hipLaunchKernelGGL(quantize_w4_kernel<false>, grid, dim3(kQuantThreads), 0, stream, W, K, N,
                           group_size, static_cast<int8_t*>(q), static_cast<uint32_t*>(packed),
                           scale, static_cast<uint16_t*>(scale_f16));
    }
    return check_launch();
}

int launch_pack_int4_along_k(const void* q, int K, int N, void* packed, hipStream_t stream) {
    const long total = (long)(K / 8) * N;
    if (total == 0) return LLMIK_OK;
    const long blocks = (total + kQuantThreads - 1) / kQuantThreads;
    if (blocks > 0x7FFFFFFFL) return set_error(LLMIK_ERR_UNSUPPORTED, "matrix too large");
    hipLaunchKernelGGL(pack_int4_kernel, dim3((unsigned)blocks), dim3(kQuantThreads), 0, stream,
                       static_cast<const int8_t*>(q), N, total, static_cast<uint32_t*>(packed));
    return check_launch();
}

}  // namespace llmik
