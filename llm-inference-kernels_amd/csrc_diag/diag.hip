// Measurement kernels: the floors that the product kernels' rooflines are
// read against. None has a counterpart in the reference; bench.py's
// --floors mode and the profile summaries that quote these floors run them.
// They are built into libllmik_diag.so (include/llmik_diag.h), apart from
// the product library, and keep their own last-error text.
//
// diag_empty_kernel: a launch that does nothing, the per-dispatch cost of a
// kernel of the same workgroup size.
//
// diag_read_kernel<L>: the plainest fast read this library knows how to
// issue. Each wave reads L KiB contiguous per iteration (L 16-byte buffer
// loads per lane, all issued before any is used, with the non-temporal
// hint), waves take L KiB units round robin over the grid, and the loaded
// words are folded with xor so that the loads cannot be dropped. One 32-bit
// value per wave is written: the xor of every word the wave read.
//
// diag_read_write_kernel<L, W>: the same read with a write stream of W bytes
// per 16 bytes read beside it (the KV writers' shape).
#include <cstdio>
#include <type_traits>

#include "../../include/llmik_diag.h"
#include "../csrc/device_common.hpp"

namespace llmik {
namespace {

thread_local char g_diag_error[256] = "";

int set_error(int code, const char* msg) {
    std::snprintf(g_diag_error, sizeof(g_diag_error), "%s", msg);
    return code;
}

int check_launch() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::snprintf(g_diag_error, sizeof(g_diag_error), "HIP launch failed: %s", hipGetErrorString(e));
        return static_cast<int>(e);
    }
    return LLMIK_OK;
}

constexpr int kDiagWaves = 8;
constexpr size_t kDiagMaxBytes = (size_t)3 << 30;   // offsets stay 32-bit

__global__ __launch_bounds__(kDiagWaves * kWave) void diag_empty_kernel() {}

template <int L>
__global__ __launch_bounds__(kDiagWaves * kWave) void diag_read_kernel(const void* src, uint32_t bytes,
                                                                         uint32_t* sink) {
    constexpr uint32_t kUnit = kWave * 16u * L;   // bytes per wave per iteration
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t gw = blockIdx.x * kDiagWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n_waves = gridDim.x * kDiagWaves;
    // Loads past `bytes` read zeros (buffer bound), which leave the xor unchanged.
    const __amdgpu_buffer_rsrc_t r = make_buffer_rsrc(src, bytes);
    const uint32_t n_units = (bytes + kUnit - 1) / kUnit;
    uint32_t x = 0;
    for (uint32_t u = gw; u < n_units; u += n_waves) {
        u32x4 v[L];
#pragma unroll
        for (int i = 0; i < L; ++i)
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(lane * 16u),
                                                         (int)(u * kUnit + (uint32_t)i * 1024u), 2);
#pragma unroll
        for (int i = 0; i < L; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o);
    if (lane == 0) sink[gw] = x;
}

// diag_read_write_kernel<L, W>: the read of diag_read_kernel<L> with a
// write stream beside it, the shape of the KV writers (each 16 bytes read
// give W bytes written: 8 for INT8 codes of fp16 input, 4 for packed INT4).
// For every 16-byte chunk j read, bytes [j*W, j*W + W) of dst receive the
// chunk's first W bytes, with non-temporal stores; the writes of a wave are
// contiguous, like the reads.
template <int L, int W>
__global__ __launch_bounds__(kDiagWaves * kWave) void diag_read_write_kernel(const void* src, uint32_t bytes,
                                                                               void* dst) {
    constexpr uint32_t kUnit = kWave * 16u * L;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t gw = blockIdx.x * kDiagWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n_waves = gridDim.x * kDiagWaves;
    const __amdgpu_buffer_rsrc_t r = make_buffer_rsrc(src, bytes);
    const __amdgpu_buffer_rsrc_t w = make_buffer_rsrc(dst, bytes / 16u * W);
    const uint32_t n_units = (bytes + kUnit - 1) / kUnit;
    for (uint32_t u = gw; u < n_units; u += n_waves) {
        u32x4 v[L];
#pragma unroll
        for (int i = 0; i < L; ++i)
            v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(lane * 16u),
                                                         (int)(u * kUnit + (uint32_t)i * 1024u), 2);
#pragma unroll
        for (int i = 0; i < L; ++i) {
            // Stores past the destination's end are dropped by the buffer bound.
            const uint32_t off = (u * kUnit + (uint32_t)i * 1024u) / 16u * W;
            if constexpr (W == 16)
                __builtin_amdgcn_raw_buffer_store_b128(v[i], w, (int)(lane * 16u), (int)off, 2);
            else if constexpr (W == 8)
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{v[i][0], v[i][1]}, w, (int)(lane * 8u), (int)off, 2);
            else
                __builtin_amdgcn_raw_buffer_store_b32(v[i][0], w, (int)(lane * 4u), (int)off, 2);
        }
    }
}

}  // namespace
}  // namespace llmik

extern "C" {

LLMIK_API const char* llmik_diag_last_error(void) { return llmik::g_diag_error; }

LLMIK_API llmik_status llmik_diag_empty(int n_workgroups, void* stream) {
    if (n_workgroups <= 0) return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_empty: n_workgroups must be > 0");
    hipLaunchKernelGGL(llmik::diag_empty_kernel, dim3((unsigned)n_workgroups),
                       dim3(llmik::kDiagWaves * llmik::kWave), 0, static_cast<hipStream_t>(stream));
    return llmik::check_launch();
}

LLMIK_API llmik_status llmik_diag_read(const void* src, size_t bytes, void* sink, int n_workgroups,
                                       int loads_per_lane, void* stream) {
    if (n_workgroups <= 0) return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read: n_workgroups must be > 0");
    if (bytes % 16 != 0 || bytes > llmik::kDiagMaxBytes)
        return llmik::set_error(LLMIK_ERR_INVALID,
                                "llmik_diag_read: bytes must be a multiple of 16 and at most 3 GiB");
    if (loads_per_lane != 4 && loads_per_lane != 8 && loads_per_lane != 16)
        return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read: loads_per_lane must be 4, 8 or 16");
    if (src == nullptr || sink == nullptr)
        return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read: null pointer");
    if (reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(sink) % 4 != 0)
        return llmik::set_error(LLMIK_ERR_ALIGNMENT,
                                "llmik_diag_read: src must be 16-byte and sink 4-byte aligned");
    const dim3 grid((unsigned)n_workgroups), block(llmik::kDiagWaves * llmik::kWave);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t* out = static_cast<uint32_t*>(sink);
    if (loads_per_lane == 4)
        hipLaunchKernelGGL(llmik::diag_read_kernel<4>, grid, block, 0, st, src, (uint32_t)bytes, out);
    else if (loads_per_lane == 8)
        hipLaunchKernelGGL(llmik::diag_read_kernel<8>, grid, block, 0, st, src, (uint32_t)bytes, out);
    else
        hipLaunchKernelGGL(llmik::diag_read_kernel<16>, grid, block, 0, st, src, (uint32_t)bytes, out);
    return llmik::check_launch();
}

LLMIK_API llmik_status llmik_diag_read_write(const void* src, size_t bytes, void* dst, int write_bytes_per_16,
                                             int n_workgroups, int loads_per_lane, void* stream) {
    if (n_workgroups <= 0)
        return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read_write: n_workgroups must be > 0");
    if (bytes % 16 != 0 || bytes > llmik::kDiagMaxBytes)
        return llmik::set_error(LLMIK_ERR_INVALID,
                                "llmik_diag_read_write: bytes must be a multiple of 16 and at most 3 GiB");
    if (loads_per_lane != 4 && loads_per_lane != 8)
        return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read_write: loads_per_lane must be 4 or 8");
    if (write_bytes_per_16 != 4 && write_bytes_per_16 != 8 && write_bytes_per_16 != 16)
        return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read_write: write_bytes_per_16 must be 4, 8 or 16");
    if (src == nullptr || dst == nullptr)
        return llmik::set_error(LLMIK_ERR_INVALID, "llmik_diag_read_write: null pointer");
    if (reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
        return llmik::set_error(LLMIK_ERR_ALIGNMENT, "llmik_diag_read_write: src and dst must be 16-byte aligned");
    const dim3 grid((unsigned)n_workgroups), block(llmik::kDiagWaves * llmik::kWave);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t n = (uint32_t)bytes;
    auto go = [&](auto l_tag, auto w_tag) {
        constexpr int Lc = decltype(l_tag)::value;
        constexpr int Wc = decltype(w_tag)::value;
        hipLaunchKernelGGL((llmik::diag_read_write_kernel<Lc, Wc>), grid, block, 0, st, src, n, dst);
    };
    auto by_w = [&](auto l_tag) {
        if (write_bytes_per_16 == 4) go(l_tag, std::integral_constant<int, 4>{});
        else if (write_bytes_per_16 == 8) go(l_tag, std::integral_constant<int, 8>{});
        else go(l_tag, std::integral_constant<int, 16>{});
    };
    if (loads_per_lane == 4) by_w(std::integral_constant<int, 4>{});
    else by_w(std::integral_constant<int, 8>{});
    return llmik::check_launch();
}

}  // extern "C"
