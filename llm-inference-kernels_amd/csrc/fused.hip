// Fused elementwise decode-path ops for gfx950: RMSNorm, SwiGLU, RoPE.
// Semantics follow kernels/fused/fused_ops.cu:31-86 of the reference
// (fp32 math, one fp16 rounding of each output).
#include "device_common.hpp"
#include "llmik_internal.hpp"

namespace llmik {

// One workgroup per row; 16-byte vectors when the row allows it.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      uint16_t* __restrict__ out, int hidden,
                                                      float eps) {
    const long row = blockIdx.x;
    const uint16_t* xr = x + row * hidden;
    uint16_t* orow = out + row * hidden;
    const bool vec = (hidden % 8) == 0;
    float ss = 0.0f;
    if (vec) {
        for (int i = threadIdx.x * 8; i < hidden; i += 256 * 8) {
            float v[8];
            f16x8_to_f32(load16(xr + i), v);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
        }
    } else {
        for (int i = threadIdx.x; i < hidden; i += 256) {
            const float v = h2f(xr[i]);
            ss = fmaf(v, v, ss);
        }
    }
    // wave sum: 16-lane rows, then across the 4 rows via LDS
    ss = row16_sum(ss);
    __shared__ float s_red[16];
    if ((threadIdx.x & 15) == 0) s_red[threadIdx.x >> 4] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) tot += s_red[r];
    const float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
    if (vec) {
        for (int i = threadIdx.x * 8; i < hidden; i += 256 * 8) {
            float v[8], g[8];
            f16x8_to_f32(load16(xr + i), v);
            f16x8_to_f32(load16(w + i), g);
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                o[e] = (uint32_t)f2h_bits(v[2 * e] * inv * g[2 * e]) |
                       ((uint32_t)f2h_bits(v[2 * e + 1] * inv * g[2 * e + 1]) << 16);
            *reinterpret_cast<u32x4*>(orow + i) = o;
        }
    } else {
        for (int i = threadIdx.x; i < hidden; i += 256)
            orow[i] = f2h_bits(h2f(xr[i]) * inv * h2f(w[i]));
    }
}

// Rows of up to 256 * 8 * NV fp16 (hidden % 8 == 0): the row and the weight
// are loaded once into registers, both before the reduction, so the kernel
// waits on memory once instead of twice.
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_regs_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w,
                                                           uint16_t* __restrict__ out, int hidden,
                                                           float eps) {
    const long row = blockIdx.x;
    const uint16_t* xr = x + row * hidden;
    uint16_t* orow = out + row * hidden;
    u32x4 xv[NV], wv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = (threadIdx.x + 256 * k) * 8;
        const bool ok = i < hidden;
        xv[k] = ok ? load16(xr + i) : u32x4{0u, 0u, 0u, 0u};
        wv[k] = ok ? load16(w + i) : u32x4{0u, 0u, 0u, 0u};
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float v[8];
        f16x8_to_f32(xv[k], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = row16_sum(ss);
    __shared__ float s_red[16];
    if ((threadIdx.x & 15) == 0) s_red[threadIdx.x >> 4] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) tot += s_red[r];
    const float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = (threadIdx.x + 256 * k) * 8;
        if (i >= hidden) break;
        float v[8], g[8];
        f16x8_to_f32(xv[k], v);
        f16x8_to_f32(wv[k], g);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)f2h_bits(v[2 * e] * inv * g[2 * e]) |
                   ((uint32_t)f2h_bits(v[2 * e + 1] * inv * g[2 * e + 1]) << 16);
        *reinterpret_cast<u32x4*>(orow + i) = o;
    }
}


__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ g,
                                                       const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ out, long n) {
    const long i8 = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i8 + 8 <= n) {
        float gv[8], uv[8];
        f16x8_to_f32(load16(g + i8), gv);
        f16x8_to_f32(load16(u + i8), uv);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)f2h_bits(silu_mul1(gv[2 * e], uv[2 * e])) |
                   ((uint32_t)f2h_bits(silu_mul1(gv[2 * e + 1], uv[2 * e + 1])) << 16);
        *reinterpret_cast<u32x4*>(out + i8) = o;
    } else {
        for (long i = i8; i < n; ++i) out[i] = f2h_bits(silu_mul1(h2f(g[i]), h2f(u[i])));
    }
}

// One thread per (b, h, s, d) with d < D/2: it produces out[d] and
// out[d + D/2] from the pair (x[d], x[d + D/2]).
__global__ __launch_bounds__(256) void rope_kernel(const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ cs,
                                                   const uint16_t* __restrict__ sn,
                                                   uint16_t* __restrict__ out, int B, int H,
                                                   int S, int D) {
    const int half_d = D / 2;
    const long total = (long)B * H * S * half_d;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int d = (int)(idx % half_d);
    const long bhs = idx / half_d;
    const int s = (int)(bhs % S);
    const int b = (int)(bhs / ((long)S * H));
    const long xrow = bhs * D;
    const long crow = ((long)b * S + s) * D;
    rope_pair(h2f(x[xrow + d]), h2f(x[xrow + d + half_d]), h2f(cs[crow + d]), h2f(sn[crow + d]),
              h2f(cs[crow + d + half_d]), h2f(sn[crow + d + half_d]), out[xrow + d],
              out[xrow + d + half_d]);
}

// ---------------------------------------------------------------- decode step
// Kernels that merge consecutive ops of one decode step; each computes what
// the ops it replaces compute, in the same order, so the results are the
// same bits.

// rope of the q and k heads of a fused q|k|v projection row and the new
// token's K and V written into cache slot `pos`: one thread per (b, head,
// d < D/2) over the H + 2 Hkv heads of qkv [B, H + 2 Hkv, D]. cs / sn are
// the position's [D] row of the rotary tables.
__global__ __launch_bounds__(256) void rope_qkv_append_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ cs, const uint16_t* __restrict__ sn,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kbuf, uint16_t* __restrict__ vbuf, int B, int H,
    int Hkv, int D, int max_len, int pos) {
    const int half_d = D / 2;
    const int NH = H + 2 * Hkv;
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)B * NH * half_d) return;
    const int d = (int)(idx % half_d);
    const long bj = idx / half_d;
    const int j = (int)(bj % NH);
    const int b = (int)(bj / NH);
    const uint16_t* x = qkv + bj * D;
    if (j >= H + Hkv) {
        uint16_t* dst = vbuf + (((long)b * Hkv + (j - H - Hkv)) * max_len + pos) * D;
        dst[d] = x[d];
        dst[d + half_d] = x[d + half_d];
        return;
    }
    uint16_t* dst = j < H ? q_out + ((long)b * H + j) * D
                          : kbuf + (((long)b * Hkv + (j - H)) * max_len + pos) * D;
    rope_pair(h2f(x[d]), h2f(x[d + half_d]), h2f(cs[d]), h2f(sn[d]), h2f(cs[d + half_d]),
              h2f(sn[d + half_d]), dst[d], dst[d + half_d]);
}

// h = fp16(x + r) (torch's fp16 add: fp32 sum, one rounding) and
// out = rmsnorm(h) as rmsnorm_regs_kernel computes it, one workgroup per row,
// hidden % 8 == 0 and hidden <= 256 * 8 * NV.
template <int NV>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ r,
                                                          const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ h_out,
                                                          uint16_t* __restrict__ out, int hidden,
                                                          float eps) {
    const long row = blockIdx.x;
    // Every load is issued before any is used, so the kernel waits on memory
    // once (with the h stores between the loads of two rounds, the compiler
    // waited twice).
    u32x4 xa[NV], ra[NV], hv[NV], wv[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = (threadIdx.x + 256 * k) * 8;
        const bool ok = i < hidden;
        const u32x4 z{0u, 0u, 0u, 0u};
        xa[k] = ok ? load16(x + row * hidden + i) : z;
        ra[k] = ok ? load16(r + row * hidden + i) : z;
        wv[k] = ok ? load16(w + i) : z;
    }
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = (threadIdx.x + 256 * k) * 8;
        const bool ok = i < hidden;
        float a[8], c[8];
        f16x8_to_f32(xa[k], a);
        f16x8_to_f32(ra[k], c);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            hv[k][e] = (uint32_t)f2h_bits(a[2 * e] + c[2 * e]) |
                       ((uint32_t)f2h_bits(a[2 * e + 1] + c[2 * e + 1]) << 16);
        if (ok) *reinterpret_cast<u32x4*>(h_out + row * hidden + i) = hv[k];
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        float v[8];
        f16x8_to_f32(hv[k], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = row16_sum(ss);
    __shared__ float s_red[16];
    if ((threadIdx.x & 15) == 0) s_red[threadIdx.x >> 4] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) tot += s_red[q];
    const float inv = 1.0f / sqrtf(tot / (float)hidden + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = (threadIdx.x + 256 * k) * 8;
        if (i >= hidden) break;
        float v[8], g[8];
        f16x8_to_f32(hv[k], v);
        f16x8_to_f32(wv[k], g);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)f2h_bits(v[2 * e] * inv * g[2 * e]) |
                   ((uint32_t)f2h_bits(v[2 * e + 1] * inv * g[2 * e + 1]) << 16);
        *reinterpret_cast<u32x4*>(out + row * hidden + i) = o;
    }
}

// out[r, c] = silu(gu[r, c]) * gu[r, cols + c] over a fused gate|up
// projection gu [rows, 2 cols], cols % 8 == 0.
__global__ __launch_bounds__(256) void silu_mul_halves_kernel(const uint16_t* __restrict__ gu,
                                                              uint16_t* __restrict__ out, long rows,
                                                              int cols) {
    const long i8 = ((long)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i8 >= rows * cols) return;
    const long row = i8 / cols;
    const int col = (int)(i8 % cols);
    float gv[8], uv[8];
    f16x8_to_f32(load16(gu + row * 2 * cols + col), gv);
    f16x8_to_f32(load16(gu + row * 2 * cols + cols + col), uv);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        o[e] = (uint32_t)f2h_bits(silu_mul1(gv[2 * e], uv[2 * e])) |
               ((uint32_t)f2h_bits(silu_mul1(gv[2 * e + 1], uv[2 * e + 1])) << 16);
    *reinterpret_cast<u32x4*>(out + i8) = o;
}

int launch_rmsnorm(const void* x, const void* w, void* out, int rows, int hidden, float eps,
                   hipStream_t stream) {
    if (rows == 0 || hidden == 0) return LLMIK_OK;
    const uint16_t* xs = static_cast<const uint16_t*>(x);
    const uint16_t* ws = static_cast<const uint16_t*>(w);
    uint16_t* os = static_cast<uint16_t*>(out);
    if (hidden % 8 == 0 && hidden <= 256 * 8 * 4) {
        const int nv = (hidden + 256 * 8 - 1) / (256 * 8);
        if (nv == 1)
            hipLaunchKernelGGL(rmsnorm_regs_kernel<1>, dim3(rows), dim3(256), 0, stream, xs, ws, os, hidden, eps);
        else if (nv == 2)
            hipLaunchKernelGGL(rmsnorm_regs_kernel<2>, dim3(rows), dim3(256), 0, stream, xs, ws, os, hidden, eps);
        else
            hipLaunchKernelGGL(rmsnorm_regs_kernel<4>, dim3(rows), dim3(256), 0, stream, xs, ws, os, hidden, eps);
        return check_launch();
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, stream, xs, ws, os, hidden, eps);
    return check_launch();
}

int launch_silu_mul(const void* g, const void* u, void* out, long n, hipStream_t stream) {
    if (n == 0) return LLMIK_OK;
    const long blocks = (n + 256 * 8 - 1) / (256 * 8);
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
                       static_cast<uint16_t*>(out), n);
    return check_launch();
}

int launch_rope(const void* x, const void* cs, const void* sn, void* out, int B, int H, int S,
                int D, hipStream_t stream) {
    const long total = (long)B * H * S * (D / 2);
    if (total == 0) return LLMIK_OK;
    const long blocks = (total + 255) / 256;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(cs),
                       static_cast<const uint16_t*>(sn), static_cast<uint16_t*>(out), B, H, S, D);
    return check_launch();
}

int launch_rope_qkv_append(const void* qkv, const void* cs, const void* sn, void* q_out, void* kbuf,
                           void* vbuf, int B, int H, int Hkv, int D, int max_len, int pos,
                           hipStream_t stream) {
    const long total = (long)B * (H + 2 * Hkv) * (D / 2);
    if (total == 0) return LLMIK_OK;
    hipLaunchKernelGGL(rope_qkv_append_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(qkv), static_cast<const uint16_t*>(cs),
                       static_cast<const uint16_t*>(sn), static_cast<uint16_t*>(q_out),
                       static_cast<uint16_t*>(kbuf), static_cast<uint16_t*>(vbuf), B, H, Hkv, D, max_len,
                       pos);
    return check_launch();
}

int launch_add_rmsnorm(const void* x, const void* r, const void* w, void* h_out, void* out, int rows,
                       int hidden, float eps, hipStream_t stream) {
    if (rows == 0 || hidden == 0) return LLMIK_OK;
    const uint16_t* xs = static_cast<const uint16_t*>(x);
    const uint16_t* rs = static_cast<const uint16_t*>(r);
    const uint16_t* ws = static_cast<const uint16_t*>(w);
    uint16_t* hs = static_cast<uint16_t*>(h_out);
    uint16_t* os = static_cast<uint16_t*>(out);
    const int nv = (hidden + 256 * 8 - 1) / (256 * 8);
    if (nv == 1)
        hipLaunchKernelGGL(add_rmsnorm_kernel<1>, dim3(rows), dim3(256), 0, stream, xs, rs, ws, hs, os, hidden, eps);
    else if (nv == 2)
        hipLaunchKernelGGL(add_rmsnorm_kernel<2>, dim3(rows), dim3(256), 0, stream, xs, rs, ws, hs, os, hidden, eps);
    else
        hipLaunchKernelGGL(add_rmsnorm_kernel<4>, dim3(rows), dim3(256), 0, stream, xs, rs, ws, hs, os, hidden, eps);
    return check_launch();
}

int launch_silu_mul_halves(const void* gu, void* out, long rows, int cols, hipStream_t stream) {
    const long n = rows * cols;
    if (n == 0) return LLMIK_OK;
    hipLaunchKernelGGL(silu_mul_halves_kernel, dim3((unsigned)((n + 256 * 8 - 1) / (256 * 8))), dim3(256), 0,
                       stream, static_cast<const uint16_t*>(gu), static_cast<uint16_t*>(out), rows, cols);
    return check_launch();
}

}  // namespace llmik
