// Device-side helpers shared by every gfx950 kernel in this library.
//
// Everything here is written for CDNA4 wave64: cross-lane traffic uses DPP
// row operations (a DPP "row" is 16 lanes), vector memory uses 16-byte
// global loads, and fp16 <-> fp32 conversion goes through the hardware
// converters (round-to-nearest-even).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace llmik {

constexpr int kWave = 64;

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---- DPP row (16-lane) reductions -----------------------------------------
// DPP control codes (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), Ctrl, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the result.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<kDppQuadXor1>(v);
    v += dpp_f32<kDppQuadXor2>(v);
    v += dpp_f32<kDppRowHalfMirror>(v);
    v += dpp_f32<kDppRowMirror>(v);
    return v;
}

// Max over the 16 lanes of a DPP row; every lane of the row gets the result.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
    return v;
}

// ---- conversions ----------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t bits) {
    return (float)__builtin_bit_cast(f16, bits);
}

__device__ __forceinline__ uint16_t f2h_bits(float x) {
    return __builtin_bit_cast(uint16_t, (f16)x);  // v_cvt_f16_f32, RNE
}

// Raw buffer resource over `bytes` bytes at `p` (gfx9 data-format word).
// Loads through it take a 32-bit per-lane offset plus a uniform offset, and
// return 0 beyond `bytes`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                             0x00020000);
}

// 4-byte buffer load, non-temporal (streamed once).
__device__ __forceinline__ uint32_t buffer_stream4(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 2);
}

__device__ __forceinline__ u32x4 make_u32x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4 r;
    r[0] = a; r[1] = b; r[2] = c; r[3] = d;
    return r;
}

// A constant materialised in a VGPR (a VALU op can read one scalar
// constant only; a VGPR copy lets three-operand bit ops take two).
__device__ __forceinline__ uint32_t vgpr_const(uint32_t k) {
    uint32_t v;
    asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "i"(k));
    return v;
}

// Byte permute: selector bytes 0-3 pick bytes of `lo`, 4-7 bytes of `hi`,
// 0x0C gives 0x00 (v_perm_b32).
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// NOTE: __builtin_bit_cast applied directly to an ext-vector element
// (`__builtin_bit_cast(f16x2, v[i])`) is miscompiled by this hipcc (every
// element reads as element 0). Always copy the element to a scalar first.
__device__ __forceinline__ f16x2 as_f16x2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }

// Unpack 8 fp16 stored in a 16-byte vector into fp32.
__device__ __forceinline__ void f16x8_to_f32(const u32x4 raw, float out[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = raw[i];
        const f16x2 h = as_f16x2(w);
        out[2 * i] = (float)h[0];
        out[2 * i + 1] = (float)h[1];
    }
}

// 8 signed int8 codes (two dwords, little-endian) -> fp32.
__device__ __forceinline__ void i8x8_to_f32(const u32x2 raw, float out[8]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int32_t w = (int32_t)raw[i];
        out[4 * i + 0] = (float)((w << 24) >> 24);
        out[4 * i + 1] = (float)((w << 16) >> 24);
        out[4 * i + 2] = (float)((w << 8) >> 24);
        out[4 * i + 3] = (float)(w >> 24);
    }
}

// 8 signed 4-bit codes in one dword -> fp32. Nibble i (bits 4i..4i+3) is
// element i, two's complement. This is both the KV-cache byte packing
// (even channel in the low nibble) and the W4 packing along K.
__device__ __forceinline__ void i4x8_to_f32(const uint32_t raw, float out[8]) {
    const int32_t w = (int32_t)raw;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)((w << (28 - 4 * i)) >> 28);
}

// ---- buffer loads ---------------------------------------------------------
__device__ __forceinline__ u32x4 load16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x2 load8(const void* p) {
    return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ uint32_t load4(const void* p) {
    return *reinterpret_cast<const uint32_t*>(p);
}
// Streaming loads for data read exactly once (KV cache, packed weights):
// the non-temporal hint keeps them from displacing reused lines and lifts
// sustained HBM read bandwidth on gfx950 (measured ~5.6 -> ~6.1 TB/s for a
// plain 1 GiB read).
__device__ __forceinline__ u32x4 stream16(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 stream8(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
__device__ __forceinline__ uint32_t stream4(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

// ---- cross-workgroup hand-off -------------------------------------------------
// Split partials travel between workgroups that may sit on different XCDs,
// whose L2 caches are not coherent with each other. An agent-scope relaxed
// atomic store/load is a plain `global_store/global_load ... sc1`, coherent
// across the device without the whole-L2 write-back / invalidate that an
// agent-scope fence (__threadfence) costs per workgroup. Every producing
// wave calls publish_wait() (s_waitcnt 0: its stores are complete) before
// the workgroup barrier that precedes the completion-counter increment; the
// consumer reads the partials with publish_load after it has seen the final
// count. (A plain __syncthreads does not wait for outstanding global stores
// on gfx950.)
__device__ __forceinline__ void publish_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float publish_load(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void publish_wait() { __builtin_amdgcn_s_waitcnt(0); }
// 16-byte forms through a buffer resource: cache-policy bit 4 of the buffer
// intrinsics is `sc1`, the same access the relaxed agent-scope atomics above
// lower to, four floats per instruction.
constexpr int kPublishAux = 16;
__device__ __forceinline__ void publish_store16(__amdgpu_buffer_rsrc_t r, uint32_t voff, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, 0, kPublishAux);
}
__device__ __forceinline__ u32x4 publish_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, kPublishAux);
}
// Returns true in exactly one workgroup: the last of `n` to arrive.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t n) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1;
}

// ---- SwiGLU ------------------------------------------------------------------
// silu(g) * u of one element in fp32 (the decode step's MLP activation; the
// elementwise kernels and the W4A16 SwiGLU epilogue share it, so both round
// the same value).
__device__ __forceinline__ float silu_mul1(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// ---- rotary embedding ---------------------------------------------------------
// The rotation of one pair (x[d], x[d + D/2]): rotate_half(x) = [-x[D/2:],
// x[:D/2]], so out[d] = x1 c1 - x2 s1 and out[d + D/2] = x2 c2 + x1 s2. The
// fma is written out once here so that every kernel using it (rope, the
// decode step's rope + cache append, the W4A16 q|k|v epilogue) rounds the
// same way.
__device__ __forceinline__ void rope_pair(float x1, float x2, float c1, float s1, float c2, float s2,
                                          uint16_t& o1, uint16_t& o2) {
    o1 = f2h_bits(fmaf(x1, c1, -(x2 * s1)));
    o2 = f2h_bits(fmaf(x2, c2, x1 * s2));
}

// ---- exact symmetric quantisation step ------------------------------------
// Returns rint(x / s) with x / s the IEEE correctly rounded fp32 quotient,
// which is what torch's CPU `x / scale` followed by `.round()` computes.
// `r` must be within 1 ulp of 1 / s (v_rcp_f32, recip_approx below, is).
// For |x / s| <= 256 the product y = x * r is then within 2^-14 of the
// correctly rounded quotient (256 * (2^-23 + 2^-24 + 2^-24)), so both round
// to the same integer unless y lies that close to a half-integer; within
// 2^-12 of one (a tie of the true quotient rounds to even, a near-tie may go
// either way) the true division runs. As |y - k| <= 0.5 for k = rint(y),
// "within 2^-12 of a half-integer" is |y - k| >= 0.5 - 2^-12 (one compare,
// no second subtraction). NaN and infinite quotients (y - k is NaN) come out
// of the fast path unchanged.
__device__ __forceinline__ float quant_round(float x, float s, float r) {
    const float y = x * r;
    const float k = __builtin_rintf(y);
    if (fabsf(y - k) >= 0.5f - 0x1p-12f) return __builtin_rintf(x / s);
    return k;
}

// 1 / s to within 1 ulp (v_rcp_f32): the reciprocal quant_round expects.
__device__ __forceinline__ float recip_approx(float s) { return __builtin_amdgcn_rcpf(s); }

// ---- torch's non-finite semantics for the symmetric quantisers ------------
// |x| as bits. With the sign cleared, the unsigned order of the bit patterns
// is the float order and every NaN sits above +inf, so an unsigned max over
// them is torch's `x.abs().amax()`, which propagates NaN (fmaxf drops it).
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7FFFFFFFu; }

// Unsigned max over the 16 lanes of a DPP row; every lane gets the result.
__device__ __forceinline__ uint32_t row16_umax(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppQuadXor1, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppQuadXor2, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppRowHalfMirror, 0xF, 0xF, true));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppRowMirror, 0xF, 0xF, true));
    return v;
}

// (absmax / qmax).clamp(min=1e-8) in fp32: a NaN absmax stays NaN (torch's
// clamp keeps NaN), +inf stays +inf.
__device__ __forceinline__ float sym_scale(uint32_t absmax_bits, float qmax) {
    const float s = __uint_as_float(absmax_bits) / qmax;
    return s < 1.0e-8f ? 1.0e-8f : s;
}

// clamp(round(x / s), -qmax, qmax) as an integer code (r = 1 / s). A NaN
// quotient (a NaN scale, or inf / inf) gives code 0, which is what torch's
// float -> int8 conversion of NaN stores on x86; finite / inf is 0 already.
// v_cvt_i32_f32 converts NaN to 0 and saturates out-of-range values (CDNA
// ISA), so the conversion comes first and the clamp is one integer med3; it
// is written as inline asm because a C++ float -> int conversion of NaN is
// undefined behaviour the compiler may exploit.
__device__ __forceinline__ int sym_code(float x, float s, float r, int qmax) {
    const float v = quant_round(x, s, r);
    int c;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(c) : "v"(v));
    return min(max(c, -qmax), qmax);
}

}  // namespace llmik
