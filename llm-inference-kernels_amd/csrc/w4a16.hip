// W4A16 (INT4 weight, fp16 activation, group-wise fp16 scales) GEMV/GEMM
// for gfx950.
//
//   out[m, n] = sum_k act[m, k] * q[k, n] * scale[k / group_size, n]
//
// (reference/quant_matmul_ref.py:112-135; bindings/extension.cpp:322-376.)
// weight_packed is [K/8, N] uint32: bits 4i..4i+3 of word (kp, n) hold the
// two's-complement code of K position 8*kp + i
// (reference/quant_matmul_ref.py:140-165).
//
// Split-K with a deterministic in-kernel reduction: each workgroup writes
// its fp32 partial for its (column tile, K split) to the workspace; the last
// workgroup of a column tile (completion counter) sums the splits in fixed
// order and writes the output. One launch per call, no float atomics (the
// reference accumulates split partials with atomicAdd,
// kernels/quant/quant_matmul.cu:586-597).
#include <atomic>
#include <cstdlib>

#include "device_common.hpp"
#include "llmik_internal.hpp"

#include <cstdlib>

namespace llmik {

constexpr int kGemmThreads = 256;   // 4 waves share one column tile
constexpr int kGemmWaves = kGemmThreads / kWave;

struct GemmParams {
    const uint16_t* act;
    const uint32_t* w;
    const uint16_t* scale;
    void* out;
    float* part;         // [splits, M, N]
    uint32_t* counters;  // [m_tiles * n_tiles]
    int M, N, K, group_size;
    int splits, kp_per_split, n_tiles;
    int f32_out;
    int gshift;          // log2(group_size / 32) on the matrix-core GEMV
    int nw;              // streaming GEMV: waves per workgroup
    int wave_steps;      // streaming GEMV / 32x32 GEMM: 32-K steps per wave
    int m_tiles_;        // 32x32 GEMM: row tiles
    int full_tiles;      // LDS-staged GEMM: leading tiles computed whole (no K split)
    int vec_out;         // 32x32 GEMM: out is 16-byte aligned (vector stores)
    // Streaming GEMV pair epilogues: each 64-column tile holds 32 column
    // pairs (i, i + 32). kEpiSwiglu: see store_swiglu; kEpiQkvRope: see
    // store_qkv_rope (rotary tables of the position, q output, KV cache).
    int epilogue;
    const uint16_t* rope_cos;   // [128]
    const uint16_t* rope_sin;   // [128]
    uint16_t* q_out;            // [M, n_q_heads, 128]
    uint16_t* k_cache;          // [M, n_kv_heads, cache_len, 128]
    uint16_t* v_cache;
    int n_q_heads, n_kv_heads, cache_len, cache_pos;
};
constexpr int kEpiPlain = 0, kEpiSwiglu = 1, kEpiQkvRope = 2;

// Eight int4 codes of one word -> four fp16 pairs, exact. Pair j holds the
// codes of K positions (j, j + 4):
//   u = code + 8 (xor 0x8 per nibble); 0x6400 | u is the fp16 value 1024 + u,
//   and 0x6400 | (u << 4) is 1024 + 16u; subtracting / rescaling recovers
//   the code exactly.
// The masked nibbles and the exponent bits never overlap, so
//   ((w ^ 0x88888888) & m) | 0x6400 6400  ==  (w & m) ^ (0x6400 6400 | (0x88888888 & m)),
// one three-operand bit op per pair when the mask and the xor constant sit
// in VGPRs (CodeMasks, built once per kernel: vgpr_const is volatile and is
// never re-materialised).
struct CodeMasks {
    uint32_t m_lo, m_hi, x_lo, x_hi;
};
__device__ __forceinline__ CodeMasks code_masks() {
    return {vgpr_const(0x000F000Fu), vgpr_const(0x00F000F0u), vgpr_const(0x64086408u),
            vgpr_const(0x64806480u)};
}
__device__ __forceinline__ void i4x8_to_f16_pairs(uint32_t w, f16x2 out[4], const CodeMasks& k) {
    const uint32_t w8 = w >> 8;
    const uint32_t a = (w & k.m_lo) ^ k.x_lo;
    const uint32_t b = (w & k.m_hi) ^ k.x_hi;
    const uint32_t c = (w8 & k.m_lo) ^ k.x_lo;
    const uint32_t d = (w8 & k.m_hi) ^ k.x_hi;
    const f16x2 bias = {(f16)1032.0f, (f16)1032.0f};
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 bias16 = {(f16)72.0f, (f16)72.0f};
    out[0] = as_f16x2(a) - bias;
    out[1] = as_f16x2(b) * sixteenth - bias16;
    out[2] = as_f16x2(c) - bias;
    out[3] = as_f16x2(d) * sixteenth - bias16;
}

// Activation pairs matching i4x8_to_f16_pairs: (a0,a4), (a1,a5), (a2,a6), (a3,a7).
__device__ __forceinline__ void act_pairs(const u32x4 a, f16x2 out[4]) {
    const uint32_t w0 = a[0], w1 = a[1], w2 = a[2], w3 = a[3];
    const f16x2 lo0 = as_f16x2(w0);   // a0 a1
    const f16x2 lo1 = as_f16x2(w1);   // a2 a3
    const f16x2 hi0 = as_f16x2(w2);   // a4 a5
    const f16x2 hi1 = as_f16x2(w3);   // a6 a7
    out[0] = f16x2{lo0[0], hi0[0]};
    out[1] = f16x2{lo0[1], hi0[1]};
    out[2] = f16x2{lo1[0], hi1[0]};
    out[3] = f16x2{lo1[1], hi1[1]};
}

// Sum of n split partials p[0], p[stride], ... in split order. The loads are
// issued in independent batches so the reduction costs a few memory round
// trips instead of one per split.
__device__ __forceinline__ float sum_splits(const float* p, long stride, int n) {
    constexpr int kBatch = 8;
    float v = 0.0f;
    for (int s0 = 0; s0 < n; s0 += kBatch) {
        float x[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) x[u] = publish_load(p + (long)min(s0 + u, n - 1) * stride);
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v += (s0 + u < n) ? x[u] : 0.0f;
    }
    return v;
}

// Store the workgroup's column-tile result, or publish it as a split partial
// and let the last split of the tile reduce. `vals[j]` belongs to column
// n0 + j for j < count (thread-local columns), row m.
__device__ __forceinline__ void store_out(const GemmParams& p, int m, int n, float v) {
    if (p.f32_out) {
        static_cast<float*>(p.out)[(long)m * p.N + n] = v;
    } else {
        static_cast<uint16_t*>(p.out)[(long)m * p.N + n] = f2h_bits(v);
    }
}

// SwiGLU epilogue of the streaming GEMV. The weight's columns come in 64-column
// tiles of 32 gate columns followed by the matching 32 up columns; column c of
// the [M, N / 2] fp16 output is silu(g) * u of the fp16-rounded gate and up
// products, the same value an fp16 gate|up product followed by silu_mul rounds.
__device__ __forceinline__ void store_swiglu(const GemmParams& p, int m, int c, float g, float u) {
    const float gh = h2f(f2h_bits(g)), uh = h2f(f2h_bits(u));
    static_cast<uint16_t*>(p.out)[(long)m * (p.N / 2) + c] = f2h_bits(silu_mul1(gh, uh));
}

// q|k|v epilogue of the streaming GEMV (head_dim 128). The weight's columns
// are those of the concatenated q | k | v projection with each head's two
// 64-dimension halves interleaved in 32-column blocks: tile t is head t / 2,
// dimensions 32 (t % 2) .. + 31, then the same dimensions + 64, so pair i of
// tile t is the rotary pair (d, d + 64), d = 32 (t % 2) + i. Both values are
// rounded to fp16 (the fp16 q|k|v output) and stored as rope_qkv_append
// stores them: q heads and k heads rotated (q to q_out, k into cache slot
// cache_pos), v heads copied into their slot.
__device__ __forceinline__ void store_qkv_rope(const GemmParams& p, int b, int tile, int i, float v1,
                                               float v2) {
    const int head = tile >> 1;
    const int d = 32 * (tile & 1) + i;
    const uint16_t h1 = f2h_bits(v1), h2 = f2h_bits(v2);
    const int H = p.n_q_heads, Hkv = p.n_kv_heads;
    if (head >= H + Hkv) {
        uint16_t* dst = p.v_cache + (((long)b * Hkv + (head - H - Hkv)) * p.cache_len + p.cache_pos) * 128;
        dst[d] = h1;
        dst[d + 64] = h2;
        return;
    }
    uint16_t* dst = head < H ? p.q_out + ((long)b * H + head) * 128
                             : p.k_cache + (((long)b * Hkv + (head - H)) * p.cache_len + p.cache_pos) * 128;
    rope_pair(h2f(h1), h2f(h2), h2f(p.rope_cos[d]), h2f(p.rope_sin[d]), h2f(p.rope_cos[d + 64]),
              h2f(p.rope_sin[d + 64]), dst[d], dst[d + 64]);
}

__device__ __forceinline__ void store_pair(const GemmParams& p, int m, int tile, int i, float a, float b) {
    if (p.epilogue == kEpiSwiglu) store_swiglu(p, m, tile * 32 + i, a, b);
    else store_qkv_rope(p, m, tile, i, a, b);
}

// 4 consecutive outputs of row m from column n (a multiple of 4): one 16- /
// 8-byte store when the output allows it (vec_out: base 16-byte aligned),
// else one store per value.
__device__ __forceinline__ void store_out4(const GemmParams& p, int m, int n, const f32x4 v) {
    const long base = (long)m * p.N + n;
    if (!p.vec_out) {
#pragma unroll
        for (int e = 0; e < 4; ++e) store_out(p, m, n + e, v[e]);
    } else if (p.f32_out) {
        *reinterpret_cast<f32x4*>(static_cast<float*>(p.out) + base) = v;
    } else {
        const uint32_t lo = (uint32_t)f2h_bits(v[0]) | ((uint32_t)f2h_bits(v[1]) << 16);
        const uint32_t hi = (uint32_t)f2h_bits(v[2]) | ((uint32_t)f2h_bits(v[3]) << 16);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.out) + base) = u32x2{lo, hi};
    }
}

// ---------------------------------------------------------------------------
// M == 1: each lane owns COLS adjacent columns (one 4*COLS-byte load per
// packed row); the 4 waves of a workgroup cover contiguous slices of the
// workgroup's K range and are summed in LDS.
// ---------------------------------------------------------------------------
template <int COLS>
__global__ __launch_bounds__(kGemmThreads) void w4a16_gemv_kernel(GemmParams p) {
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = tile * (64 * COLS) + lane * COLS;
    const bool active = n0 < p.N;

    const int kp_total = p.K / 8;
    const int kp_split0 = split * p.kp_per_split;
    const int kp_split1 = min(kp_split0 + p.kp_per_split, kp_total);
    const int per_wave = (p.kp_per_split + kGemmWaves - 1) / kGemmWaves;
    const int kp0 = min(kp_split0 + wave * per_wave, kp_split1);
    const int kp1 = min(kp0 + per_wave, kp_split1);
    const int kp_per_group = p.group_size / 8;

    float acc[COLS], accg[COLS];
    const CodeMasks km = code_masks();
#pragma unroll
    for (int j = 0; j < COLS; ++j) acc[j] = accg[j] = 0.0f;
    int g_cur = kp0 / kp_per_group;

    for (int kp = kp0; kp < kp1; ++kp) {
        const int g = kp / kp_per_group;
        if (g != g_cur) {
            if (active) {
#pragma unroll
                for (int j = 0; j < COLS; ++j) {
                    acc[j] = fmaf(h2f(p.scale[(long)g_cur * p.N + n0 + j]), accg[j], acc[j]);
                    accg[j] = 0.0f;
                }
            }
            g_cur = g;
        }
        f16x2 ap[4];
        act_pairs(load16(p.act + 8 * kp), ap);
        if (active) {
            uint32_t wv[COLS];
            if constexpr (COLS == 4) {
                const u32x4 raw = stream16(p.w + (long)kp * p.N + n0);
                wv[0] = raw[0]; wv[1] = raw[1]; wv[2] = raw[2]; wv[3] = raw[3];
            } else {
                wv[0] = stream4(p.w + (long)kp * p.N + n0);
            }
#pragma unroll
            for (int j = 0; j < COLS; ++j) {
                f16x2 wp[4];
                i4x8_to_f16_pairs(wv[j], wp, km);
#pragma unroll
                for (int i = 0; i < 4; ++i) accg[j] = __builtin_amdgcn_fdot2(ap[i], wp[i], accg[j], false);
            }
        }
    }
    if (active && kp0 < kp1) {
#pragma unroll
        for (int j = 0; j < COLS; ++j)
            acc[j] = fmaf(h2f(p.scale[(long)g_cur * p.N + n0 + j]), accg[j], acc[j]);
    }

    __shared__ float s_part[kGemmWaves][64 * COLS];
    __shared__ uint32_t s_last;
#pragma unroll
    for (int j = 0; j < COLS; ++j) s_part[wave][lane * COLS + j] = acc[j];
    __syncthreads();

    const int tile_n = 64 * COLS;
    const int nbase = tile * tile_n;
    float tot[(64 * COLS + kGemmThreads - 1) / kGemmThreads];
#pragma unroll
    for (int i = 0; i < (64 * COLS + kGemmThreads - 1) / kGemmThreads; ++i) {
        const int col = threadIdx.x + i * kGemmThreads;
        tot[i] = 0.0f;
        if (col < tile_n) {
#pragma unroll
            for (int w = 0; w < kGemmWaves; ++w) tot[i] += s_part[w][col];
        }
    }

    if (p.splits == 1) {
#pragma unroll
        for (int i = 0; i < (64 * COLS + kGemmThreads - 1) / kGemmThreads; ++i) {
            const int col = threadIdx.x + i * kGemmThreads;
            if (col < tile_n && nbase + col < p.N) store_out(p, 0, nbase + col, tot[i]);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < (64 * COLS + kGemmThreads - 1) / kGemmThreads; ++i) {
        const int col = threadIdx.x + i * kGemmThreads;
        if (col < tile_n && nbase + col < p.N) publish_store(&p.part[(long)split * p.N + nbase + col], tot[i]);
    }
    publish_wait();
    __syncthreads();
    if (threadIdx.x == 0) s_last = arrive_last(&p.counters[tile], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
#pragma unroll
    for (int i = 0; i < (64 * COLS + kGemmThreads - 1) / kGemmThreads; ++i) {
        const int col = threadIdx.x + i * kGemmThreads;
        if (col < tile_n && nbase + col < p.N)
            store_out(p, 0, nbase + col, sum_splits(p.part + nbase + col, (long)p.N, p.splits));
    }
    if (threadIdx.x == 0) p.counters[tile] = 0u;
}

// ---------------------------------------------------------------------------
// M == 1 on the matrix cores (group_size a power of two >= 32).
//
// Work unit: a tile of 16 * CB columns and one K split. The grid is laid
// out so that each XCD (workgroup id mod 8) takes a contiguous run of tiles:
// neighbouring column strips of a packed row are then read by one L2 at
// about the same time. Within a workgroup, kGemvWaves waves own whole
// batches of the split's 32-K steps and are summed in LDS; with several
// splits the last split of a tile adds the partials in split order.
//
// In a 16x16x32 MFMA the B operand of a lane is one packed word: 8 K
// positions of one column. Lane l loads CB adjacent words of packed row
// 4 * step + (l >> 4), columns n0 + CB * (l & 15) + j, and feeds word j to
// MFMA j (columns j, j + CB, j + 2CB, ... of the tile).
//
// The word goes into the MFMA still biased: with u = code + 8, the low
// nibbles (even K offsets i) become the fp16 value 1024 + u and the high
// nibbles (odd i) 1024 + 16u (exact bit patterns 0x6400 | u, 0x6400 | u<<4),
// in the pair order (i0,i4), (i1,i5), (i2,i6), (i3,i7). The activation is
// staged per workgroup in LDS in that order, with odd offsets divided by 16
// (exact), so for each K position the product is
//   even: a (1024 + u)        = a * code + 1032 a
//   odd : (a / 16)(1024 + 16u) = a * code +   72 a
// and a 32-K step of the MFMA yields sum(a * code) + corr[step], with
// corr[step] = 1032 * sum_even(a) + 72 * sum_odd(a) staged beside it. Each
// step lies inside one scale group: acc += scale[g][n] * (t - corr[step]).
// Every row of the 16x16 product is the same; row 0 is used.
//
// Loads: the activation loads of all waves are issued first, then each
// wave's first two batches (weight words and group scales) before the
// activation is staged, later batches one batch ahead of use (ping-pong). Step and group indices are clamped to the tensors, so
// every load stays in bounds; steps past the split meet a zero-padded
// activation and add 0.
// ---------------------------------------------------------------------------
#ifndef LLMIK_GEMV_CB
#define LLMIK_GEMV_CB 2           // words per lane per step: tile = 16 * CB columns
#endif
#ifndef LLMIK_GEMV_WGS_PER_CU
#define LLMIK_GEMV_WGS_PER_CU 1   // K splits are added until tiles * splits reaches this per CU
#endif
constexpr int kGemvWaves = 8;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kGemvBatch = 8;          // 32-K steps per load batch (256 * CB bytes per step)
constexpr int kGemvMaxK = 16384;        // K per split: activation and corrections in LDS
constexpr int kGemvMaxStage = kGemvMaxK / 8 / kGemvThreads;

// LDS bytes for a split of `sps` steps with `sb`-step batches: activation
// (plus one zero batch) in fp16, per-chunk and per-step corrections in fp32.
__host__ __device__ constexpr size_t gemv_lds_bytes(int sps, int sb) {
    return (size_t)(sps + sb) * 64 + (size_t)sps * 16 + (size_t)(sps + sb) * 4;
}

template <int N_>
struct UIntVec;
template <> struct UIntVec<1> { using T = uint32_t; };
template <> struct UIntVec<2> { using T = u32x2; };
template <> struct UIntVec<4> { using T = u32x4; };

template <int CB>
__device__ __forceinline__ typename UIntVec<CB>::T buffer_load_words(__amdgpu_buffer_rsrc_t r,
                                                                     uint32_t voff, uint32_t soff) {
    if constexpr (CB == 1) return __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 2);
    else if constexpr (CB == 2) return __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 2);
    else return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2);
}

template <int CB>
__device__ __forceinline__ uint32_t word_of(const typename UIntVec<CB>::T& v, int j) {
    if constexpr (CB == 1) return v;
    else return v[j];
}

// Weight words and scales of one batch of SB steps. GSHIFT = min(log2 of
// steps per group, log2 SB): the batch touches NG groups; a group's scales
// for the lane's CB columns are CB adjacent fp16.
template <int CB, int GSHIFT>
struct GemvBatch {
    static constexpr int SB = kGemvBatch;
    static constexpr int NG = SB >> GSHIFT;
    static constexpr int SW = (CB + 1) / 2;   // dwords of CB fp16 scales
    typename UIntVec<CB>::T w[SB];
    typename UIntVec<SW>::T s[NG];
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs,
                                         uint32_t w_off, uint32_t s_off, uint32_t step_bytes,
                                         uint32_t grp_bytes, int step0, int last_step,
                                         int gshift, int last_grp) {
        // Steps past the split's last one re-read that step (same CU, cached).
#pragma unroll
        for (int j = 0; j < SB; ++j)
            w[j] = buffer_load_words<CB>(rw, w_off, (uint32_t)min(step0 + j, last_step) * step_bytes);
        const int g0 = step0 >> gshift;
#pragma unroll
        for (int u = 0; u < NG; ++u) {
            const uint32_t so = (uint32_t)min(g0 + u, last_grp) * grp_bytes;
            if constexpr (CB == 1) s[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)s_off, (int)so, 0);
            else s[u] = buffer_load_words<SW>(rs, s_off, so);
        }
    }
    __device__ __forceinline__ float scale(int j, int cb) const {
        const int u = j >> GSHIFT;
        uint32_t d;
        if constexpr (CB == 1) d = s[u];
        else d = word_of<SW>(s[u], cb >> 1);
        return h2f((uint16_t)((cb & 1) ? (d >> 16) : d));
    }
};

// MULTI: every wave owns more than one batch (the host knows from the
// plan). The two paths issue a fixed number of loads before the staging, so
// the wait for the activation never includes weight loads.
template <int CB, int NSTAGE, int GSHIFT, bool MULTI>
__global__ __launch_bounds__(kGemvThreads) void w4a16_gemv_mfma_kernel(GemmParams p) {
    constexpr int SB = kGemvBatch;
    constexpr int TN = 16 * CB;
    extern __shared__ __attribute__((aligned(16))) uint16_t s_dyn[];
    __shared__ float s_red[kGemvWaves][TN];
    __shared__ uint32_t s_last;

    // XCD-contiguous order: workgroup b runs on XCD b % 8.
    int b = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
    const int tile = b % p.n_tiles;
    const int split = b / p.n_tiles;

    const int steps = p.K / 32;
    const int sps = p.kp_per_split / 4;          // steps per split, a multiple of SB
    const int k0 = split * sps;
    const int nst = min(sps, steps - k0);        // steps of this split
    uint16_t* s_act = s_dyn;                                                 // [sps + SB][32]
    float* s_cchunk = reinterpret_cast<float*>(s_dyn + 32 * (sps + SB));     // [4 * sps]
    float* s_corr = s_cchunk + 4 * sps;                                      // [sps + SB]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int kq = lane >> 4;
    const int n0 = tile * TN;
    const int col0 = n0 + CB * c;

    // ---- activation staging loads first (the split's 8-element chunks) ----
    const int n_act = 4 * nst;
    const uint16_t* act = p.act + 32 * k0;
    u32x4 stage[NSTAGE];
#pragma unroll
    for (int i = 0; i < NSTAGE; ++i)
        stage[i] = load16(act + 8 * min((int)threadIdx.x + i * kGemvThreads, n_act - 1));

    // Every wave's activation loads enter the CU's memory pipeline before any
    // weight load (a bare barrier: it waits for no memory counter), so the
    // staging does not queue behind other waves' weight streams.
    __builtin_amdgcn_s_barrier();

    // ---- then the wave's first two batches ----
    const int per_wave = p.kp_per_split / 4 / kGemvWaves;   // whole batches, same for all waves
    const int s0 = wave * per_wave;                          // past nst in a short last split
    const int s1 = min(s0 + per_wave, nst);
    const int last = k0 + nst - 1;
    const int n_grp = p.K / p.group_size;
    const __amdgpu_buffer_rsrc_t rw = make_buffer_rsrc(p.w, (uint32_t)(p.K / 8) * p.N * 4u);
    const __amdgpu_buffer_rsrc_t rs = make_buffer_rsrc(p.scale, (uint32_t)n_grp * p.N * 2u);
    const uint32_t w_off = ((uint32_t)kq * p.N + col0) * 4u;
    const uint32_t s_off = (uint32_t)col0 * 2u;
    const uint32_t step_bytes = (uint32_t)p.N * 16u;
    const uint32_t grp_bytes = (uint32_t)p.N * 2u;
    GemvBatch<CB, GSHIFT> ba, bb;
    ba.load(rw, rs, w_off, s_off, step_bytes, grp_bytes, k0 + s0, last, p.gshift, n_grp - 1);
    if constexpr (MULTI)
        bb.load(rw, rs, w_off, s_off, step_bytes, grp_bytes, k0 + s0 + SB, last, p.gshift, n_grp - 1);

    // ---- stage the activation in pair order, odd offsets / 16 ----
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
#pragma unroll
    for (int i = 0; i < NSTAGE; ++i) {
        const int idx = (int)threadIdx.x + i * kGemvThreads;
        if (idx < n_act) {
            const u32x4 a = stage[i];
            const f16x2 odd0 = as_f16x2(perm_b32(a[2], a[0], 0x07060302u)) * sixteenth;   // a1 a5
            const f16x2 odd1 = as_f16x2(perm_b32(a[3], a[1], 0x07060302u)) * sixteenth;   // a3 a7
            u32x4 r;
            r[0] = perm_b32(a[2], a[0], 0x05040100u);   // a0 a4
            r[1] = __builtin_bit_cast(uint32_t, odd0);
            r[2] = perm_b32(a[3], a[1], 0x05040100u);   // a2 a6
            r[3] = __builtin_bit_cast(uint32_t, odd1);
            *reinterpret_cast<u32x4*>(&s_act[8 * idx]) = r;
            float av[8];
            f16x8_to_f32(a, av);
            s_cchunk[idx] = 1032.0f * ((av[0] + av[2]) + (av[4] + av[6])) +
                            72.0f * ((av[1] + av[3]) + (av[5] + av[7]));
        }
    }
    // zero padding: activation and corrections of the steps [nst, nst + SB)
    for (int t = threadIdx.x; t < 4 * SB; t += kGemvThreads)
        *reinterpret_cast<u32x4*>(&s_act[32 * nst + 8 * t]) = u32x4{0u, 0u, 0u, 0u};
    if ((int)threadIdx.x < SB) s_corr[nst + threadIdx.x] = 0.0f;
    __syncthreads();
    for (int st = threadIdx.x; st < nst; st += kGemvThreads) {
        const float* q = s_cchunk + 4 * st;
        s_corr[st] = (q[0] + q[1]) + (q[2] + q[3]);
    }
    __syncthreads();

    // The masks and the exponent bits live in VGPRs so that each
    // (word & mask) | bias is a single three-operand bit op.
    const uint32_t m_lo = vgpr_const(0x000F000Fu);
    const uint32_t m_hi = vgpr_const(0x00F000F0u);
    const uint32_t bias = vgpr_const(0x64006400u);
    float acc[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[j] = 0.0f;
    auto consume = [&](const GemvBatch<CB, GSHIFT>& bt, int b0) {
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const int st = b0 + j;
            const f16x8 aop = __builtin_bit_cast(
                f16x8, *reinterpret_cast<const u32x4*>(&s_act[32 * st + 8 * kq]));
            const float corr = s_corr[st];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                const uint32_t w = word_of<CB>(bt.w[j], cb) ^ 0x88888888u;
                const uint32_t w8 = w >> 8;
                const u32x4 braw = make_u32x4((w & m_lo) | bias, (w & m_hi) | bias,
                                              (w8 & m_lo) | bias, (w8 & m_hi) | bias);
                const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    aop, __builtin_bit_cast(f16x8, braw), f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                acc[cb] = fmaf(bt.scale(j, cb), t[0] - corr, acc[cb]);
            }
        }
    };
    if constexpr (!MULTI) {
        if (s0 < s1) consume(ba, s0);
    } else if (s0 < s1) {
        for (int b0 = s0;; b0 += 2 * SB) {
            consume(ba, b0);
            if (b0 + SB >= s1) break;
            // Issued unconditionally (clamped) so the wait before each use stays exact.
            ba.load(rw, rs, w_off, s_off, step_bytes, grp_bytes, k0 + b0 + 2 * SB, last, p.gshift,
                    n_grp - 1);
            __builtin_amdgcn_sched_barrier(0);
            consume(bb, b0 + SB);
            if (b0 + 2 * SB >= s1) break;
            bb.load(rw, rs, w_off, s_off, step_bytes, grp_bytes, k0 + b0 + 3 * SB, last, p.gshift,
                    n_grp - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    if (kq == 0) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) s_red[wave][CB * c + cb] = acc[cb];
    }
    __syncthreads();
    const int t = threadIdx.x;
    float v = 0.0f;
    if (t < TN) {
#pragma unroll
        for (int w = 0; w < kGemvWaves; ++w) v += s_red[w][t];
    }
    if (p.splits == 1) {
        if (t < TN) store_out(p, 0, n0 + t, v);
        return;
    }
    if (t < TN) publish_store(&p.part[(long)split * p.N + n0 + t], v);
    publish_wait();
    __syncthreads();
    if (t == 0) s_last = arrive_last(&p.counters[tile], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    if (t < TN) store_out(p, 0, n0 + t, sum_splits(p.part + n0 + t, (long)p.N, p.splits));
    if (t == 0) p.counters[tile] = 0u;
}

template <int CB, int NSTAGE, bool MULTI>
static void launch_gemv_cb_stage(const GemmParams& p, int grid, size_t lds, hipStream_t stream) {
    const dim3 g(grid), blk(kGemvThreads);
    switch (min(p.gshift, 3)) {   // 3 = log2(kGemvBatch): a batch inside one group
        case 0: hipLaunchKernelGGL((w4a16_gemv_mfma_kernel<CB, NSTAGE, 0, MULTI>), g, blk, lds, stream, p); break;
        case 1: hipLaunchKernelGGL((w4a16_gemv_mfma_kernel<CB, NSTAGE, 1, MULTI>), g, blk, lds, stream, p); break;
        case 2: hipLaunchKernelGGL((w4a16_gemv_mfma_kernel<CB, NSTAGE, 2, MULTI>), g, blk, lds, stream, p); break;
        default: hipLaunchKernelGGL((w4a16_gemv_mfma_kernel<CB, NSTAGE, 3, MULTI>), g, blk, lds, stream, p); break;
    }
}

template <int CB>
static void launch_gemv_cb(const GemmParams& p, int grid, int sps, hipStream_t stream) {
    const size_t lds = gemv_lds_bytes(sps, kGemvBatch);
    const bool multi = sps / kGemvWaves > kGemvBatch;
    const int stage = (4 * sps + kGemvThreads - 1) / kGemvThreads;
    if (multi) {
        switch (stage) {
            case 1: launch_gemv_cb_stage<CB, 1, true>(p, grid, lds, stream); break;
            case 2: launch_gemv_cb_stage<CB, 2, true>(p, grid, lds, stream); break;
            case 3: launch_gemv_cb_stage<CB, 3, true>(p, grid, lds, stream); break;
            default: launch_gemv_cb_stage<CB, kGemvMaxStage, true>(p, grid, lds, stream); break;
        }
    } else {
        switch (stage) {
            case 1: launch_gemv_cb_stage<CB, 1, false>(p, grid, lds, stream); break;
            case 2: launch_gemv_cb_stage<CB, 2, false>(p, grid, lds, stream); break;
            case 3: launch_gemv_cb_stage<CB, 3, false>(p, grid, lds, stream); break;
            default: launch_gemv_cb_stage<CB, kGemvMaxStage, false>(p, grid, lds, stream); break;
        }
    }
}

// ---------------------------------------------------------------------------
// 1 <= M <= 16, N % 64 == 0, group_size a power of two >= 32: streaming
// matrix-core GEMV (plan kind 5; the default for the decode shapes).
//
// A workgroup owns a 64-column tile and one K split; its nw (8..16) waves
// take consecutive ranges of wave_steps 32-K steps. Lane (kq, c) owns tile
// columns 4c..4c+3: per step it loads the 16-byte word quad of packed row
// 4*step + kq and, beside it, its own 16-byte fragment of activation row c
// (K offset 32*step + 8*kq; rows >= M read as zero). Weights and activation
// arrive together, so a step's arithmetic needs nothing staged and no
// barrier (an activation staged per workgroup would queue behind the
// weight stream of the whole chip before the first product could start).
// Every load of a batch is issued before any arithmetic waits on one; at
// most two batches are in flight per wave.
//
// Words enter the MFMA biased: with u = code + 8, 0x6400 | u is the fp16
// value 1024 + u and 0x6400 | u << 4 is 1024 + 16u, in the pair order
// (i0,i4), (i1,i5), (i2,i6), (i3,i7). The activation fragment is permuted
// to that order with the odd offsets divided by 16 (exact), so a product
// carries a bias of 1032 a (even offsets) or 72 a (odd offsets). One more
// MFMA per step, of the same activation against the constant operand
// (-1032, -1032, -1152, -1152, ...), accumulates minus that bias beside the
// four column accumulators; the scale is applied once per scale group:
//   acc[n] += scale[g][n] * (C_g[n] + Cbias_g).
// The waves' [MR x 64] partials are added in LDS in a fixed order.
// ---------------------------------------------------------------------------
constexpr int kStreamMaxWaves = 16;
constexpr int kStreamTile = 64;

template <int SB, int GSHIFT>
struct StreamBatch {
    static constexpr int NG = ((SB >> GSHIFT) > 0) ? (SB >> GSHIFT) : 1;
    u32x4 w[SB];
    u32x4 a[SB];
    u32x2 s[NG];
};

// NB > 0: the wave's NB batches are all issued up front. NB == 0: a loop
// over wave_steps / SB (even, >= 4) batches with two in flight.
template <int MR, int SB, int GSHIFT, int NB>
__global__ __launch_bounds__(kStreamMaxWaves * kWave) void w4a16_gemv_stream_kernel(GemmParams p) {
    constexpr int SPG = 1 << GSHIFT;   // steps per scale flush (a group, or the batch)
    constexpr int TN = kStreamTile;
    constexpr int NRED = kStreamMaxWaves / 2;
    __shared__ float s_red[NRED][MR][TN + 1];
    __shared__ uint32_t s_last;

    const int b = blockIdx.x;
    const int tile = b % p.n_tiles;
    const int split = b / p.n_tiles;
    const int steps = p.K / 32;
    const int sps = p.kp_per_split / 4;
    const int k0 = split * sps;
    const int nst = min(sps, steps - k0);
    const int nw = p.nw;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int kq = lane >> 4;
    const int n0 = tile * TN;
    const int col0 = n0 + 4 * c;
    const int ws0 = k0 + wave * p.wave_steps;                  // the wave's first step
    const int ws1 = min(ws0 + p.wave_steps, k0 + nst);         // one past its last
    // Loads of steps outside [ws0, ws1) re-read a step of the split (in
    // bounds, cached) and meet a zero activation, so they add exactly 0.
    const int lastvalid = (ws1 > ws0) ? ws1 - 1 : k0 + nst - 1;
    const int n_grp = p.K / p.group_size;

    const __amdgpu_buffer_rsrc_t rw = make_buffer_rsrc(p.w, (uint32_t)(p.K / 8) * p.N * 4u);
    const __amdgpu_buffer_rsrc_t ra = make_buffer_rsrc(p.act, (uint32_t)p.M * p.K * 2u);
    const __amdgpu_buffer_rsrc_t rs = make_buffer_rsrc(p.scale, (uint32_t)n_grp * p.N * 2u);
    const uint32_t w_off = ((uint32_t)kq * p.N + col0) * 4u;
    const uint32_t a_off = ((uint32_t)min(c, p.M - 1) * p.K + 8u * kq) * 2u;
    const uint32_t s_off = (uint32_t)col0 * 2u;
    const uint32_t step_bytes = (uint32_t)p.N * 16u;
    const uint32_t grp_bytes = (uint32_t)p.N * 2u;
    const bool row_ok = c < p.M;

    using Batch = StreamBatch<SB, GSHIFT>;
    auto load_batch = [&](Batch& bt, int sb0) {
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const uint32_t st = (uint32_t)min(sb0 + j, lastvalid);
            bt.w[j] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)w_off, (int)(st * step_bytes), 2);
            bt.a[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)a_off, (int)(st * 64u), 0);
        }
        const int g0 = min(sb0, lastvalid) >> p.gshift;
#pragma unroll
        for (int u = 0; u < Batch::NG; ++u) {
            const uint32_t so = (uint32_t)min(g0 + u, n_grp - 1) * grp_bytes;
            bt.s[u] = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)s_off, (int)so, 0);
        }
    };

    // The masks and the exponent bits live in VGPRs so that each
    // (word & mask) | bias is a single three-operand bit op.
    const uint32_t m_lo = vgpr_const(0x000F000Fu);
    const uint32_t m_hi = vgpr_const(0x00F000F0u);
    const uint32_t bias = vgpr_const(0x64006400u);
    // fp16 -1032 = 0xE408, -1152 = 0xE480
    const f16x8 bias_op =
        __builtin_bit_cast(f16x8, make_u32x4(0xE408E408u, 0xE480E480u, 0xE408E408u, 0xE480E480u));
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    f32x4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](const Batch& bt, int sb0) {
        f32x4 cg[4], cb4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) cg[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            u32x4 a = bt.a[j];
            if (!row_ok || sb0 + j >= ws1) a = u32x4{0u, 0u, 0u, 0u};
            const f16x2 odd0 = as_f16x2(perm_b32(a[2], a[0], 0x07060302u)) * sixteenth;   // a1 a5
            const f16x2 odd1 = as_f16x2(perm_b32(a[3], a[1], 0x07060302u)) * sixteenth;   // a3 a7
            const f16x8 aop = __builtin_bit_cast(f16x8, make_u32x4(
                perm_b32(a[2], a[0], 0x05040100u), __builtin_bit_cast(uint32_t, odd0),     // a0 a4
                perm_b32(a[3], a[1], 0x05040100u), __builtin_bit_cast(uint32_t, odd1)));   // a2 a6
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t wv = bt.w[j][q] ^ 0x88888888u;
                const uint32_t w8 = wv >> 8;
                const u32x4 braw = make_u32x4((wv & m_lo) | bias, (wv & m_hi) | bias,
                                              (w8 & m_lo) | bias, (w8 & m_hi) | bias);
                cg[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, __builtin_bit_cast(f16x8, braw),
                                                                cg[q], 0, 0, 0);
            }
            cb4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bias_op, cb4, 0, 0, 0);
            if ((j & (SPG - 1)) == SPG - 1) {
                const u32x2 sv = bt.s[j >> GSHIFT];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t d = sv[q >> 1];
                    const float scv = h2f((uint16_t)((q & 1) ? (d >> 16) : d));
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[q][i] = fmaf(scv, cg[q][i] + cb4[i], acc[q][i]);
                    cg[q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
                cb4 = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    };

    if constexpr (NB > 0) {
        Batch bt[NB];
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) load_batch(bt[ib], ws0 + ib * SB);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) consume(bt[ib], ws0 + ib * SB);
    } else {
        const int nbw = p.wave_steps / SB;   // even, >= 4
        Batch b0, b1;
        load_batch(b0, ws0);
        load_batch(b1, ws0 + SB);
        __builtin_amdgcn_sched_barrier(0);
        int i = 0;
        for (; i + 2 < nbw; i += 2) {
            consume(b0, ws0 + i * SB);
            load_batch(b0, ws0 + (i + 2) * SB);
            __builtin_amdgcn_sched_barrier(0);
            consume(b1, ws0 + (i + 1) * SB);
            load_batch(b1, ws0 + (i + 3) * SB);
            __builtin_amdgcn_sched_barrier(0);
        }
        consume(b0, ws0 + i * SB);
        consume(b1, ws0 + (i + 1) * SB);
    }

    // C layout: lane (c, kq) holds rows 4kq + i of tile columns 4c + q.
    // Waves >= NRED hand their partial to wave - NRED, which adds it; the
    // NRED slots are then summed in order.
    auto put = [&](int slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 4 * kq + i;
            if (row < MR) {
#pragma unroll
                for (int q = 0; q < 4; ++q) s_red[slot][row][4 * c + q] = acc[q][i];
            }
        }
    };
    if (wave >= NRED) put(wave - NRED);
    __syncthreads();
    if (wave < NRED) {
        if (wave + NRED < nw) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 4 * kq + i;
                if (row < MR) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[q][i] += s_red[wave][row][4 * c + q];
                }
            }
        }
        put(wave);
    }
    __syncthreads();
    // Outputs of the tile (min(M, MR) rows x 64 columns), strided over the
    // workgroup's nw * 64 threads.
    const int t = threadIdx.x;
    const int nthreads = nw * kWave;
    const int nout = min(p.M, MR) * TN;
    const int nslots = min(nw, NRED);
    auto tile_sum = [&](int o) {
        float v = 0.0f;
        for (int w = 0; w < nslots; ++w) v += s_red[w][o / TN][o % TN];
        return v;
    };
    constexpr int TH = TN / 2;
    const int nhalf = min(p.M, MR) * TH;   // SwiGLU outputs of the tile
    if (p.splits == 1) {
        if (p.epilogue != kEpiPlain) {
            for (int o = t; o < nhalf; o += nthreads) {
                const int row = o / TH, j = o % TH;
                store_pair(p, row, tile, j, tile_sum(row * TN + j), tile_sum(row * TN + TH + j));
            }
        } else {
            for (int o = t; o < nout; o += nthreads) store_out(p, o / TN, n0 + o % TN, tile_sum(o));
        }
        return;
    }
    for (int o = t; o < nout; o += nthreads)
        publish_store(&p.part[((long)split * p.M + o / TN) * p.N + n0 + o % TN], tile_sum(o));
    publish_wait();
    __syncthreads();
    if (t == 0) s_last = arrive_last(&p.counters[tile], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    if (p.epilogue != kEpiPlain) {
        for (int o = t; o < nhalf; o += nthreads) {
            const int row = o / TH, j = o % TH;
            const float* base = p.part + (long)row * p.N + n0;
            store_pair(p, row, tile, j, sum_splits(base + j, (long)p.M * p.N, p.splits),
                       sum_splits(base + TH + j, (long)p.M * p.N, p.splits));
        }
    } else {
        for (int o = t; o < nout; o += nthreads) {
            const int row = o / TN, col = o % TN;
            store_out(p, row, n0 + col,
                      sum_splits(p.part + (long)row * p.N + n0 + col, (long)p.M * p.N, p.splits));
        }
    }
    if (t == 0) p.counters[tile] = 0u;
}

template <int MR, int SB, int NB>
static void launch_stream_sb(const GemmParams& p, int grid, hipStream_t stream) {
    const dim3 g(grid), blk(p.nw * kWave);
    constexpr int MAXG = (SB >= 4) ? 2 : 1;   // log2 SB
    switch (min(p.gshift, MAXG)) {
        case 0: hipLaunchKernelGGL((w4a16_gemv_stream_kernel<MR, SB, 0, NB>), g, blk, 0, stream, p); break;
        case 1: hipLaunchKernelGGL((w4a16_gemv_stream_kernel<MR, SB, 1, NB>), g, blk, 0, stream, p); break;
        default: hipLaunchKernelGGL((w4a16_gemv_stream_kernel<MR, SB, MAXG, NB>), g, blk, 0, stream, p); break;
    }
}

template <int MR>
static void launch_stream(const GemmParams& p, int grid, hipStream_t stream) {
    switch (p.wave_steps) {
        case 2: launch_stream_sb<MR, 2, 1>(p, grid, stream); break;
        case 4: launch_stream_sb<MR, 4, 1>(p, grid, stream); break;
        case 8: launch_stream_sb<MR, 4, 2>(p, grid, stream); break;
        default: launch_stream_sb<MR, 4, 0>(p, grid, stream); break;
    }
}

// ---------------------------------------------------------------------------
// 2 <= M <= 16 on the matrix cores: the single-row GEMV's structure (16 * CB
// column tiles, K splits, 8 waves on whole batches of 32-K steps, two
// batches in flight per wave, XCD-contiguous tiles, last-split combine) with
// the A operand now 16 activation rows. A lane streams its own 16 bytes of
// the activation per step (row l & 15, K quarter l >> 4; L2-resident, shared
// by every tile) beside the weight words, so there is no staging. The words
// are dequantised to exact fp16 codes, the step products accumulate in fp32
// per scale group (MFMA accumulator) and are scaled at each group's end.
// Rows >= M read zeros. The waves' [16 x TN] results are added in LDS.
// ---------------------------------------------------------------------------
template <int CB, int GSHIFT>
struct Gemv16Batch {
    static constexpr int SB = kGemvBatch;
    static constexpr int NG = SB >> GSHIFT;
    static constexpr int SW = (CB + 1) / 2;
    typename UIntVec<CB>::T w[SB];
    u32x4 a[SB];
    typename UIntVec<SW>::T s[NG];
    __device__ __forceinline__ void load(const GemmParams& p, __amdgpu_buffer_rsrc_t rw,
                                         __amdgpu_buffer_rsrc_t rs, const uint16_t* arow, bool arow_ok,
                                         uint32_t w_off, uint32_t s_off, uint32_t step_bytes,
                                         uint32_t grp_bytes, int step0, int last_step, int last_grp) {
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            // Steps past the split re-read its last step (in bounds) with a
            // zero activation, so they add exactly 0.
            const int st = min(step0 + j, last_step);
            w[j] = buffer_load_words<CB>(rw, w_off, (uint32_t)st * step_bytes);
            const u32x4 v = load16(arow + 32 * st);
            a[j] = (arow_ok && step0 + j <= last_step) ? v : u32x4{0u, 0u, 0u, 0u};
        }
        const int g0 = step0 >> p.gshift;
#pragma unroll
        for (int u = 0; u < NG; ++u) {
            const uint32_t so = (uint32_t)min(g0 + u, last_grp) * grp_bytes;
            if constexpr (CB == 1) s[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)s_off, (int)so, 0);
            else s[u] = buffer_load_words<SW>(rs, s_off, so);
        }
    }
    __device__ __forceinline__ float scale(int u, int cb) const {
        uint32_t d;
        if constexpr (CB == 1) d = s[u];
        else d = word_of<SW>(s[u], cb >> 1);
        return h2f((uint16_t)((cb & 1) ? (d >> 16) : d));
    }
};

template <int CB, int GSHIFT, bool MULTI>
__global__ __launch_bounds__(kGemvThreads) void w4a16_gemv16_kernel(GemmParams p) {
    constexpr int SB = kGemvBatch;
    constexpr int TN = 16 * CB;
    constexpr int SPG = 1 << GSHIFT;   // steps per group inside a batch (GSHIFT <= log2 SB)
    __shared__ float s_red[kGemvWaves][16][TN + 1];
    __shared__ uint32_t s_last;

    int b = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
    const int tile = b % p.n_tiles;
    const int split = b / p.n_tiles;

    const int steps = p.K / 32;
    const int sps = p.kp_per_split / 4;
    const int k0 = split * sps;
    const int nst = min(sps, steps - k0);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int kq = lane >> 4;
    const int n0 = tile * TN;
    const int col0 = n0 + CB * c;

    const int per_wave = sps / kGemvWaves;     // whole batches
    const int s0 = wave * per_wave;
    const int s1 = min(s0 + per_wave, nst);
    const int last = k0 + nst - 1;
    const int n_grp = p.K / p.group_size;
    const __amdgpu_buffer_rsrc_t rw = make_buffer_rsrc(p.w, (uint32_t)(p.K / 8) * p.N * 4u);
    const __amdgpu_buffer_rsrc_t rs = make_buffer_rsrc(p.scale, (uint32_t)n_grp * p.N * 2u);
    const uint32_t w_off = ((uint32_t)kq * p.N + col0) * 4u;
    const uint32_t s_off = (uint32_t)col0 * 2u;
    const uint32_t step_bytes = (uint32_t)p.N * 16u;
    const uint32_t grp_bytes = (uint32_t)p.N * 2u;
    const bool arow_ok = c < p.M;
    const uint16_t* arow = p.act + (long)min(c, p.M - 1) * p.K + 8 * kq;

    Gemv16Batch<CB, GSHIFT> ba, bb;
    ba.load(p, rw, rs, arow, arow_ok, w_off, s_off, step_bytes, grp_bytes, k0 + s0, last, n_grp - 1);
    if constexpr (MULTI)
        bb.load(p, rw, rs, arow, arow_ok, w_off, s_off, step_bytes, grp_bytes, k0 + s0 + SB, last,
                n_grp - 1);

    f32x4 acc[CB], cg[CB];
    const CodeMasks km = code_masks();
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
        acc[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        cg[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // Batches start on multiples of SB steps and groups span SPG steps
    // (or the whole batch), so group ends fall at fixed batch offsets; a
    // batch's steps past the split carry zero activations.
    auto consume = [&](const Gemv16Batch<CB, GSHIFT>& bt) {
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const u32x4 a = bt.a[j];
            u32x4 r;
            r[0] = perm_b32(a[2], a[0], 0x05040100u);   // a0 a4
            r[1] = perm_b32(a[2], a[0], 0x07060302u);   // a1 a5
            r[2] = perm_b32(a[3], a[1], 0x05040100u);   // a2 a6
            r[3] = perm_b32(a[3], a[1], 0x07060302u);   // a3 a7
            const f16x8 aop = __builtin_bit_cast(f16x8, r);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                f16x2 wp[4];
                i4x8_to_f16_pairs(word_of<CB>(bt.w[j], cb), wp, km);
                f16x8 bop;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bop[2 * i] = wp[i][0];
                    bop[2 * i + 1] = wp[i][1];
                }
                cg[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, cg[cb], 0, 0, 0);
            }
            if ((j % SPG) == SPG - 1) {   // end of a group (or of the batch when groups are longer)
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    const float scv = bt.scale(j >> GSHIFT, cb);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[cb][i] = fmaf(scv, cg[cb][i], acc[cb][i]);
                    cg[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                }
            }
        }
    };
    if constexpr (!MULTI) {
        if (s0 < s1) consume(ba);
    } else if (s0 < s1) {
        for (int b0 = s0;; b0 += 2 * SB) {
            consume(ba);
            if (b0 + SB >= s1) break;
            ba.load(p, rw, rs, arow, arow_ok, w_off, s_off, step_bytes, grp_bytes, k0 + b0 + 2 * SB,
                    last, n_grp - 1);
            __builtin_amdgcn_sched_barrier(0);
            consume(bb);
            if (b0 + 2 * SB >= s1) break;
            bb.load(p, rw, rs, arow, arow_ok, w_off, s_off, step_bytes, grp_bytes, k0 + b0 + 3 * SB,
                    last, n_grp - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // C layout: lane (c, kq) holds rows 4kq..4kq+3 of MFMA cb's columns
    // (tile column CB * c + cb).
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_red[wave][4 * kq + i][CB * c + cb] = acc[cb][i];
    __syncthreads();
    const int t = threadIdx.x;
    const int row = t / TN, col = t % TN;   // 16 * TN <= kGemvThreads outputs, one per thread
    float v = 0.0f;
    const bool mine = t < 16 * TN && row < p.M;
    if (mine) {
#pragma unroll
        for (int w = 0; w < kGemvWaves; ++w) v += s_red[w][row][col];
    }
    if (p.splits == 1) {
        if (mine) store_out(p, row, n0 + col, v);
        return;
    }
    if (mine) publish_store(&p.part[((long)split * p.M + row) * p.N + n0 + col], v);
    publish_wait();
    __syncthreads();
    if (t == 0) s_last = arrive_last(&p.counters[tile], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    if (mine)
        store_out(p, row, n0 + col,
                  sum_splits(p.part + (long)row * p.N + n0 + col, (long)p.M * p.N, p.splits));
    if (t == 0) p.counters[tile] = 0u;
}

template <int CB, bool MULTI>
static void launch_gemv16_cb(const GemmParams& p, int grid, hipStream_t stream) {
    const dim3 g(grid), blk(kGemvThreads);
    switch (min(p.gshift, 3)) {
        case 0: hipLaunchKernelGGL((w4a16_gemv16_kernel<CB, 0, MULTI>), g, blk, 0, stream, p); break;
        case 1: hipLaunchKernelGGL((w4a16_gemv16_kernel<CB, 1, MULTI>), g, blk, 0, stream, p); break;
        case 2: hipLaunchKernelGGL((w4a16_gemv16_kernel<CB, 2, MULTI>), g, blk, 0, stream, p); break;
        default: hipLaunchKernelGGL((w4a16_gemv16_kernel<CB, 3, MULTI>), g, blk, 0, stream, p); break;
    }
}

// ---------------------------------------------------------------------------
// M >= 2 on the matrix cores (N % 64 == 0, group_size a power of two >= 32).
//
// A workgroup of 4 waves computes a tile of TM = 16 * RT rows by 64 columns
// over one K split; wave w owns the 16-column block n0 + 16w. For each 32-K
// step a lane dequantises one packed word (column n0 + 16w + (l & 15),
// packed row 4 * step + (l >> 4)) to exact fp16 codes and feeds it as the B
// operand to RT MFMAs, one per 16-row tile of the activation. The
// activation rows of a chunk of KC steps are staged once per workgroup in
// LDS, in the pair order of the dequantised word, and read by all four
// waves; the next chunk is loaded into registers while the current one is
// consumed. The step products accumulate in fp32 per scale group and are
// scaled at the end of each group: acc += scale[g][n] * C_group.
// ---------------------------------------------------------------------------
constexpr int kMmaThreads = 256;

template <int RT>
struct MmaShape {
    static constexpr int TM = 16 * RT;
    static constexpr int KC = (RT >= 8) ? 4 : (RT >= 4 ? 8 : 16);   // steps per LDS chunk
    static constexpr int A_LOADS = TM * KC * 4 / kMmaThreads;      // 16-byte loads per thread
};

template <int RT>
__global__ __launch_bounds__(kMmaThreads) void w4a16_gemm_mfma_kernel(GemmParams p) {
    using S = MmaShape<RT>;
    constexpr int TM = S::TM, KC = S::KC;
    __shared__ __attribute__((aligned(16))) uint16_t s_a[KC][TM][32];
    __shared__ uint32_t s_last;

    // (tile, split, m-tile) from an XCD-contiguous order of workgroup ids.
    int b = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
    const int tile = b % p.n_tiles;
    const int rest = b / p.n_tiles;
    const int split = rest % p.splits;
    const int mtile = rest / p.splits;

    const int steps = p.K / 32;
    const int sps = p.kp_per_split / 4;
    const int k0 = split * sps;
    const int nst = min(sps, steps - k0);
    const int m0 = mtile * TM;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int kq = lane >> 4;
    const int n0 = tile * 64;
    const int n = n0 + 16 * wave + c;

    const int n_grp = p.K / p.group_size;
    const int spg_mask = (1 << p.gshift) - 1;   // steps per group - 1
    const __amdgpu_buffer_rsrc_t rw = make_buffer_rsrc(p.w, (uint32_t)(p.K / 8) * p.N * 4u);
    const __amdgpu_buffer_rsrc_t rs = make_buffer_rsrc(p.scale, (uint32_t)n_grp * p.N * 2u);
    const uint32_t w_off = ((uint32_t)kq * p.N + n) * 4u;
    const uint32_t s_off = (uint32_t)n * 2u;
    const uint32_t step_bytes = (uint32_t)p.N * 16u;
    const uint32_t grp_bytes = (uint32_t)p.N * 2u;
    const int last = k0 + nst - 1;

    // Activation chunk loads of this thread: chunk i covers steps
    // [k0 + i*KC, ...); slot j -> (step, row, 8-value quarter).
    u32x4 areg[S::A_LOADS];
    auto load_a = [&](int chunk) {
#pragma unroll
        for (int j = 0; j < S::A_LOADS; ++j) {
            const int idx = threadIdx.x + j * kMmaThreads;
            const int st = idx / (TM * 4);
            const int row = (idx >> 2) % TM;
            const int qq = idx & 3;
            const int gst = chunk * KC + st;            // step within the split
            const int m = m0 + row;
            const bool ok = (gst < nst) && (m < p.M);
            const long off = (long)min(m, p.M - 1) * p.K + 32L * (k0 + min(gst, nst - 1)) + 8 * qq;
            const u32x4 v = load16(p.act + off);
            areg[j] = ok ? v : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store_a = [&]() {
#pragma unroll
        for (int j = 0; j < S::A_LOADS; ++j) {
            const int idx = threadIdx.x + j * kMmaThreads;
            const int st = idx / (TM * 4);
            const int row = (idx >> 2) % TM;
            const int qq = idx & 3;
            const u32x4 a = areg[j];
            u32x4 r;
            r[0] = perm_b32(a[2], a[0], 0x05040100u);   // a0 a4
            r[1] = perm_b32(a[2], a[0], 0x07060302u);   // a1 a5
            r[2] = perm_b32(a[3], a[1], 0x05040100u);   // a2 a6
            r[3] = perm_b32(a[3], a[1], 0x07060302u);   // a3 a7
            *reinterpret_cast<u32x4*>(&s_a[st][row][8 * qq]) = r;
        }
    };
    // Weight words and scales of a chunk (clamped to the split: in bounds).
    struct WChunk {
        uint32_t w[KC];
        uint32_t sc[KC];
    };
    auto load_w = [&](WChunk& wc, int chunk) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int gs = min(k0 + chunk * KC + j, last);
            wc.w[j] = buffer_stream4(rw, w_off, (uint32_t)gs * step_bytes);
            wc.sc[j] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)s_off,
                                                            (int)((uint32_t)(gs >> p.gshift) * grp_bytes), 0);
        }
    };

    f32x4 acc[RT], cg[RT];
    const CodeMasks km = code_masks();
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        acc[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        cg[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const int n_chunks = (nst + KC - 1) / KC;
    WChunk wa, wb;
    load_a(0);
    load_w(wa, 0);
    auto compute = [&](const WChunk& wc, int chunk) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int sl = chunk * KC + j;              // step within the split
            if (sl < nst) {
                f16x2 wp[4];
                i4x8_to_f16_pairs(wc.w[j], wp, km);
                f16x8 bop;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bop[2 * i] = wp[i][0];
                    bop[2 * i + 1] = wp[i][1];
                }
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                    const f16x8 aop = __builtin_bit_cast(
                        f16x8, *reinterpret_cast<const u32x4*>(&s_a[j][16 * r + c][8 * kq]));
                    cg[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, cg[r], 0, 0, 0);
                }
                const int gst = k0 + sl;
                if (((gst & spg_mask) == spg_mask) || sl == nst - 1) {   // end of a scale group
                    const float scv = h2f((uint16_t)wc.sc[j]);
#pragma unroll
                    for (int r = 0; r < RT; ++r) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(scv, cg[r][i], acc[r][i]);
                        cg[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    }
                }
            }
        }
    };
    for (int ch = 0; ch < n_chunks; ch += 2) {
        __syncthreads();                 // previous chunk's reads of s_a are done
        store_a();
        __syncthreads();
        if (ch + 1 < n_chunks) {
            load_a(ch + 1);
            load_w(wb, ch + 1);
        }
        compute(wa, ch);
        if (ch + 1 >= n_chunks) break;
        __syncthreads();
        store_a();
        __syncthreads();
        if (ch + 2 < n_chunks) {
            load_a(ch + 2);
            load_w(wa, ch + 2);
        }
        compute(wb, ch + 1);
    }

    // C layout: lane (c, kq) holds rows 4kq..4kq+3 of each 16-row tile, column n.
    auto out_index = [&](int r, int i) { return m0 + 16 * r + 4 * kq + i; };
    if (p.splits == 1) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (out_index(r, i) < p.M) store_out(p, out_index(r, i), n, acc[r][i]);
        return;
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (out_index(r, i) < p.M)
                publish_store(&p.part[((long)split * p.M + out_index(r, i)) * p.N + n], acc[r][i]);
    publish_wait();
    __syncthreads();
    const int counter = mtile * p.n_tiles + tile;
    if (threadIdx.x == 0) s_last = arrive_last(&p.counters[counter], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    // Last split: add the partials in split order. The loads of two splits
    // for all of this thread's outputs are issued together, so the combine
    // costs one memory round trip per two splits.
    constexpr int NO = RT * 4;
    float tot[NO];
#pragma unroll
    for (int o = 0; o < NO; ++o) tot[o] = 0.0f;
    for (int s0 = 0; s0 < p.splits; s0 += 2) {
        float v[2][NO];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const long sp = min(s0 + u, p.splits - 1);
#pragma unroll
            for (int o = 0; o < NO; ++o) {
                const int m = min(out_index(o >> 2, o & 3), p.M - 1);
                v[u][o] = publish_load(&p.part[(sp * p.M + m) * p.N + n]);
            }
        }
        // Padding slots add +0.0f (exact: tot is never -0); unconditional adds
        // keep both splits' loads ahead of the first use.
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int o = 0; o < NO; ++o) tot[o] += (s0 + u < p.splits) ? v[u][o] : 0.0f;
    }
#pragma unroll
    for (int o = 0; o < NO; ++o) {
        const int m = out_index(o >> 2, o & 3);
        if (m < p.M) store_out(p, m, n, tot[o]);
    }
    if (threadIdx.x == 0) p.counters[counter] = 0u;
}

// ---------------------------------------------------------------------------
// M > 16 on 32x32x16 matrix cores (plan kind 6; N % 128 == 0, group size a
// power of two >= 32, K % 32 == 0).
//
// A workgroup of 8 waves computes a tile of 64 rows by 128 columns over one
// K split. Wave w = 2 kg + ch owns columns 64 ch .. 64 ch + 63 of the tile,
// all 64 rows, and the kg-th of the split's 4 contiguous K ranges (whole
// scale groups where the split allows); the 4 partial tiles of a column half
// are added in LDS at the end in a fixed tree order.
//
// Activations. The two waves of a K range share its activation rows: per
// stage of two 32-K steps each loads 32 rows x 128 bytes with full-line
// 16-byte loads, permutes every 8 values to the pair order of the weight
// codes (i, i + 4) and writes them to the K range's LDS slot (row stride
// 144 bytes: the fragment reads of 8 consecutive rows hit distinct banks).
// A fragment of v_mfma_f32_32x32x16_f16 is then one 16-byte LDS read: lane
// (h = l / 32, c = l % 32) takes row 32 rb + c, K 16 kc + 8 h of the step.
// Stage s + 1 is loaded while stage s is computed (double-buffered slots).
//
// Weights. Lane (h, c) loads, per step and 16-K chunk kc, the 8-byte pair of
// words of columns 2c and 2c + 1 (packed row 4 st + 2 kc + h): the B
// fragments of two MFMAs whose 32 columns are 2c' + j (j = 0, 1). Words are
// held in a three-stage register ring, two stages ahead of their use. They
// become exact fp16 codes (i4x8_to_f16_pairs); products accumulate per
// scale group in fp32 (the group's first chunk starts from zero) and are
// scaled at the group's end:
//   acc += scale[g][n] * C_g.
// Each dequantised word serves the 64 rows of the tile.
// ---------------------------------------------------------------------------
constexpr int kG32RowHalves = 72;
constexpr int kG32Waves = 8;
constexpr int kG32Threads = kG32Waves * kWave;
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct G32W {
    u32x2 w[2][2];     // [step][kc]: words of columns 2c, 2c + 1
    uint32_t s[2];     // [step]: scales of columns 2c, 2c + 1
};

__global__ __launch_bounds__(kG32Threads) void w4a16_gemm_mfma32_kernel(GemmParams p) {
    constexpr int TM = 64;
    constexpr int KG = 4;
    __shared__ __attribute__((aligned(16))) uint16_t s_a[KG][2][TM][kG32RowHalves];   // 72 KiB
    __shared__ uint32_t s_last;

    // (m-tile, split, tile) from an XCD-contiguous order of workgroup ids
    // (the dispatcher deals ids to the 8 XCDs round robin): the m-tiles and
    // K splits of a column tile are neighbours, so they share its weights in
    // one XCD's L2, and, when the column tiles are a multiple of 8, the
    // splits that hand partials to each other run on one XCD. Against splits
    // outermost (each split's tiles on their own XCDs), M=128 (4096, 4096)
    // 19.9-20.6 -> 15.8-16.3 us, M=64 18.4 -> 14.8 us. The hand-off stays
    // coherent across XCDs, so nothing depends on where the workgroups run.
    int bid = blockIdx.x;
    const int nwg = gridDim.x;
    if ((nwg & 7) == 0) bid = (bid & 7) * (nwg >> 3) + (bid >> 3);
    const int mtile = bid % p.m_tiles_;
    const int rest = bid / p.m_tiles_;
    const int split = rest % p.splits;
    const int tile = rest / p.splits;
    const int counter = tile * p.m_tiles_ + mtile;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ch = wave & 1;
    const int kg = wave >> 1;
    const int c = lane & 31;
    const int h = lane >> 5;

    const int steps = p.K / 32;
    const int sps = p.kp_per_split / 4;
    const int k0 = split * sps;
    const int nst = min(sps, steps - k0);
    const int ws0 = k0 + min(kg * p.wave_steps, nst);
    const int ws1 = k0 + min((kg + 1) * p.wave_steps, nst);
    const int n0 = tile * 128 + 64 * ch;
    const int m0 = mtile * TM;
    const int n_grp = p.K / p.group_size;
    const int spg_mask = (1 << p.gshift) - 1;

    const __amdgpu_buffer_rsrc_t rw = make_buffer_rsrc(p.w, (uint32_t)(p.K / 8) * p.N * 4u);
    const __amdgpu_buffer_rsrc_t ra = make_buffer_rsrc(p.act, (uint32_t)p.M * p.K * 2u);
    const __amdgpu_buffer_rsrc_t rs = make_buffer_rsrc(p.scale, (uint32_t)n_grp * p.N * 2u);
    const uint32_t w_off = ((uint32_t)h * p.N + n0 + 2 * c) * 4u;
    const uint32_t w_kc = (uint32_t)p.N * 8u;    // bytes between the packed rows of two chunks
    const uint32_t w_step = (uint32_t)p.N * 16u;
    const uint32_t s_off = (uint32_t)(n0 + 2 * c) * 2u;
    const uint32_t grp_bytes = (uint32_t)p.N * 2u;
    // Activation staging: this wave loads rows 32 ch + (l >> 3) + 8 i of the
    // stage, 16-byte column q = l & 7 (rows past M point beyond the buffer
    // bound and load zeros).
    const int q = lane & 7;
    uint32_t a_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 32 * ch + (lane >> 3) + 8 * i;
        a_off[i] = (row < p.M) ? ((uint32_t)row * p.K + 8u * q) * 2u : 0x80000000u;
    }

    // Steps past the wave's range re-read its last step (in bounds) and are
    // never consumed.
    auto clamp_step = [&](int st) { return (uint32_t)max(min(st, ws1 - 1), 0); };
    auto load_w = [&](G32W& t, int st0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t st = clamp_step(st0 + j);
#pragma unroll
            for (int kc = 0; kc < 2; ++kc)
                t.w[j][kc] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                    rw, (int)(w_off + kc * w_kc), (int)(st * w_step), 2));
            t.s[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)s_off,
                                                          (int)((st >> p.gshift) * grp_bytes), 0);
        }
    };
    u32x4 areg[4];
    auto load_a = [&](int st0) {
        const uint32_t st = clamp_step(st0);   // a stage starts at an even step of the range
#pragma unroll
        for (int i = 0; i < 4; ++i)
            areg[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, (int)a_off[i], (int)(st * 64u), 0);
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 a = areg[i];
            const u32x4 r = make_u32x4(perm_b32(a[2], a[0], 0x05040100u), perm_b32(a[2], a[0], 0x07060302u),
                                       perm_b32(a[3], a[1], 0x05040100u), perm_b32(a[3], a[1], 0x07060302u));
            *reinterpret_cast<u32x4*>(&s_a[kg][buf][32 * ch + (lane >> 3) + 8 * i][8 * q]) = r;
        }
    };

    f32x16 acc[2][2], cg[2][2];
    const CodeMasks km = code_masks();
    const f32x16 zero16 = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f,
                           0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[rb][j] = zero16;
            cg[rb][j] = zero16;
        }

    auto compute = [&](const G32W& t, int buf, int st0) {
#pragma unroll
        for (int js = 0; js < 2; ++js) {
            const int st = st0 + js;
            if (st >= ws1) break;   // wave-uniform
            // The first chunk of a scale group starts its accumulators from
            // zero (an inline-zero C operand), so nothing is cleared at the
            // group's end.
            const bool first = ((st & spg_mask) == 0) || st == ws0;
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
                f16x8 bop[2], aop[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    f16x2 wp[4];
                    i4x8_to_f16_pairs(t.w[js][kc][j], wp, km);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        bop[j][2 * i] = wp[i][0];
                        bop[j][2 * i + 1] = wp[i][1];
                    }
                }
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
                    aop[rb] = __builtin_bit_cast(f16x8, *reinterpret_cast<const u32x4*>(
                        &s_a[kg][buf][32 * rb + c][32 * js + 16 * kc + 8 * h]));
                if (kc == 0 && first) {
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            cg[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[rb], bop[j], zero16, 0, 0, 0);
                } else {
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            cg[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[rb], bop[j], cg[rb][j], 0, 0, 0);
                }
            }
            if (((st & spg_mask) == spg_mask) || st == ws1 - 1) {   // end of a scale group
                const float s0 = h2f((uint16_t)t.s[js]);
                const float s1 = h2f((uint16_t)(t.s[js] >> 16));
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[rb][0][r] = fmaf(s0, cg[rb][0][r], acc[rb][0][r]);
                        acc[rb][1][r] = fmaf(s1, cg[rb][1][r], acc[rb][1][r]);
                    }
            }
        }
    };

    // Stage loop: every wave runs the same number of stages (the longest K
    // range of the workgroup) so that the barriers match; a wave whose range
    // is shorter or empty computes nothing in the extra stages.
    const int n_stages = (p.wave_steps + 1) / 2;
    {
        G32W wr[3];
        load_w(wr[0], ws0);
        load_w(wr[1], ws0 + 2);
        load_a(ws0);
        __builtin_amdgcn_sched_barrier(0);
        store_a(0);
        load_a(ws0 + 2);
        __syncthreads();
        // One pass of the unrolled body handles stages s, s + 1, s + 2 with
        // ring slots 0, 1, 2 and LDS buffers alternating from `buf`.
        // The stage's MFMAs at raised wave priority (as in the LDS-staged
        // GEMM): same bits, 0-3 % faster on one box (M=128 (4096, 14336)
        // 24.92 -> 24.50 us, M=512 (4096, 4096) 25.53 -> 24.79).
        auto stage = [&](G32W& cur, G32W& ahead2, int s, int buf) {
            load_w(ahead2, ws0 + 2 * (s + 2));
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            compute(cur, buf, ws0 + 2 * s);
            __builtin_amdgcn_s_setprio(0);
            store_a(buf ^ 1);          // stage s + 1, loaded during stage s - 1 / the prologue
            load_a(ws0 + 2 * (s + 2));
            __syncthreads();
        };
        int s = 0;
        int buf = 0;
        while (true) {
            if (s >= n_stages) break;
            stage(wr[0], wr[2], s, buf); ++s; buf ^= 1;
            if (s >= n_stages) break;
            stage(wr[1], wr[0], s, buf); ++s; buf ^= 1;
            if (s >= n_stages) break;
            stage(wr[2], wr[1], s, buf); ++s; buf ^= 1;
        }
    }

    // Add the 4 K-range tiles of each column half (waves kg in [half, 2 half)
    // hand theirs to kg - half) through LDS, reusing the activation slots.
    float* s_red = reinterpret_cast<float*>(&s_a[0][0][0][0]);   // [2][2][64 values][64 lanes]
    constexpr int kVals = 2 * 2 * 16;
#pragma unroll
    for (int half = KG / 2; half >= 1; half /= 2) {
        if (kg >= half && kg < 2 * half) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        s_red[(((kg - half) * 2 + ch) * kVals + (rb * 2 + j) * 16 + r) * kWave + lane] =
                            acc[rb][j][r];
        }
        __syncthreads();
        if (kg < half) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        acc[rb][j][r] += s_red[((kg * 2 + ch) * kVals + (rb * 2 + j) * 16 + r) * kWave + lane];
        }
        __syncthreads();
    }

    // The workgroup's tile (held by the kg == 0 waves) goes through LDS to
    // row-major order; thread t then owns columns 4 (t % 32) .. + 3 of rows
    // t / 32 + 16 i (i < 4), so that every 16-byte access instruction covers
    // whole rows (32 lanes x 16 bytes): the split partials, their combine and
    // the output. C layout of v_mfma_f32_32x32x16: value r of lane l is row
    // 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of the block.
    constexpr int kTRow = 132;   // floats per LDS row (128 + 4 of padding)
    float* s_t = reinterpret_cast<float*>(&s_a[0][0][0][0]);   // [TM][kTRow]
    if (kg == 0) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 32 * rb + 8 * (r >> 2) + 4 * h + (r & 3);
                *reinterpret_cast<f32x2*>(&s_t[row * kTRow + 64 * ch + 2 * c]) =
                    f32x2{acc[rb][0][r], acc[rb][1][r]};
            }
    }
    __syncthreads();
    const int tcol = 4 * (threadIdx.x & 31);
    const int nt0 = tile * 128;
    f32x4 v[4];
    int mi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = (threadIdx.x >> 5) + 16 * i;
        mi[i] = m0 + row;
        v[i] = *reinterpret_cast<const f32x4*>(&s_t[row * kTRow + tcol]);
    }
    if (p.splits == 1) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (mi[i] < p.M) store_out4(p, mi[i], nt0 + tcol, v[i]);
        return;
    }
    const uint32_t slab = (uint32_t)p.M * p.N * 4u;   // bytes per split (plan: < 2 GiB)
    uint32_t off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) off[i] = ((uint32_t)min(mi[i], p.M - 1) * p.N + nt0 + tcol) * 4u;
    {
        const __amdgpu_buffer_rsrc_t rp = make_buffer_rsrc(p.part + (long)split * p.M * p.N, slab);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (mi[i] < p.M) publish_store16(rp, off[i], __builtin_bit_cast(u32x4, v[i]));
    }
    publish_wait();
    __syncthreads();
    if (threadIdx.x == 0) s_last = arrive_last(&p.counters[counter], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    // Last split of the tile: the partials are added in split order, with the
    // loads of two splits issued together. The padding slot adds +0.0f, an
    // exact no-op (the sum starts at +0 and is never -0); the unconditional
    // add keeps both batches' loads ahead of the first use.
    f32x4 tot[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) tot[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < p.splits; s0 += 2) {
        u32x4 x[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int sp = min(s0 + u, p.splits - 1);
            const __amdgpu_buffer_rsrc_t rp = make_buffer_rsrc(p.part + (long)sp * p.M * p.N, slab);
            if (sp == split) {   // this workgroup's own partial, the same bits it stored
#pragma unroll
                for (int i = 0; i < 4; ++i) x[u][i] = __builtin_bit_cast(u32x4, v[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) x[u][i] = publish_load16(rp, off[i]);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const bool live = s0 + u < p.splits;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t b = x[u][i][e];
                    tot[i][e] += live ? __uint_as_float(b) : 0.0f;
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (mi[i] < p.M) store_out4(p, mi[i], nt0 + tcol, tot[i]);
    if (threadIdx.x == 0) p.counters[counter] = 0u;
}

// ---------------------------------------------------------------------------
// M >= 256 on 32x32x16 matrix cores (plan kind 7; N % 128 == 0, K % 64 == 0,
// group size a power of two >= 32).
//
// A workgroup of 8 waves computes a tile of 256 rows by 128 columns over one
// K split, in stages of 64 K, with both operands in LDS as fp16 rows of 128
// bytes (64 K values). The 16-byte chunk j of row r sits in slot j ^ (r % 8)
// of the row, so the fragment reads of 8 consecutive rows (same chunk) and
// the chunk stores of 8 consecutive rows hit distinct banks.
//   * Activations go from memory straight into LDS (buffer_load ... lds, 1
//     KiB of 8 swizzled rows per instruction, four per wave per stage; rows
//     past M read zeros) into a three-slot ring, two stages ahead.
//   * Weight words (the stage's 8 packed rows x 128 columns, two per thread)
//     and group scales are loaded into registers two stages ahead. After a
//     stage's MFMAs the words of the next stage are dequantised once for
//     the whole workgroup into the exact fp16 codes of their 8 K positions
//     in K order (i4x8_to_f16_natural) and stored as their columns' chunks
//     of the next stage's slot (two slots).
// Wave w computes rows 64 (w % 4) .. + 63 and columns 64 (w / 4) .. + 63 as
// 2 x 2 blocks of v_mfma_f32_32x32x16_f16; an A or B fragment is one 16-byte
// LDS read (lane (h, c): row / column 32 blk + c, chunk 2 kc + h of the
// stage), read one chunk ahead of its MFMAs. Products accumulate per scale
// group in fp32 from a zero C operand and are scaled at the group's end,
// acc += scale[g][n] * C_g, so no weight is rounded. One barrier per stage.
// Against the 64 x 128 tiles of kind 6 each weight word is dequantised once
// per 256 rows instead of once per 64, and the activations are neither
// permuted nor staged through registers.
// ---------------------------------------------------------------------------
constexpr int kL7TN = 128;
constexpr int kL7TM = 256;
constexpr int kL7Waves = 8;
constexpr int kL7Threads = kL7Waves * kWave;
// LDS-staged GEMM: m-tiles per group in the order of unsplit tiles (0: all
// of them, i.e. m-tile fastest). With 2, one XCD's 32 concurrent
// workgroups cover 2 m-tiles x 16 column tiles instead of 8 x 4 (M = 2048),
// so each XCD streams a quarter of the activation rows: measured on one box
// against 0, M=3072 (4096, 14336) 433.9 -> 419.3 us, M=4096 579.6 -> 545.4,
// M <= 2048 within 1.5 % (1 and 4: 421.9 / 548.3 and 423.4 / 545.9).
#ifndef LLMIK_L7_GM
#define LLMIK_L7_GM 2
#endif

// Eight int4 codes of one word -> four fp16 pairs in K order, exact: pair i
// holds the codes of K positions (2i, 2i + 1). Byte i of the word (code 2i
// in bits 0-3, code 2i + 1 in bits 4-7) is copied to bytes 0 and 2; the mask
// m = 0x00F0000F keeps code 2i in bits 0-3 of the low half and code 2i + 1
// in bits 4-7 of the high half; x = 0x54806408 turns u = code + 8 (xor 8 per
// nibble) into 0x6400 | u = 1024 + u and 0x5400 | (u << 4) = 64 + u (the
// fp16 ulp at 64 is 1/16), and subtracting (1032, 72) leaves the codes.
// With m and x in VGPRs each pair is one v_perm, one v_bitop3 and one
// v_pk_add_f16.
__device__ __forceinline__ u32x4 i4x8_to_f16_natural(uint32_t w, uint32_t m, uint32_t x) {
    const f16x2 bias = {(f16)1032.0f, (f16)72.0f};
    u32x4 out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t b = perm_b32(0u, w, 0x0C000C00u | ((uint32_t)i << 16) | (uint32_t)i);
        out[i] = __builtin_bit_cast(uint32_t, as_f16x2((b & m) ^ x) - bias);
    }
    return out;
}

struct L7Words {
    uint32_t w[2];      // packed rows (t >> 7) + 4 j of column t & 127
    uint16_t s[2][2];   // [cb][u]: scales of the groups of chunks 1 and 3
};

// G32: group size 32 (two group ends per stage, four scale loads per lane
// per stage; otherwise one group end and two).
template <bool G32>
__global__ __launch_bounds__(kL7Threads) void w4a16_gemm_lds_kernel(GemmParams p) {
    constexpr int kLoads = 4 + 2 + (G32 ? 4 : 2);   // vector memory instructions per stage
    // Three separate activation slots: the copies into one slot and the
    // fragment reads of another are then known not to alias, so the reads
    // do not wait for copies still in flight.
    __shared__ __attribute__((aligned(16))) uint8_t s_a0[kL7TM * 128];   // 3 x 32 KiB
    __shared__ __attribute__((aligned(16))) uint8_t s_a1[kL7TM * 128];
    __shared__ __attribute__((aligned(16))) uint8_t s_a2[kL7TM * 128];
    __shared__ __attribute__((aligned(16))) uint8_t s_b[2][kL7TN * 128];   // 32 KiB
    __shared__ uint32_t s_last;

    // Tiles are numbered m-tile fastest (tl = tile * m_tiles + mtile). The
    // first full_tiles workgroups (whole rounds of the CUs) compute tiles
    // 0 .. full_tiles - 1 over all of K, XCD-contiguously when that count is
    // a multiple of 8
    // (the dispatcher deals ids to the 8 XCDs round robin). The rest split
    // the K range of each remaining tile `splits` ways; they are dispatched
    // last and fill the final round. With full_tiles = 0 every tile is split
    // and the order is kind 6's (m-tiles, then splits, of a column tile
    // neighbours on one XCD). A split tile q (its rank among the split
    // tiles) owns counter q and partial slots q * splits .. + splits - 1.
    const int F = p.full_tiles;
    const int bx = blockIdx.x;
    // Unsplit tiles in groups of G m-tiles: index b -> (m-tile group, column
    // tile, m-tile in the group), so that consecutive indices (one XCD's
    // concurrent workgroups) cover G m-tiles of many column tiles.
    const int G = (LLMIK_L7_GM > 0 && p.m_tiles_ % LLMIK_L7_GM == 0) ? LLMIK_L7_GM : p.m_tiles_;
    auto tile_of = [&](int b, int& mt, int& nt) {
        const int mg = b / (G * p.n_tiles);
        const int r = b - mg * G * p.n_tiles;
        nt = r / G;
        mt = mg * G + (r - nt * G);
    };
    int mtile, tile, split, nsplit, q;
    if (bx < F) {
        const int b = ((F & 7) == 0) ? (bx & 7) * (F >> 3) + (bx >> 3) : bx;
        tile_of(b, mtile, tile);
        split = 0;
        nsplit = 1;
        q = 0;
    } else if (F == 0) {
        int b = bx;
        const int nwg = gridDim.x;
        if ((nwg & 7) == 0) b = (b & 7) * (nwg >> 3) + (b >> 3);
        if (p.splits == 1) {
            tile_of(b, mtile, tile);
            split = 0;
        } else {
            mtile = b % p.m_tiles_;
            const int rest = b / p.m_tiles_;
            split = rest % p.splits;
            tile = rest / p.splits;
        }
        nsplit = p.splits;
        q = tile * p.m_tiles_ + mtile;
    } else {
        const int b = bx - F;
        q = b / p.splits;
        split = b % p.splits;
        tile_of(F + q, mtile, tile);
        nsplit = p.splits;
    }

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave & 3;
    const int wn = wave >> 2;
    const int c = lane & 31;
    const int h = lane >> 5;

    const int stages = p.K / 64;
    const int st0 = nsplit == 1 ? 0 : split * p.wave_steps;   // wave_steps: stages per split
    const int st1 = nsplit == 1 ? stages : min(st0 + p.wave_steps, stages);
    const int m0 = mtile * kL7TM;
    const int n0 = tile * kL7TN;
    const int lcpg = p.gshift + 1;           // log2(16-K chunks per group)
    const int cpg_mask = (1 << lcpg) - 1;

    const __amdgpu_buffer_rsrc_t rw = make_buffer_rsrc(p.w, (uint32_t)(p.K / 8) * p.N * 4u);
    const __amdgpu_buffer_rsrc_t ra = make_buffer_rsrc(p.act, (uint32_t)p.M * p.K * 2u);
    const __amdgpu_buffer_rsrc_t rs = make_buffer_rsrc(p.scale, (uint32_t)(p.K / p.group_size) * p.N * 2u);
    // Activation copy: instruction i of wave w fills rows 8 (w + 8 i) .. + 7;
    // lane l writes slot l % 8 of row 8 (w + 8 i) + l / 8, i.e. chunk
    // (l % 8) ^ (l / 8) of that row. Rows past M point beyond the bound.
    uint32_t a_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = m0 + 8 * (wave + 8 * i) + (lane >> 3);
        a_off[i] = (row < p.M) ? ((uint32_t)row * p.K * 2u + 16u * (uint32_t)((lane & 7) ^ (lane >> 3)))
                               : 0x80000000u;
    }
    const int bn = t & 127;
    const int bk = t >> 7;
    const uint32_t w_off = ((uint32_t)bk * p.N + n0 + bn) * 4u;
    const uint32_t w_four = (uint32_t)p.N * 16u;   // 4 packed rows
    const uint32_t w_stage = (uint32_t)p.N * 32u;  // 8 packed rows
    const uint32_t s_off = (uint32_t)(n0 + 64 * wn + c) * 2u;
    const uint32_t grp_bytes = (uint32_t)p.N * 2u;
    const uint32_t km = vgpr_const(0x00F0000Fu);
    const uint32_t kx = vgpr_const(0x54806408u);

    // Loads for stage st (clamped into the split: a stage past it re-reads
    // the last one, in bounds, and is never used), always issued in full so
    // that every stage issues the same number of vector memory instructions.
    auto load_a = [&](uint8_t* slot, int st) {
        const uint32_t sc = (uint32_t)min(st, st1 - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (__attribute__((address_space(3))) void*)(slot + 1024 * (wave + 8 * i)), 16,
                (int)a_off[i], (int)(sc * 128u), 0, 0);
    };
    auto load_w = [&](L7Words& g, int st) {
        const int sc = min(st, st1 - 1);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            g.w[j] = __builtin_amdgcn_raw_buffer_load_b32(rw, (int)(w_off + j * w_four), (int)(sc * w_stage), 0);
#pragma unroll
        for (int u = G32 ? 0 : 1; u < 2; ++u) {
            const uint32_t grp = (uint32_t)((4 * sc + 1 + 2 * u) >> lcpg);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
                g.s[cb][u] = __builtin_amdgcn_raw_buffer_load_b16(rs, (int)(s_off + 64u * cb),
                                                                  (int)(grp * grp_bytes), 0);
        }
    };
    auto store_w = [&](const L7Words& g, int st) {
        uint8_t* slot = &s_b[(st - st0) & 1][0];
#pragma unroll
        for (int j = 0; j < 2; ++j)
            *reinterpret_cast<u32x4*>(slot + bn * 128 + 16 * ((bk + 4 * j) ^ (bn & 7))) =
                i4x8_to_f16_natural(g.w[j], km, kx);
    };

    f32x16 acc[2][2], cg[2][2];
    const f32x16 zero16 = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f,
                           0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
            acc[rb][cb] = zero16;
            cg[rb][cb] = zero16;
        }
    const int ra_row0 = 64 * wm + c;   // + 32 rb; rows and columns are = c (mod 8)
    const int rb_col0 = 64 * wn + c;   // + 32 cb
    const int sw = c & 7;

    // One stage: chunk kk = 4 st + kc starts a scale group (or the split)
    // only at even kc and ends one only at odd kc (groups are >= 2 chunks,
    // splits whole stages); at kc = 1 only when the group is 32.
    auto compute = [&](const uint8_t* sa, int st, const uint16_t (&scl)[2][2]) {
        const uint8_t* sb = &s_b[(st - st0) & 1][0];
        f16x8 aop[2][2], bop[2][2];   // [parity of kc][block]
        auto read_frags = [&](int kc) {
            const int slot = 16 * ((2 * kc + h) ^ sw);
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
                aop[kc & 1][rb] = __builtin_bit_cast(
                    f16x8, *reinterpret_cast<const u32x4*>(sa + (ra_row0 + 32 * rb) * 128 + slot));
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
                bop[kc & 1][cb] = __builtin_bit_cast(
                    f16x8, *reinterpret_cast<const u32x4*>(sb + (rb_col0 + 32 * cb) * 128 + slot));
        };
        read_frags(0);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
            const int kk = 4 * st + kc;
            if (kc < 3) read_frags(kc + 1);
            const int x = kc & 1;
            if ((kc & 1) == 0 && (((kk & cpg_mask) == 0) || kk == 4 * st0)) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
                        cg[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[x][rb], bop[x][cb], zero16, 0, 0, 0);
            } else {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
                        cg[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(aop[x][rb], bop[x][cb], cg[rb][cb], 0, 0, 0);
            }
            if ((kc == 3 || (G32 && kc == 1)) && (((kk & cpg_mask) == cpg_mask) || kk == 4 * st1 - 1)) {
                const float s0 = h2f(scl[0][kc >> 1]);
                const float s1 = h2f(scl[1][kc >> 1]);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[rb][0][r] = fmaf(s0, cg[rb][0][r], acc[rb][0][r]);
                        acc[rb][1][r] = fmaf(s1, cg[rb][1][r], acc[rb][1][r]);
                    }
            }
        }
    };

    // Prologue: stages st0 and st0 + 1 in flight, st0's weights dequantised.
    // In the loop, stage st issues stage st + 2's loads, runs its MFMAs,
    // dequantises and stores stage st + 1's words, and before its barrier
    // waits for every load but the ones it issued itself (stage st + 1's
    // activations are then in LDS).
    L7Words wcur, wnext, wfar;   // stages st, st + 1, st + 2
    load_a(s_a0, st0);
    load_w(wcur, st0);
    load_a(s_a1, st0 + 1);
    load_w(wnext, st0 + 1);
    store_w(wcur, st0);
    __builtin_amdgcn_s_waitcnt(kLoads | 0x0F70);   // vmcnt(kLoads): stage st0's loads are complete
    __syncthreads();
    // Stage st reads activation slot (st - st0) % 3 and fills slot
    // (st - st0 + 2) % 3; the loop is unrolled by three so that every slot
    // is a fixed array.
    auto stage = [&](uint8_t* cur, uint8_t* far, int st) {
        load_a(far, st + 2);
        load_w(wfar, st + 2);
        __builtin_amdgcn_sched_barrier(0);
        const bool more = st + 1 < st1;   // workgroup-uniform
        // The MFMAs at raised wave priority, so that a SIMD's other wave's
        // dequantisation and stores yield to them: same bits, 0.7-2 % faster
        // at M = 512 .. 4096 on one box (M=2048 (14336, 4096) 245.5 ->
        // 243.9 us, M=4096 (4096, 14336) 509.0 -> 504.2).
        __builtin_amdgcn_s_setprio(1);
        compute(cur, st, wcur.s);
        __builtin_amdgcn_s_setprio(0);
        if (more) store_w(wnext, st + 1);
        // Every load but this stage's kLoads (4 copies, 2 words, the scales)
        // is complete, so stage st + 1's activations are in LDS, and this
        // wave's weight chunk stores are done; then the workgroup barrier. A
        // bare s_barrier: __syncthreads' release fence would also wait for
        // the copies of stage st + 2 issued above. The memory clobber keeps
        // the compiler from moving LDS accesses across it.
        __builtin_amdgcn_s_waitcnt(kLoads | (7 << 4));   // vmcnt(kLoads) lgkmcnt(0)
        asm volatile("s_barrier" ::: "memory");
        wcur = wnext;
        wnext = wfar;
    };
    for (int st = st0; st < st1; st += 3) {
        stage(s_a0, s_a2, st);
        if (st + 1 >= st1) break;
        stage(s_a1, s_a0, st + 1);
        if (st + 2 >= st1) break;
        stage(s_a2, s_a1, st + 2);
    }
    __builtin_amdgcn_s_waitcnt(0);   // the loads past the split land before the LDS is reused

    // C layout of v_mfma_f32_32x32x16: value r of lane l is row 8 (r / 4) +
    // 4 (l / 32) + r % 4, column l % 32 of the block. The epilogue uses buffer
    // accesses bounded by M rows: stores to rows past M are dropped and loads
    // from them return zeros, so no access needs a row test.
    const uint32_t esz = p.f32_out ? 4u : 2u;
    const __amdgpu_buffer_rsrc_t ro = make_buffer_rsrc(p.out, (uint32_t)p.M * p.N * esz);   // plan: M N 4 < 2^31
    uint32_t eoff[2];                            // element offset of value r = 0 of block row rb
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) eoff[rb] = (uint32_t)(m0 + 64 * wm + 32 * rb + 4 * h) * p.N + n0 + 64 * wn + c;
    auto roff = [&](int r) { return (uint32_t)(8 * (r >> 2) + (r & 3)) * p.N; };
    auto store_res = [&](int rb, int cb, int r, float v) {
        const uint32_t e = eoff[rb] + roff(r) + 32 * cb;
        if (p.f32_out) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ro, (int)(e * 4u), 0, 0);
        else __builtin_amdgcn_raw_buffer_store_b16(f2h_bits(v), ro, (int)(e * 2u), 0, 0);
    };
    if (nsplit == 1) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int r = 0; r < 16; ++r) store_res(rb, cb, r, acc[rb][cb][r]);
        return;
    }
    // Split partials in the threads' own fragment layout: four-value group j
    // (acc[rb][cb][4 jj .. 4 jj + 3], j = 4 (2 rb + cb) + jj) of thread t
    // sits at float offset 4 (512 j + t) of the tile's slot, so every access
    // instruction moves 16 bytes per lane, contiguous across the lanes, and
    // the last arriver's thread t reads back exactly the values it adds.
    constexpr uint32_t kTileElems = kL7TM * kL7TN;
    auto part_rsrc = [&](int sp) {
        return make_buffer_rsrc(p.part + ((long)q * nsplit + sp) * kTileElems, kTileElems * 4u);
    };
    auto grp_off = [&](int rb, int cb, int jj) {
        return (uint32_t)((4 * (2 * rb + cb) + jj) * kL7Threads + t) * 16u;
    };
    {
        const __amdgpu_buffer_rsrc_t rp = part_rsrc(split);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    publish_store16(rp, grp_off(rb, cb, jj),
                                    u32x4{__float_as_uint(acc[rb][cb][4 * jj]), __float_as_uint(acc[rb][cb][4 * jj + 1]),
                                          __float_as_uint(acc[rb][cb][4 * jj + 2]), __float_as_uint(acc[rb][cb][4 * jj + 3])});
    }
    publish_wait();
    __syncthreads();
    if (t == 0) s_last = arrive_last(&p.counters[q], (uint32_t)nsplit) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
    // Last split of the tile: the partials are added in split order (this
    // workgroup's own from registers, the same bits it stored), each split's
    // 64 values per thread loaded together.
    f32x16 tot[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) tot[rb][cb] = zero16;
    for (int sp = 0; sp < nsplit; ++sp) {
        if (sp == split) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int cb = 0; cb < 2; ++cb) tot[rb][cb] += acc[rb][cb];
            continue;
        }
        const __amdgpu_buffer_rsrc_t rp = part_rsrc(sp);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const u32x4 v = publish_load16(rp, grp_off(rb, cb, jj));
#pragma unroll
                    for (int e = 0; e < 4; ++e) cg[rb][cb][4 * jj + e] = __uint_as_float(v[e]);
                }
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) tot[rb][cb] += cg[rb][cb];
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int r = 0; r < 16; ++r) store_res(rb, cb, r, tot[rb][cb][r]);
    if (t == 0) p.counters[q] = 0u;
}

// ---------------------------------------------------------------------------
// M > 1: each lane owns COLS columns and MT rows; the weight is dequantised
// once per packed word into fp32 (code * scale, exact) and reused across the
// MT rows. Grid z walks the row tiles.
// ---------------------------------------------------------------------------
template <int COLS, int MT>
__global__ __launch_bounds__(kGemmThreads) void w4a16_gemm_tiled_kernel(GemmParams p) {
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int mtile = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = tile * (64 * COLS) + lane * COLS;
    const bool active = n0 < p.N;
    const int m0 = mtile * MT;
    const int mrows = min(MT, p.M - m0);

    const int kp_total = p.K / 8;
    const int kp_split0 = split * p.kp_per_split;
    const int kp_split1 = min(kp_split0 + p.kp_per_split, kp_total);
    const int per_wave = (p.kp_per_split + kGemmWaves - 1) / kGemmWaves;
    const int kp0 = min(kp_split0 + wave * per_wave, kp_split1);
    const int kp1 = min(kp0 + per_wave, kp_split1);
    const int kp_per_group = p.group_size / 8;

    float acc[MT][COLS];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < COLS; ++j) acc[m][j] = 0.0f;

    for (int kp = kp0; kp < kp1; ++kp) {
        const int g = kp / kp_per_group;
        float wf[COLS][8];
        if (active) {
#pragma unroll
            for (int j = 0; j < COLS; ++j) {
                const float s = h2f(p.scale[(long)g * p.N + n0 + j]);
                float codes[8];
                i4x8_to_f32(p.w[(long)kp * p.N + n0 + j], codes);
#pragma unroll
                for (int e = 0; e < 8; ++e) wf[j][e] = codes[e] * s;
            }
        } else {
#pragma unroll
            for (int j = 0; j < COLS; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) wf[j][e] = 0.0f;
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < mrows) {
                float a[8];
                f16x8_to_f32(load16(p.act + (long)(m0 + m) * p.K + 8 * kp), a);
#pragma unroll
                for (int j = 0; j < COLS; ++j)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[m][j] = fmaf(a[e], wf[j][e], acc[m][j]);
            }
        }
    }

    __shared__ float s_part[kGemmWaves][MT][64 * COLS];
    __shared__ uint32_t s_last;
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < COLS; ++j) s_part[wave][m][lane * COLS + j] = acc[m][j];
    __syncthreads();

    const int tile_n = 64 * COLS;
    const int nbase = tile * tile_n;
    const int outs = MT * tile_n;
    constexpr int kPer = (MT * 64 * COLS + kGemmThreads - 1) / kGemmThreads;
    float tot[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int idx = threadIdx.x + i * kGemmThreads;
        tot[i] = 0.0f;
        if (idx < outs) {
            const int m = idx / tile_n, col = idx % tile_n;
#pragma unroll
            for (int w = 0; w < kGemmWaves; ++w) tot[i] += s_part[w][m][col];
        }
    }
    const int counter = mtile * p.n_tiles + tile;
    if (p.splits == 1) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int idx = threadIdx.x + i * kGemmThreads;
            const int m = idx / tile_n, col = idx % tile_n;
            if (idx < outs && m < mrows && nbase + col < p.N) store_out(p, m0 + m, nbase + col, tot[i]);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int idx = threadIdx.x + i * kGemmThreads;
        const int m = idx / tile_n, col = idx % tile_n;
        if (idx < outs && m < mrows && nbase + col < p.N)
            publish_store(&p.part[((long)split * p.M + m0 + m) * p.N + nbase + col], tot[i]);
    }
    publish_wait();
    __syncthreads();
    if (threadIdx.x == 0) s_last = arrive_last(&p.counters[counter], (uint32_t)p.splits) ? 1u : 0u;
    __syncthreads();
    if (s_last == 0u) return;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int idx = threadIdx.x + i * kGemmThreads;
        const int m = idx / tile_n, col = idx % tile_n;
        if (idx < outs && m < mrows && nbase + col < p.N)
            store_out(p, m0 + m, nbase + col,
                      sum_splits(p.part + (long)(m0 + m) * p.N + nbase + col, (long)p.M * p.N,
                                 p.splits));
    }
    if (threadIdx.x == 0) p.counters[counter] = 0u;
}

// ---------------------------------------------------------------------------
// Dequantise: one thread per (packed row, 4 columns) -> 8 rows x 4 fp16.
// W[k, n] = fp16(code * scale) with the product exact in fp32
// (kernels/quant/quant_matmul.cu:612-627 semantics).
// ---------------------------------------------------------------------------
template <int COLS>
__global__ __launch_bounds__(256) void w4a16_dequantize_kernel(const uint32_t* __restrict__ w,
                                                               const uint16_t* __restrict__ scale,
                                                               uint16_t* __restrict__ out, int K,
                                                               int N, int group_size) {
    const int n0 = (blockIdx.x * 256 + threadIdx.x) * COLS;
    const int kp = blockIdx.y;
    if (n0 >= N) return;
    const int g = (kp * 8) / group_size;
    float codes[COLS][8];
    float s[COLS];
    if constexpr (COLS == 4) {
        const u32x4 raw = load16(w + (long)kp * N + n0);
#pragma unroll
        for (int j = 0; j < 4; ++j) i4x8_to_f32(raw[j], codes[j]);
        const u32x2 sr = load8(scale + (long)g * N + n0);
        s[0] = h2f(sr[0] & 0xFFFF); s[1] = h2f(sr[0] >> 16);
        s[2] = h2f(sr[1] & 0xFFFF); s[3] = h2f(sr[1] >> 16);
    } else {
        i4x8_to_f32(w[(long)kp * N + n0], codes[0]);
        s[0] = h2f(scale[(long)g * N + n0]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint16_t* dst = out + (long)(kp * 8 + e) * N + n0;
        if constexpr (COLS == 4) {
            u32x2 v;
            v[0] = (uint32_t)f2h_bits(codes[0][e] * s[0]) | ((uint32_t)f2h_bits(codes[1][e] * s[1]) << 16);
            v[1] = (uint32_t)f2h_bits(codes[2][e] * s[2]) | ((uint32_t)f2h_bits(codes[3][e] * s[3]) << 16);
            *reinterpret_cast<u32x2*>(dst) = v;
        } else {
            dst[0] = f2h_bits(codes[0][e] * s[0]);
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Streaming GEMV selection: 1 forces it wherever the shape allows, 0
// disables it; unset (-1), it serves packed weights of more than
// kStreamMinWeightBytes. Measured on MI355X at M = 1, 8 and 16: the
// single-row / 16-row GEMVs with 32-column tiles are faster at (4096, 4096)
// (8 MiB) and (14336, 1024); the streaming GEMV from (4096, 4608) (9 MiB)
// and at (14336, 2048) up (up to 27 % faster at M = 16). A positive split count
// forces the streaming GEMV's K split count (clamped to what the K extent
// allows). Both are measurement knobs: read once from LLMIK_W4A16_STREAM /
// LLMIK_W4A16_STREAM_SPLITS when the library loads, and settable with
// llmik_w4a16_set_plan_override.
constexpr long kStreamMinWeightBytes = 8L << 20;
// Rows from which the 256 x 128 LDS-staged GEMM (kind 7) serves M > 16.
#ifndef LLMIK_W4A16_LDS_MIN_M
#define LLMIK_W4A16_LDS_MIN_M 256
#endif

namespace {
int env_int(const char* name, bool as_flag) {
    const char* e = getenv(name);
    if (e == nullptr || *e == '\0') return -1;
    return as_flag ? ((*e == '0') ? 0 : 1) : atoi(e);
}
std::atomic<int> g_stream_mode{env_int("LLMIK_W4A16_STREAM", true)};
std::atomic<int> g_stream_splits{env_int("LLMIK_W4A16_STREAM_SPLITS", false)};
}  // namespace

void set_w4a16_plan_override(int stream_mode, int stream_splits) {
    g_stream_mode.store(stream_mode < 0 ? -1 : (stream_mode ? 1 : 0), std::memory_order_relaxed);
    g_stream_splits.store(stream_splits > 0 ? stream_splits : -1, std::memory_order_relaxed);
}

static int stream_override() { return g_stream_mode.load(std::memory_order_relaxed); }
static int stream_splits_override() { return g_stream_splits.load(std::memory_order_relaxed); }

// stream_mode: 1 forces the streaming GEMV where its shape rule holds, 0 rules
// it out, -1 applies the size rule.
static GemmPlan plan_w4a16_mode(int M, int N, int K, int group_size, int stream_mode) {
    GemmPlan pl{};
    const bool pow2_group = group_size >= 32 && (group_size & (group_size - 1)) == 0;
    const bool stream_size_ok = (long)K * N / 2 > kStreamMinWeightBytes;
    if (M >= 1 && M <= 16 && N % 64 == 0 && pow2_group && K % 32 == 0 &&
        (long)(K / 8) * N * 4 < (1L << 31) && (long)M * K * 2 < (1L << 31) &&
        (stream_mode == 1 || (stream_mode < 0 && stream_size_ok))) {
        // Streaming GEMV: as many K splits as whole workgroups per CU allow
        // (no second round of workgroups), then the wave count (8..16) and
        // steps per wave that cover a split with the fewest idle steps.
        const int steps = K / 32;
        const int tiles = N / 64;
        long want = (long)device_cu_count() / tiles;
        if (want < 1 || tiles > kMaxCounters) want = 1;
        const int forced = stream_splits_override();
        if (forced > 0 && tiles <= kMaxCounters) want = forced;
        if (want > steps / 2) want = steps / 2 > 0 ? steps / 2 : 1;
        const int need = (int)((steps + want - 1) / want);
        int best_nw = kStreamMaxWaves, best_ws = 0;
        long best_waste = -1;
        // Among equally padded choices: the most waves per workgroup when
        // the workgroups fit the CUs in one round; the fewest (8, two
        // workgroups per CU at <= 128 VGPRs) when they do not, so that they
        // all stay resident (N = 28672: M=8 18.5-19.0 -> 17.3-18.0 us,
        // M=16 21.0-22.3 -> 20.0).
        const bool two_rounds = (long)tiles * want > device_cu_count();
        for (int i = 0; i <= kStreamMaxWaves / 2; ++i) {
            const int nw = two_rounds ? kStreamMaxWaves / 2 + i : kStreamMaxWaves - i;
            int ws = (need + nw - 1) / nw;
            ws = ws <= 2 ? 2 : ws <= 4 ? 4 : (ws + 7) / 8 * 8;
            const long waste = (long)nw * ws - need;
            if (best_waste < 0 || waste < best_waste) {
                best_waste = waste;
                best_nw = nw;
                best_ws = ws;
            }
        }
        const int sps = best_nw * best_ws;
        pl.kind = 5;
        pl.waves = best_nw;
        pl.wave_steps = best_ws;
        pl.cols_per_lane = 4;
        pl.tile_n = kStreamTile;
        pl.tile_m = 16;
        pl.n_tiles = tiles;
        pl.m_tiles = 1;
        pl.kp_per_split = 4 * sps;
        pl.splits = (steps + sps - 1) / sps;
        pl.off_part = kCounterBytes;
        pl.workspace_bytes = (pl.splits > 1)
            ? kCounterBytes + align_up((size_t)pl.splits * M * N * sizeof(float), 256) : 0;
        return pl;
    }
    if (M == 1 && N % 16 == 0 && pow2_group && K % 32 == 0 && (long)(K / 8) * N * 4 < (1L << 31)) {
        // Matrix-core GEMV: widest tile (16 * cb columns) that divides N.
        int cb = LLMIK_GEMV_CB;
        while (cb > 1 && N % (16 * cb) != 0) cb /= 2;
        const int sb = kGemvBatch * kGemvWaves;   // a split is whole batches for every wave
        const int steps = K / 32;
        const int tiles = N / (16 * cb);
        const long target = (long)LLMIK_GEMV_WGS_PER_CU * device_cu_count();
        long want = (target + tiles - 1) / tiles;
        const long max_splits = (steps + sb - 1) / sb;
        if (want > max_splits) want = max_splits;
        if (tiles > kMaxCounters) want = 1;
        if (want < 1) want = 1;
        int sps = (int)((steps + want - 1) / want);
        sps = (sps + sb - 1) / sb * sb;
        if (sps * 32 <= kGemvMaxK) {
            pl.kind = 2;
            pl.cols_per_lane = cb;
            pl.tile_n = 16 * cb;
            pl.tile_m = 1;
            pl.n_tiles = tiles;
            pl.m_tiles = 1;
            pl.kp_per_split = 4 * sps;
            pl.splits = (steps + sps - 1) / sps;
            pl.off_part = kCounterBytes;
            pl.workspace_bytes =
                (pl.splits > 1) ? kCounterBytes + align_up((size_t)pl.splits * N * sizeof(float), 256) : 0;
            return pl;
        }
    }
    if (M >= 2 && M <= 16 && N % 32 == 0 && pow2_group && K % 32 == 0 &&
        (long)(K / 8) * N * 4 < (1L << 31)) {
        // Matrix-core GEMV over 16 rows: the single-row plan with 32-column tiles.
        const int cb = 2;
        const int sb = kGemvBatch * kGemvWaves;
        const int steps = K / 32;
        const int tiles = N / (16 * cb);
        const long target = (long)LLMIK_GEMV_WGS_PER_CU * device_cu_count();
        long want = (target + tiles - 1) / tiles;
        const long max_splits = (steps + sb - 1) / sb;
        if (want > max_splits) want = max_splits;
        if (tiles > kMaxCounters) want = 1;
        if (want < 1) want = 1;
        int sps = (int)((steps + want - 1) / want);
        sps = (sps + sb - 1) / sb * sb;
        pl.kind = 4;
        pl.cols_per_lane = cb;
        pl.tile_n = 16 * cb;
        pl.tile_m = 16;
        pl.n_tiles = tiles;
        pl.m_tiles = 1;
        pl.kp_per_split = 4 * sps;
        pl.splits = (steps + sps - 1) / sps;
        pl.off_part = kCounterBytes;
        pl.workspace_bytes =
            (pl.splits > 1) ? kCounterBytes + align_up((size_t)pl.splits * M * N * sizeof(float), 256) : 0;
        return pl;
    }
    if (M >= LLMIK_W4A16_LDS_MIN_M && N % 128 == 0 && pow2_group && K % 64 == 0 &&
        (long)(K / 8) * N * 4 < (1L << 31) && (long)M * K * 2 < (1L << 31) &&
        (long)M * N * 4 < (1L << 31) &&
        3L * ((M + kL7TM - 1) / kL7TM) * (N / kL7TN) > device_cu_count()) {
        // 256 x 128 tiles with both operands staged in LDS; K splits (whole
        // scale groups where they allow) until the tiles fill the CUs once.
        // Chosen over kind 6 when its tiles need at most 2 splits (its split
        // hand-off is slower than kind 6's, and with 4 or more splits kind 6
        // is as fast or faster: M=512 (4096, 4096) 25.6 against 32.5 us,
        // (14336, 4096) 77.2 against 76.0; M=768, 2 splits, 46.8 -> 44.4 and
        // 137.5 -> 126.4).
        const int stages = K / 64;
        const int spg = group_size / 64;   // stages per scale group (0 when it is 32)
        pl.kind = 7;
        pl.cols_per_lane = 2;
        pl.tile_n = kL7TN;
        pl.tile_m = kL7TM;
        pl.n_tiles = N / kL7TN;
        pl.m_tiles = (M + kL7TM - 1) / kL7TM;
        pl.waves = kL7Waves;
        const long cus = device_cu_count();
        const long tiles = (long)pl.n_tiles * pl.m_tiles;
        // Tiles in whole rounds of the CUs run unsplit; the rest (or all of
        // them, when they do not fill one round) may split K s ways (s <= 4).
        // Cost of the rest in stages: rounds ceil(rest * s / CUs) times
        // (stages / s + 8), plus 4 per round for the hand-off when s > 1 (a
        // round's prologue, epilogue and hand-off measure ~8 and ~4 stages);
        // a split is taken when it saves 15 %. M=768 (4096, 14336), 336
        // tiles: 256 unsplit and 80 in 3 splits, 135 -> 107 us; M=1024, 192
        // left, stays unsplit (4 splits measured 139 -> 172 us).
        long full = 0, want = 1, rest = tiles;
        if (tiles <= cus) {
            want = cus / tiles;
        } else {
            full = tiles / cus * cus;
            rest = tiles - full;
            auto cost = [&](long sp) {
                const long rounds = (rest * sp + cus - 1) / cus;
                return (double)rounds * ((double)(stages + sp - 1) / sp + 8.0 + (sp > 1 ? 4.0 : 0.0));
            };
            const double one = cost(1);
            double best = 0.85 * one;
            for (long sp = 2; sp <= 4 && rest > 0; ++sp)
                if (cost(sp) < best) { best = cost(sp); want = sp; }
            if (want == 1) full = 0, rest = tiles;   // no split: one plain launch order
        }
        if (rest > kMaxCounters) want = 1, full = 0, rest = tiles;
        if (want < 1) want = 1;
        if (want > stages) want = stages;
        int sps = (int)((stages + want - 1) / want);
        if (spg > 1 && sps > spg) sps = (sps + spg - 1) / spg * spg;
        pl.wave_steps = sps;
        pl.kp_per_split = 8 * sps;
        pl.splits = (stages + sps - 1) / sps;
        if (pl.splits == 1) full = 0, rest = tiles;
        pl.full_tiles = (int)full;
        pl.split_tiles = (int)rest;
        pl.off_part = kCounterBytes;
        pl.workspace_bytes = (pl.splits > 1)
            ? kCounterBytes + align_up((size_t)rest * pl.splits * kL7TM * kL7TN * sizeof(float), 256) : 0;
        return pl;
    }
    if (M > 16 && N % 128 == 0 && pow2_group && K % 32 == 0 && (long)(K / 8) * N * 4 < (1L << 31) &&
        (long)M * K * 2 < (1L << 31) && (long)M * N * 4 < (1L << 31)) {
        // 32x32x16 matrix-core GEMM: tiles of 64 rows by 128 columns, 8 waves
        // = 2 column halves x 4 K ranges of whole scale groups; K splits
        // until the tiles fill the CUs once (no second round).
        constexpr int kgs = 4;
        const int steps = K / 32;
        const int spg = group_size / 32;
        pl.kind = 6;
        pl.cols_per_lane = 2;
        pl.tile_n = 128;
        pl.tile_m = 64;
        pl.n_tiles = N / 128;
        pl.m_tiles = (M + 63) / 64;
        const long base = (long)pl.n_tiles * pl.m_tiles;
        long want = device_cu_count() / base;
        if (base > kMaxCounters) want = 1;
        if (want < 1) want = 1;
        int ws = (int)((steps + want * kgs - 1) / (want * kgs));
        if (ws > spg) ws = (ws + spg - 1) / spg * spg;
        ws = (ws + 1) / 2 * 2;   // whole two-step stages
        pl.wave_steps = ws;
        pl.waves = kG32Waves;
        pl.kp_per_split = 4 * ws * kgs;
        pl.splits = (steps + ws * kgs - 1) / (ws * kgs);
        pl.off_part = kCounterBytes;
        pl.workspace_bytes =
            (pl.splits > 1) ? kCounterBytes + align_up((size_t)pl.splits * M * N * sizeof(float), 256) : 0;
        return pl;
    }
    if (M >= 2 && N % 64 == 0 && pow2_group && K % 32 == 0 && (long)(K / 8) * N * 4 < (1L << 31)) {
        // Matrix-core GEMM: tiles of 16 * rt rows by 64 columns.
        int rt = 1;
        while (rt < 8 && 16 * rt < M) rt *= 2;
        const int kc = (rt >= 8) ? 4 : (rt >= 4 ? 8 : 16);
        const int steps = K / 32;
        pl.kind = 3;
        pl.cols_per_lane = 1;
        pl.tile_n = 64;
        pl.tile_m = 16 * rt;
        pl.n_tiles = N / 64;
        pl.m_tiles = (M + pl.tile_m - 1) / pl.tile_m;
        const long base = (long)pl.n_tiles * pl.m_tiles;
        const long target = device_cu_count();
        long want = (target + base - 1) / base;
        const long max_splits = (steps + kc - 1) / kc;
        if (want > max_splits) want = max_splits;
        if (base > kMaxCounters) want = 1;
        if (want < 1) want = 1;
        int sps = (int)((steps + want - 1) / want);
        sps = (sps + kc - 1) / kc * kc;
        pl.kp_per_split = 4 * sps;
        pl.splits = (steps + sps - 1) / sps;
        pl.off_part = kCounterBytes;
        pl.workspace_bytes =
            (pl.splits > 1) ? kCounterBytes + align_up((size_t)pl.splits * M * N * sizeof(float), 256) : 0;
        return pl;
    }
    pl.cols_per_lane = (N % 4 == 0) ? 4 : 1;
    pl.tile_n = 64 * pl.cols_per_lane;
    pl.n_tiles = (N + pl.tile_n - 1) / pl.tile_n;
    pl.kind = (M == 1) ? 0 : 1;
    pl.tile_m = (M == 1) ? 1 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16));
    if (pl.kind == 1 && pl.cols_per_lane == 4 && pl.tile_m > 8) pl.tile_m = 8;
    pl.m_tiles = (M + pl.tile_m - 1) / pl.tile_m;
    const int kp_total = K / 8;
    const int cus = device_cu_count();
    const long base = (long)pl.n_tiles * pl.m_tiles;
    // Target ~2 workgroups per CU; keep >= 4 packed rows per wave.
    long want = (2L * cus + base - 1) / base;
    const long max_splits = (kp_total + 4 * kGemmWaves - 1) / (4 * kGemmWaves);
    if (want > max_splits) want = max_splits;
    if (base > kMaxCounters) want = 1;   // enough workgroups without splitting
    if (want < 1) want = 1;
    int kps = (int)((kp_total + want - 1) / want);
    kps = (kps + kGemmWaves - 1) / kGemmWaves * kGemmWaves;
    pl.kp_per_split = kps;
    pl.splits = (kp_total + kps - 1) / kps;
    const size_t part = align_up((size_t)pl.splits * M * N * sizeof(float), 256);
    pl.off_part = kCounterBytes;
    pl.workspace_bytes = (pl.splits > 1) ? kCounterBytes + part : 0;
    return pl;
}

GemmPlan plan_w4a16(int M, int N, int K, int group_size) {
    return plan_w4a16_mode(M, N, K, group_size, stream_override());
}

// The pair epilogues (SwiGLU, q|k|v rope) always run the streaming GEMV (they
// pair the two 32-column halves of each 64-column tile), so they need that
// kernel's shape.
static_assert(kStreamTile == 64, "the pair epilogues assume 64-column tiles");
static bool swiglu_shape_ok(int M, int N, int K, int group_size) {
    const bool pow2_group = group_size >= 32 && (group_size & (group_size - 1)) == 0;
    return M >= 1 && M <= 16 && N > 0 && N % 64 == 0 && K > 0 && K % 32 == 0 && pow2_group &&
           (long)(K / 8) * N * 4 < (1L << 31) && (long)M * K * 2 < (1L << 31);
}

GemmPlan plan_w4a16_stream_forced(int M, int N, int K, int group_size) {
    if (!swiglu_shape_ok(M, N, K, group_size)) return GemmPlan{};
    return plan_w4a16_mode(M, N, K, group_size, 1);
}

static GemmParams gemm_params(const GemmPlan& pl, const void* act, const void* w, const void* scale,
                              void* out, bool f32_out, int M, int N, int K, int group_size, void* ws) {
    GemmParams p{};
    p.act = static_cast<const uint16_t*>(act);
    p.w = static_cast<const uint32_t*>(w);
    p.scale = static_cast<const uint16_t*>(scale);
    p.out = out;
    char* wsp = static_cast<char*>(ws);
    p.counters = reinterpret_cast<uint32_t*>(wsp);
    p.part = wsp ? reinterpret_cast<float*>(wsp + pl.off_part) : nullptr;
    p.M = M; p.N = N; p.K = K; p.group_size = group_size;
    p.splits = pl.splits;
    p.kp_per_split = pl.kp_per_split;
    p.n_tiles = pl.n_tiles;
    p.f32_out = f32_out ? 1 : 0;
    p.gshift = 0;
    while ((32 << p.gshift) < group_size) ++p.gshift;
    p.nw = pl.waves;
    p.wave_steps = pl.wave_steps;
    return p;
}

int launch_w4a16_swiglu(const void* act, const void* w, const void* scale, void* out, int M, int N,
                        int K, int group_size, void* ws, size_t ws_bytes, hipStream_t stream) {
    if (!swiglu_shape_ok(M, N, K, group_size))
        return set_error(LLMIK_ERR_UNSUPPORTED,
                         "w4a16 SwiGLU needs 1 <= M <= 16, N % 64 == 0, K % 32 == 0 and a power-of-two "
                         "group_size >= 32");
    const GemmPlan pl = plan_w4a16_stream_forced(M, N, K, group_size);
    if (pl.kind != 5) return set_error(LLMIK_ERR_UNSUPPORTED, "w4a16 SwiGLU: no streaming plan");
    if (pl.splits > 1 && ws_bytes < pl.workspace_bytes)
        return set_error(LLMIK_ERR_WORKSPACE, "workspace too small for this W4A16 call");
    GemmParams p = gemm_params(pl, act, w, scale, out, false, M, N, K, group_size, ws);
    p.epilogue = kEpiSwiglu;
    const int grid = pl.n_tiles * pl.splits;
    if (M == 1) launch_stream<1>(p, grid, stream);
    else launch_stream<16>(p, grid, stream);
    return check_launch();
}

int launch_w4a16_qkv_rope(const void* act, const void* w, const void* scale, const void* cs, const void* sn,
                          void* q_out, void* k_cache, void* v_cache, int M, int K, int group_size,
                          int n_heads, int n_kv_heads, int max_len, int pos, void* ws, size_t ws_bytes,
                          hipStream_t stream) {
    const int N = (n_heads + 2 * n_kv_heads) * 128;
    if (!swiglu_shape_ok(M, N, K, group_size))
        return set_error(LLMIK_ERR_UNSUPPORTED,
                         "w4a16 q|k|v rope needs 1 <= M <= 16, K % 32 == 0 and a power-of-two "
                         "group_size >= 32");
    const GemmPlan pl = plan_w4a16_stream_forced(M, N, K, group_size);
    if (pl.kind != 5) return set_error(LLMIK_ERR_UNSUPPORTED, "w4a16 q|k|v rope: no streaming plan");
    if (pl.splits > 1 && ws_bytes < pl.workspace_bytes)
        return set_error(LLMIK_ERR_WORKSPACE, "workspace too small for this W4A16 call");
    GemmParams p = gemm_params(pl, act, w, scale, nullptr, false, M, N, K, group_size, ws);
    p.epilogue = kEpiQkvRope;
    p.rope_cos = static_cast<const uint16_t*>(cs);
    p.rope_sin = static_cast<const uint16_t*>(sn);
    p.q_out = static_cast<uint16_t*>(q_out);
    p.k_cache = static_cast<uint16_t*>(k_cache);
    p.v_cache = static_cast<uint16_t*>(v_cache);
    p.n_q_heads = n_heads;
    p.n_kv_heads = n_kv_heads;
    p.cache_len = max_len;
    p.cache_pos = pos;
    const int grid = pl.n_tiles * pl.splits;
    if (M == 1) launch_stream<1>(p, grid, stream);
    else launch_stream<16>(p, grid, stream);
    return check_launch();
}

int launch_w4a16(const void* act, const void* w, const void* scale, void* out, bool f32_out,
                 int M, int N, int K, int group_size, void* ws, size_t ws_bytes,
                 hipStream_t stream) {
    if (M == 0 || N == 0) return LLMIK_OK;
    const GemmPlan pl = plan_w4a16(M, N, K, group_size);
    if (pl.splits > 1 && ws_bytes < pl.workspace_bytes)
        return set_error(LLMIK_ERR_WORKSPACE, "workspace too small for this W4A16 call");
    if (pl.m_tiles > 65535 || pl.splits > 65535)
        return set_error(LLMIK_ERR_UNSUPPORTED, "W4A16 grid too large");
    GemmParams p = gemm_params(pl, act, w, scale, out, f32_out, M, N, K, group_size, ws);
    dim3 block(kGemmThreads);
    if (pl.kind == 5) {
        const int grid = pl.n_tiles * pl.splits;
        if (M == 1) launch_stream<1>(p, grid, stream);
        else launch_stream<16>(p, grid, stream);
        return check_launch();
    }
    if (pl.kind == 2) {
        const int grid = pl.n_tiles * pl.splits;
        const int sps = pl.kp_per_split / 4;
        switch (pl.cols_per_lane) {
            case 4: launch_gemv_cb<4>(p, grid, sps, stream); break;
            case 2: launch_gemv_cb<2>(p, grid, sps, stream); break;
            default: launch_gemv_cb<1>(p, grid, sps, stream); break;
        }
    } else if (pl.kind == 4) {
        const int grid = pl.n_tiles * pl.splits;
        if (pl.kp_per_split / 4 / kGemvWaves > kGemvBatch) launch_gemv16_cb<2, true>(p, grid, stream);
        else launch_gemv16_cb<2, false>(p, grid, stream);
    } else if (pl.kind == 6) {
        p.m_tiles_ = pl.m_tiles;
        p.vec_out = (reinterpret_cast<uintptr_t>(out) % 16 == 0) ? 1 : 0;
        const dim3 grid(pl.n_tiles * pl.splits * pl.m_tiles), blk(kG32Threads);
        hipLaunchKernelGGL(w4a16_gemm_mfma32_kernel, grid, blk, 0, stream, p);
    } else if (pl.kind == 7) {
        p.m_tiles_ = pl.m_tiles;
        p.full_tiles = pl.full_tiles;
        const dim3 grid(pl.full_tiles + pl.split_tiles * pl.splits), blk(kL7Threads);
        if (group_size == 32) hipLaunchKernelGGL(w4a16_gemm_lds_kernel<true>, grid, blk, 0, stream, p);
        else hipLaunchKernelGGL(w4a16_gemm_lds_kernel<false>, grid, blk, 0, stream, p);
    } else if (pl.kind == 3) {
        const dim3 grid(pl.n_tiles * pl.splits * pl.m_tiles), blk(kMmaThreads);
        switch (pl.tile_m) {
            case 16: hipLaunchKernelGGL(w4a16_gemm_mfma_kernel<1>, grid, blk, 0, stream, p); break;
            case 32: hipLaunchKernelGGL(w4a16_gemm_mfma_kernel<2>, grid, blk, 0, stream, p); break;
            case 64: hipLaunchKernelGGL(w4a16_gemm_mfma_kernel<4>, grid, blk, 0, stream, p); break;
            default: hipLaunchKernelGGL(w4a16_gemm_mfma_kernel<8>, grid, blk, 0, stream, p); break;
        }
    } else if (pl.kind == 0) {
        dim3 grid(pl.n_tiles, pl.splits);
        if (pl.cols_per_lane == 4) hipLaunchKernelGGL(w4a16_gemv_kernel<4>, grid, block, 0, stream, p);
        else hipLaunchKernelGGL(w4a16_gemv_kernel<1>, grid, block, 0, stream, p);
    } else {
        dim3 grid(pl.n_tiles, pl.splits, pl.m_tiles);
        if (pl.cols_per_lane == 4) {
            if (pl.tile_m == 4) hipLaunchKernelGGL((w4a16_gemm_tiled_kernel<4, 4>), grid, block, 0, stream, p);
            else hipLaunchKernelGGL((w4a16_gemm_tiled_kernel<4, 8>), grid, block, 0, stream, p);
        } else {
            if (pl.tile_m == 4) hipLaunchKernelGGL((w4a16_gemm_tiled_kernel<1, 4>), grid, block, 0, stream, p);
            else if (pl.tile_m == 8) hipLaunchKernelGGL((w4a16_gemm_tiled_kernel<1, 8>), grid, block, 0, stream, p);
            else hipLaunchKernelGGL((w4a16_gemm_tiled_kernel<1, 16>), grid, block, 0, stream, p);
        }
    }
    return check_launch();
}

int launch_w4a16_dequantize(const void* w, const void* scale, void* out, int K, int N,
                            int group_size, hipStream_t stream) {
    if (K == 0 || N == 0) return LLMIK_OK;
    const int kp_total = K / 8;
    if (kp_total > 65535) return set_error(LLMIK_ERR_UNSUPPORTED, "K/8 exceeds 65535");
    if (N % 4 == 0) {
        dim3 grid((N / 4 + 255) / 256, kp_total);
        hipLaunchKernelGGL(w4a16_dequantize_kernel<4>, grid, dim3(256), 0, stream,
                           static_cast<const uint32_t*>(w), static_cast<const uint16_t*>(scale),
                           static_cast<uint16_t*>(out), K, N, group_size);
    } else {
        dim3 grid((N + 255) / 256, kp_total);
        hipLaunchKernelGGL(w4a16_dequantize_kernel<1>, grid, dim3(256), 0, stream,
                           static_cast<const uint32_t*>(w), static_cast<const uint16_t*>(scale),
                           static_cast<uint16_t*>(out), K, N, group_size);
    }
    return check_launch();
}

}  // namespace llmik
