// Split-K ("FlashDecoding") GQA decode attention over an fp16, INT8
// per-token or INT4 KIVI KV cache, for gfx950.
//
// Math (reference/attention_ref.py:43-80, bindings/extension.cpp:26-83):
//   out[b,h,:] = softmax(scale * q[b,h] . K[b,h/G,0:S]^T) @ V[b,h/G,0:S]
// with the cache addressed at stride kv_buf_len and read over [0, seqlen).
//
// Work decomposition
//   * One workgroup owns one (batch, kv_head, head_chunk, split): the
//     HPW <= 4 query heads that share a kv head are processed together, so
//     every K/V byte of the split is read from HBM exactly once (the
//     reference re-reads each kv head once per query head,
//     kernels/attention/fused_attention_splitk.cu:84-90).
//   * 256 threads = 16 DPP rows of 16 lanes. Lane c of a row owns the
//     channels 8c..8c+7 of one token; row r walks the split's tokens
//     r, r+16, r+32, ... four at a time, so each 64-token step of the
//     workgroup reads one contiguous block of the cache.
//   * Dot products are reduced inside a DPP row; each row keeps its own
//     online-softmax state (m, l, o) in the log2 domain. Rows are merged
//     through LDS at the end, then the split's un-normalised (o, m, l) is
//     written to the workspace. The last workgroup to finish a
//     (batch, kv_head, head_chunk) merges all splits and writes fp16 out,
//     so a call is one kernel launch. The merge order is fixed (split 0..n),
//     so results are deterministic.
//
// KV formats (packing is kernels/kv_cache/kv_compress.cuh:25-28 and
// kernels/common/cuda_utils.cuh:85-119 of the reference):
//   F16: k,v [B,Hkv,L,128] fp16
//   I8 : k,v [B,Hkv,L,128] int8, k_scale,v_scale [B,Hkv,L] fp16 (per token)
//   I4 : k,v [B,Hkv,L,64] packed int4 (even channel in the low nibble),
//        k_scale [B,Hkv,n_groups,128] fp16 (per channel, per group of
//        group_size tokens), v_scale [B,Hkv,L] fp16 (per token)
#include "device_common.hpp"
#include "llmik_internal.hpp"

namespace llmik {

enum class KvFormat { F16, I8, I4 };

constexpr int kAttnThreads = 256;
constexpr int kRows = kAttnThreads / 16;   // 16 token rows per workgroup
constexpr int kUnroll = 4;                 // tokens per row per step
constexpr int kStepTokens = kRows * kUnroll;
constexpr int kHeadDim = 128;
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

template <KvFormat F, int HPW>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(AttnParams p) {
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

    // INT4 K scales: per-channel, constant over a group of tokens.
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
                const int g = min(tok[u], t_end - 1) / p.group_size;
                if (g != cur_group) {
                    cur_group = g;
                    float tmp[8];
                    f16x8_to_f32(load16(ks_base + (long)g * kHeadDim), tmp);
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

    // ---- merge the 16 row states of this workgroup through LDS ----
    __shared__ float s_o[kRows][HPW][kHeadDim];
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

    constexpr int kOuts = HPW * kHeadDim;
    const int slot_group = (b * p.n_kv_heads + kvh) * p.n_hchunks + hchunk;
    const long slot = (long)slot_group * p.n_splits + split;
    float wo[(kOuts + kAttnThreads - 1) / kAttnThreads];
    float wm[(kOuts + kAttnThreads - 1) / kAttnThreads];
    float wl[(kOuts + kAttnThreads - 1) / kAttnThreads];
#pragma unroll
    for (int i = 0; i < (kOuts + kAttnThreads - 1) / kAttnThreads; ++i) {
        const int idx = tid + i * kAttnThreads;
        wo[i] = 0.0f;
        wm[i] = -INFINITY;
        wl[i] = 0.0f;
        if (idx < kOuts) {
            const int h = idx / kHeadDim, d = idx % kHeadDim;
            float gm = -INFINITY;
#pragma unroll
            for (int r = 0; r < kRows; ++r) gm = fmaxf(gm, s_m[r][h]);
            float so = 0.0f, sl = 0.0f;
            if (gm != -INFINITY) {
#pragma unroll
                for (int r = 0; r < kRows; ++r) {
                    const float w = (s_m[r][h] == -INFINITY)
                                        ? 0.0f
                                        : __builtin_amdgcn_exp2f(s_m[r][h] - gm);
                    so = fmaf(s_o[r][h][d], w, so);
                    sl = fmaf(s_l[r][h], w, sl);
                }
            }
            wo[i] = so;
            wm[i] = gm;
            wl[i] = sl;
        }
    }

    if (p.n_splits == 1) {
#pragma unroll
        for (int i = 0; i < (kOuts + kAttnThreads - 1) / kAttnThreads; ++i) {
            const int idx = tid + i * kAttnThreads;
            if (idx < kOuts) {
                const int h = idx / kHeadDim, d = idx % kHeadDim;
                const float inv = (wl[i] > 0.0f) ? 1.0f / wl[i] : 0.0f;
                p.out[((long)b * p.n_heads + head0 + h) * kHeadDim + d] = f2h_bits(wo[i] * inv);
            }
        }
        return;
    }

    // ---- publish this split's partial; the last split to land combines ----
#pragma unroll
    for (int i = 0; i < (kOuts + kAttnThreads - 1) / kAttnThreads; ++i) {
        const int idx = tid + i * kAttnThreads;
        if (idx < kOuts) {
            const int h = idx / kHeadDim, d = idx % kHeadDim;
            p.part_o[(slot * HPW + h) * kHeadDim + d] = wo[i];
            if (d == 0) {
                p.part_ml[(slot * HPW + h) * 2 + 0] = wm[i];
                p.part_ml[(slot * HPW + h) * 2 + 1] = wl[i];
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&p.counters[slot_group], 1u);
        s_last = (prev == (uint32_t)(p.n_splits - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (s_last == 0u) return;
    __threadfence();

#pragma unroll
    for (int i = 0; i < (kOuts + kAttnThreads - 1) / kAttnThreads; ++i) {
        const int idx = tid + i * kAttnThreads;
        if (idx < kOuts) {
            const int h = idx / kHeadDim, d = idx % kHeadDim;
            const long base = (long)slot_group * p.n_splits;
            float gm = -INFINITY;
            for (int sp = 0; sp < p.n_splits; ++sp)
                gm = fmaxf(gm, __builtin_nontemporal_load(&p.part_ml[((base + sp) * HPW + h) * 2]));
            float so = 0.0f, sl = 0.0f;
            if (gm != -INFINITY) {
                for (int sp = 0; sp < p.n_splits; ++sp) {
                    const float ms = __builtin_nontemporal_load(&p.part_ml[((base + sp) * HPW + h) * 2]);
                    if (ms == -INFINITY) continue;
                    const float w = __builtin_amdgcn_exp2f(ms - gm);
                    so = fmaf(__builtin_nontemporal_load(&p.part_o[((base + sp) * HPW + h) * kHeadDim + d]), w, so);
                    sl = fmaf(__builtin_nontemporal_load(&p.part_ml[((base + sp) * HPW + h) * 2 + 1]), w, sl);
                }
            }
            const float inv = (sl > 0.0f) ? 1.0f / sl : 0.0f;
            p.out[((long)b * p.n_heads + head0 + h) * kHeadDim + d] = f2h_bits(so * inv);
        }
    }
    if (tid == 0) p.counters[slot_group] = 0u;   // leave the counter zeroed for the next call
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
    // Aim for ~4 resident workgroups per CU, with at least one 64-token step
    // per split so every split does real work.
    const long target = 4L * cus;
    long want = (target + base_wgs - 1) / base_wgs;
    const long max_useful = (seqlen + kStepTokens - 1) / kStepTokens;
    if (want > max_useful) want = max_useful;
    if (want > kMaxAttnSplits) want = kMaxAttnSplits;
    if (want < 1) want = 1;
    int chunk = (int)((seqlen + want - 1) / want);
    chunk = ((chunk + kStepTokens - 1) / kStepTokens) * kStepTokens;
    if (chunk < kStepTokens) chunk = kStepTokens;
    pl.chunk = chunk;
    pl.n_splits = seqlen > 0 ? (seqlen + chunk - 1) / chunk : 1;
    pl.n_slot_groups = base_wgs;
    const size_t counters = align_up((size_t)base_wgs * sizeof(uint32_t), 256);
    const size_t slots = (size_t)base_wgs * pl.n_splits * pl.hpw;
    const size_t ml = align_up(slots * 2 * sizeof(float), 256);
    const size_t po = align_up(slots * kHeadDim * sizeof(float), 256);
    pl.workspace_bytes = (pl.n_splits > 1) ? counters + ml + po : 0;
    pl.off_ml = counters;
    pl.off_o = counters + ml;
    return pl;
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

    dim3 grid(pl.n_splits, a.n_kv_heads * pl.n_hchunks, a.batch);
    dim3 block(kAttnThreads);
    switch (pl.hpw) {
        case 4: hipLaunchKernelGGL((decode_attention_kernel<F, 4>), grid, block, 0, stream, p); break;
        case 2: hipLaunchKernelGGL((decode_attention_kernel<F, 2>), grid, block, 0, stream, p); break;
        default: hipLaunchKernelGGL((decode_attention_kernel<F, 1>), grid, block, 0, stream, p); break;
    }
    return check_launch();
}

int launch_attention_f16(const AttnLaunch& a, hipStream_t s) { return launch_attention<KvFormat::F16>(a, s); }
int launch_attention_i8(const AttnLaunch& a, hipStream_t s) { return launch_attention<KvFormat::I8>(a, s); }
int launch_attention_i4(const AttnLaunch& a, hipStream_t s) { return launch_attention<KvFormat::I4>(a, s); }

}  // namespace llmik
