// extern "C" entry points of libllmik_hip.so (declared in include/llmik.h).
// This layer validates arguments, turns HIP failures into status codes
// (the reference aborts the process on a launch error,
// kernels/common/cuda_utils.cuh:12-24) and forwards to the launchers.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "llmik_internal.hpp"

namespace llmik {

namespace {
thread_local char g_last_error[512] = "";

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int invalid(const char* msg) { return set_error(LLMIK_ERR_INVALID, msg); }
}  // namespace

int set_error(int code, const char* msg) {
    std::snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
    return code;
}

int check_launch() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        std::snprintf(g_last_error, sizeof(g_last_error), "HIP launch failed: %s",
                      hipGetErrorString(e));
        return static_cast<int>(e);
    }
    return LLMIK_OK;
}

int device_cu_count() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return 256;
    }
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0) {
            (void)hipGetLastError();
            cus = 256;
        }
        cache[dev] = cus;
    }
    return cache[dev];
}

}  // namespace llmik

using namespace llmik;

namespace {

int check_attention_common(const void* q, const void* out, int batch, int n_heads,
                           int n_kv_heads, int seqlen, int head_dim, int kv_buf_len) {
    if (batch < 0 || n_heads <= 0 || n_kv_heads <= 0)
        return invalid("batch must be >= 0 and head counts positive");
    if (head_dim != 128) return invalid("only head_dim=128 supported");
    if (n_heads % n_kv_heads != 0) return invalid("n_heads must be a multiple of n_kv_heads");
    if (seqlen < 0 || kv_buf_len < 0) return invalid("seqlen and kv_buf_len must be >= 0");
    if (seqlen > kv_buf_len) return invalid("seqlen exceeds allocated cache length");
    if ((long)batch * n_kv_heads > 65535L) return invalid("batch * n_kv_heads exceeds 65535");
    if (batch > 0 && (q == nullptr || out == nullptr)) return invalid("null q/out pointer");
    if (!aligned(q, 16) || !aligned(out, 16))
        return set_error(LLMIK_ERR_ALIGNMENT, "q/out must be 16-byte aligned");
    return LLMIK_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace

extern "C" {

LLMIK_API const char* llmik_last_error(void) { return g_last_error; }

LLMIK_API int llmik_abi_version(void) { return 1; }

LLMIK_API size_t llmik_attention_workspace_size(int batch, int n_heads, int n_kv_heads,
                                                int seqlen, int head_dim) {
    if (batch <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim != 128 ||
        n_heads % n_kv_heads != 0 || seqlen <= 0)
        return 0;
    return plan_attention(batch, n_heads, n_kv_heads, seqlen).workspace_bytes;
}

LLMIK_API llmik_status llmik_decode_attention_f16(const void* q, const void* k, const void* v,
                                                  void* out, int batch, int n_heads,
                                                  int n_kv_heads, int seqlen, int head_dim,
                                                  int kv_buf_len, float softmax_scale,
                                                  void* workspace, size_t workspace_bytes,
                                                  void* stream) {
    int st = check_attention_common(q, out, batch, n_heads, n_kv_heads, seqlen, head_dim,
                                    kv_buf_len);
    if (st != LLMIK_OK) return st;
    if (batch == 0) return LLMIK_OK;
    if (seqlen > 0 && (k == nullptr || v == nullptr)) return invalid("null k/v pointer");
    if (!aligned(k, 16) || !aligned(v, 16))
        return set_error(LLMIK_ERR_ALIGNMENT, "k/v must be 16-byte aligned");
    AttnLaunch a{};
    a.q = q; a.k = k; a.v = v; a.out = out;
    a.batch = batch; a.n_heads = n_heads; a.n_kv_heads = n_kv_heads;
    a.seqlen = seqlen; a.kv_buf_len = kv_buf_len;
    a.softmax_scale = softmax_scale;
    a.workspace = workspace; a.workspace_bytes = workspace_bytes;
    return launch_attention_f16(a, as_stream(stream));
}

LLMIK_API llmik_status llmik_decode_attention_int8(const void* q, const void* k_q,
                                                   const void* k_scale, const void* v_q,
                                                   const void* v_scale, void* out, int batch,
                                                   int n_heads, int n_kv_heads, int seqlen,
                                                   int head_dim, int kv_buf_len,
                                                   float softmax_scale, void* workspace,
                                                   size_t workspace_bytes, void* stream) {
    int st = check_attention_common(q, out, batch, n_heads, n_kv_heads, seqlen, head_dim,
                                    kv_buf_len);
    if (st != LLMIK_OK) return st;
    if (batch == 0) return LLMIK_OK;
    if (seqlen > 0 && (!k_q || !v_q || !k_scale || !v_scale)) return invalid("null KV pointer");
    if (!aligned(k_q, 16) || !aligned(v_q, 16) || !aligned(k_scale, 2) || !aligned(v_scale, 2))
        return set_error(LLMIK_ERR_ALIGNMENT, "int8 KV must be 16-byte aligned");
    AttnLaunch a{};
    a.q = q; a.k = k_q; a.v = v_q; a.k_scale = k_scale; a.v_scale = v_scale; a.out = out;
    a.batch = batch; a.n_heads = n_heads; a.n_kv_heads = n_kv_heads;
    a.seqlen = seqlen; a.kv_buf_len = kv_buf_len;
    a.softmax_scale = softmax_scale;
    a.workspace = workspace; a.workspace_bytes = workspace_bytes;
    return launch_attention_i8(a, as_stream(stream));
}

LLMIK_API llmik_status llmik_decode_attention_int4(const void* q, const void* k_q,
                                                   const void* k_scale, const void* v_q,
                                                   const void* v_scale, void* out, int batch,
                                                   int n_heads, int n_kv_heads, int seqlen,
                                                   int head_dim, int kv_buf_len, int group_size,
                                                   int n_groups, float softmax_scale,
                                                   void* workspace, size_t workspace_bytes,
                                                   void* stream) {
    int st = check_attention_common(q, out, batch, n_heads, n_kv_heads, seqlen, head_dim,
                                    kv_buf_len);
    if (st != LLMIK_OK) return st;
    if (group_size <= 0) return invalid("group_size must be positive");
    if (n_groups < 0) return invalid("n_groups must be >= 0");
    if (seqlen > 0 && (long)n_groups * group_size < seqlen)
        return invalid("k_scale has fewer groups than seqlen requires");
    if (batch == 0) return LLMIK_OK;
    if (seqlen > 0 && (!k_q || !v_q || !k_scale || !v_scale)) return invalid("null KV pointer");
    if (!aligned(k_q, 16) || !aligned(v_q, 16) || !aligned(k_scale, 16) || !aligned(v_scale, 2))
        return set_error(LLMIK_ERR_ALIGNMENT, "int4 KV and k_scale must be 16-byte aligned");
    AttnLaunch a{};
    a.q = q; a.k = k_q; a.v = v_q; a.k_scale = k_scale; a.v_scale = v_scale; a.out = out;
    a.batch = batch; a.n_heads = n_heads; a.n_kv_heads = n_kv_heads;
    a.seqlen = seqlen; a.kv_buf_len = kv_buf_len;
    a.group_size = group_size; a.n_groups = n_groups;
    a.softmax_scale = softmax_scale;
    a.workspace = workspace; a.workspace_bytes = workspace_bytes;
    return launch_attention_i4(a, as_stream(stream));
}

namespace {
int check_writer(const void* x, const void* q, const void* scale, int batch, int n_kv_heads,
                 int seqlen, int head_dim) {
    if (batch < 0 || n_kv_heads < 0 || seqlen < 0) return invalid("negative dimension");
    if (head_dim != 128) return invalid("only head_dim=128 supported");
    const long rows = (long)batch * n_kv_heads * seqlen;
    if (rows > 0 && (!x || !q || !scale)) return invalid("null pointer");
    if (!aligned(x, 16) || !aligned(q, 4) || !aligned(scale, 2))
        return set_error(LLMIK_ERR_ALIGNMENT, "x must be 16-byte aligned, q 4-byte aligned");
    return LLMIK_OK;
}
}  // namespace

LLMIK_API llmik_status llmik_quantize_per_token_int8(const void* x, void* q, void* scale,
                                                     int batch, int n_kv_heads, int seqlen,
                                                     int head_dim, void* stream) {
    int st = check_writer(x, q, scale, batch, n_kv_heads, seqlen, head_dim);
    if (st != LLMIK_OK) return st;
    if (!aligned(q, 8)) return set_error(LLMIK_ERR_ALIGNMENT, "q must be 8-byte aligned");
    return launch_quantize_per_token(x, q, scale, batch * n_kv_heads, seqlen, seqlen, seqlen, 0,
                                     127, false, as_stream(stream));
}
LLMIK_API llmik_status llmik_quantize_k_per_channel_groupwise_int4(const void* x, void* q,
                                                                   void* scale, int batch,
                                                                   int n_kv_heads, int seqlen,
                                                                   int head_dim, int group_size,
                                                                   void* stream) {
    int st = check_writer(x, q, scale, batch, n_kv_heads, seqlen, head_dim);
    if (st != LLMIK_OK) return st;
    if (group_size <= 0) return invalid("group_size must be positive");
    const int n_groups = seqlen > 0 ? (seqlen + group_size - 1) / group_size : 0;
    return launch_quantize_k_groupwise_int4(x, q, scale, batch * n_kv_heads, seqlen, seqlen,
                                            seqlen, 0, n_groups, group_size, as_stream(stream));
}
LLMIK_API llmik_status llmik_quantize_v_per_token_int4(const void* x, void* q, void* scale,
                                                       int batch, int n_kv_heads, int seqlen,
                                                       int head_dim, void* stream) {
    int st = check_writer(x, q, scale, batch, n_kv_heads, seqlen, head_dim);
    if (st != LLMIK_OK) return st;
    return launch_quantize_per_token(x, q, scale, batch * n_kv_heads, seqlen, seqlen, seqlen, 0, 7,
                                     true, as_stream(stream));
}

// ---- in-place (cache) writers ----------------------------------------------
namespace {
int check_into(const void* x, int x_len, const void* q, const void* scale, int batch,
               int n_kv_heads, int n_tok, int head_dim, int cache_len, int offset) {
    if (batch < 0 || n_kv_heads < 0 || n_tok < 0 || x_len < 0 || cache_len < 0)
        return invalid("negative dimension");
    if (head_dim != 128) return invalid("only head_dim=128 supported");
    if (n_tok > x_len) return invalid("n_tok exceeds the token length of x");
    if (offset < 0 || (long)offset + n_tok > cache_len)
        return invalid("offset + n_tok exceeds the cache length");
    if ((long)batch * n_kv_heads > 65535L) return invalid("batch * n_kv_heads exceeds 65535");
    if ((long)batch * n_kv_heads * n_tok > 0 && (!x || !q || !scale)) return invalid("null pointer");
    if (!aligned(x, 16) || !aligned(q, 8) || !aligned(scale, 2))
        return set_error(LLMIK_ERR_ALIGNMENT, "x must be 16-byte aligned, q 8-byte aligned");
    return LLMIK_OK;
}
}  // namespace

LLMIK_API llmik_status llmik_quantize_per_token_int8_into(const void* x, int x_len, void* q_cache,
                                                          void* scale_cache, int batch,
                                                          int n_kv_heads, int n_tok, int head_dim,
                                                          int cache_len, int offset, void* stream) {
    int st = check_into(x, x_len, q_cache, scale_cache, batch, n_kv_heads, n_tok, head_dim,
                        cache_len, offset);
    if (st != LLMIK_OK) return st;
    return launch_quantize_per_token(x, q_cache, scale_cache, batch * n_kv_heads, n_tok, x_len,
                                     cache_len, offset, 127, false, as_stream(stream));
}
LLMIK_API llmik_status llmik_quantize_v_per_token_int4_into(const void* x, int x_len, void* q_cache,
                                                            void* scale_cache, int batch,
                                                            int n_kv_heads, int n_tok, int head_dim,
                                                            int cache_len, int offset, void* stream) {
    int st = check_into(x, x_len, q_cache, scale_cache, batch, n_kv_heads, n_tok, head_dim,
                        cache_len, offset);
    if (st != LLMIK_OK) return st;
    return launch_quantize_per_token(x, q_cache, scale_cache, batch * n_kv_heads, n_tok, x_len,
                                     cache_len, offset, 7, true, as_stream(stream));
}
LLMIK_API llmik_status llmik_quantize_k_per_channel_groupwise_int4_into(
    const void* x, int x_len, void* q_cache, void* scale_cache, int batch, int n_kv_heads,
    int n_tok, int head_dim, int cache_len, int offset, int group_size, void* stream) {
    int st = check_into(x, x_len, q_cache, scale_cache, batch, n_kv_heads, n_tok, head_dim,
                        cache_len, offset);
    if (st != LLMIK_OK) return st;
    if (group_size <= 0) return invalid("group_size must be positive");
    if (offset % group_size != 0) return invalid("offset must be a multiple of group_size");
    const int cache_groups = (cache_len + group_size - 1) / group_size;
    return launch_quantize_k_groupwise_int4(x, q_cache, scale_cache, batch * n_kv_heads, n_tok,
                                            x_len, cache_len, offset, cache_groups, group_size,
                                            as_stream(stream));
}

LLMIK_API llmik_status llmik_kivi_append_token_int4(
    const void* k, int k_len, const void* v, int v_len, void* k_open, void* k_q, void* k_scale, void* v_q,
    void* v_scale, int batch, int n_kv_heads, int head_dim, int max_len, int group_size, int length,
    void* stream) {
    if (batch < 0 || n_kv_heads < 0 || k_len < 1 || v_len < 1 || max_len < 0)
        return invalid("negative dimension");
    if (head_dim != 128) return invalid("only head_dim=128 supported");
    if (group_size <= 0 || group_size > 128) return invalid("group_size must be in 1..128");
    if (length < 0 || length >= max_len) return invalid("the cache is full");
    if ((long)batch * n_kv_heads > 65535L) return invalid("batch * n_kv_heads exceeds 65535");
    if ((long)batch * n_kv_heads > 0 && (!k || !v || !k_open || !k_q || !k_scale || !v_q || !v_scale))
        return invalid("null pointer");
    if (!aligned(k, 16) || !aligned(v, 16) || !aligned(k_open, 16) || !aligned(k_q, 4) ||
        !aligned(v_q, 4) || !aligned(k_scale, 2) || !aligned(v_scale, 2))
        return set_error(LLMIK_ERR_ALIGNMENT, "k, v and k_open must be 16-byte aligned");
    const int n_groups = (max_len + group_size - 1) / group_size;
    return launch_kivi_append_token(k, (long)k_len * 128, v, (long)v_len * 128, k_open, k_q, k_scale, v_q,
                                    v_scale, batch * n_kv_heads, length % group_size, length, group_size,
                                    max_len, n_groups, as_stream(stream));
}

namespace {
int check_gemm(const void* act, const void* w, const void* scale, const void* out, int M, int N,
               int K, int group_size) {
    if (M < 0 || N < 0 || K < 0) return invalid("negative dimension");
    if (K % 8 != 0) return invalid("act.K must equal weight_packed.K_packs * 8");
    if (group_size <= 0 || group_size % 8 != 0)
        return invalid("group_size must be a positive multiple of 8");
    if (K % group_size != 0) return invalid("K must equal n_groups * group_size");
    if ((long)M * N > 0 && K > 0 && (!act || !w || !scale || !out)) return invalid("null pointer");
    if (!aligned(act, 16) || !aligned(w, 16) || !aligned(scale, 8) || !aligned(out, 4))
        return set_error(LLMIK_ERR_ALIGNMENT,
                         "act/weight must be 16-byte, scale 8-byte and out 4-byte aligned");
    return LLMIK_OK;
}
}  // namespace

LLMIK_API size_t llmik_w4a16_workspace_size(int M, int N, int K, int group_size) {
    if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || group_size % 8 || K % group_size) return 0;
    return plan_w4a16(M, N, K, group_size).workspace_bytes;
}

LLMIK_API llmik_status llmik_w4a16_gemm(const void* act, const void* weight_packed,
                                        const void* scale, void* out, int M, int N, int K,
                                        int group_size, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    int st = check_gemm(act, weight_packed, scale, out, M, N, K, group_size);
    if (st != LLMIK_OK) return st;
    if (K == 0) return invalid("K must be positive");
    return launch_w4a16(act, weight_packed, scale, out, false, M, N, K, group_size, workspace,
                        workspace_bytes, as_stream(stream));
}

LLMIK_API llmik_status llmik_w4a16_gemm_f32out(const void* act, const void* weight_packed,
                                               const void* scale, void* out_f32, int M, int N,
                                               int K, int group_size, void* workspace,
                                               size_t workspace_bytes, void* stream) {
    int st = check_gemm(act, weight_packed, scale, out_f32, M, N, K, group_size);
    if (st != LLMIK_OK) return st;
    if (K == 0) return invalid("K must be positive");
    return launch_w4a16(act, weight_packed, scale, out_f32, true, M, N, K, group_size, workspace,
                        workspace_bytes, as_stream(stream));
}

LLMIK_API size_t llmik_w4a16_swiglu_workspace_size(int M, int N, int K, int group_size) {
    return plan_w4a16_stream_forced(M, N, K, group_size).workspace_bytes;
}

LLMIK_API size_t llmik_w4a16_qkv_rope_workspace_size(int batch, int n_heads, int n_kv_heads, int K,
                                                     int group_size) {
    if (n_heads <= 0 || n_kv_heads <= 0) return 0;
    return plan_w4a16_stream_forced(batch, (n_heads + 2 * n_kv_heads) * 128, K, group_size).workspace_bytes;
}

LLMIK_API llmik_status llmik_w4a16_gemm_qkv_rope_f16(
    const void* act, const void* weight_packed, const void* scale, const void* cos, const void* sin,
    void* q_out, void* k_cache, void* v_cache, int batch, int K, int group_size, int n_heads,
    int n_kv_heads, int max_len, int pos, void* workspace, size_t workspace_bytes, void* stream) {
    if (batch < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0)
        return invalid("n_heads must be a positive multiple of n_kv_heads");
    if (pos < 0 || pos >= max_len) return invalid("pos outside the cache");
    const int N = (n_heads + 2 * n_kv_heads) * 128;
    int st = check_gemm(act, weight_packed, scale, q_out, batch, N, K, group_size);
    if (st != LLMIK_OK) return st;
    if (!cos || !sin || !k_cache || !v_cache) return invalid("null pointer");
    if (!aligned(cos, 2) || !aligned(sin, 2) || !aligned(k_cache, 2) || !aligned(v_cache, 2))
        return set_error(LLMIK_ERR_ALIGNMENT, "cos, sin and the caches must be 2-byte aligned");
    if (batch == 0) return LLMIK_OK;
    return launch_w4a16_qkv_rope(act, weight_packed, scale, cos, sin, q_out, k_cache, v_cache, batch, K,
                                 group_size, n_heads, n_kv_heads, max_len, pos, workspace,
                                 workspace_bytes, as_stream(stream));
}

LLMIK_API llmik_status llmik_w4a16_gemm_swiglu(const void* act, const void* weight_packed,
                                               const void* scale, void* out, int M, int N, int K,
                                               int group_size, void* workspace, size_t workspace_bytes,
                                               void* stream) {
    int st = check_gemm(act, weight_packed, scale, out, M, N, K, group_size);
    if (st != LLMIK_OK) return st;
    if (M == 0 || N == 0) return LLMIK_OK;
    return launch_w4a16_swiglu(act, weight_packed, scale, out, M, N, K, group_size, workspace,
                               workspace_bytes, as_stream(stream));
}

LLMIK_API void llmik_w4a16_set_plan_override(int stream_mode, int stream_splits) {
    set_w4a16_plan_override(stream_mode, stream_splits);
}

LLMIK_API void llmik_attention_set_plan_override(int f16_half_tiles) {
    set_attention_plan_override(f16_half_tiles);
}

LLMIK_API llmik_status llmik_w4a16_dequantize(const void* weight_packed, const void* scale,
                                              void* out, int K, int N, int group_size,
                                              void* stream) {
    if (K < 0 || N < 0) return invalid("negative dimension");
    if (K % 8 != 0) return invalid("K must be a multiple of 8");
    if (group_size <= 0 || K % group_size != 0)
        return invalid("K must be a multiple of group_size");
    if ((long)K * N > 0 && (!weight_packed || !scale || !out)) return invalid("null pointer");
    if (!aligned(weight_packed, 16) || !aligned(scale, 8) || !aligned(out, 8))
        return set_error(LLMIK_ERR_ALIGNMENT, "weight_packed must be 16-byte aligned");
    return launch_w4a16_dequantize(weight_packed, scale, out, K, N, group_size, as_stream(stream));
}

LLMIK_API llmik_status llmik_quantize_weights_int4_groupwise(const void* W, int w_fp16, int K, int N,
                                                             int group_size, void* q, void* packed,
                                                             void* scale, void* scale_f16,
                                                             void* stream) {
    if (K < 0 || N < 0) return invalid("negative dimension");
    if (group_size <= 0) return invalid("group_size must be positive");
    if (packed && (K % 8 != 0 || group_size % 8 != 0))
        return invalid("packing needs K and group_size to be multiples of 8");
    if ((long)K * N > 0 && !W) return invalid("null pointer");
    if ((long)K * N >= (1L << 31)) return set_error(LLMIK_ERR_UNSUPPORTED, "W has 2^31 or more elements");
    if (!aligned(W, w_fp16 ? 2 : 4) || !aligned(scale, w_fp16 ? 2 : 4) || !aligned(scale_f16, 2) ||
        !aligned(packed, 4))
        return set_error(LLMIK_ERR_ALIGNMENT, "misaligned buffer");
    return launch_quantize_weights_int4(W, w_fp16 != 0, K, N, group_size, q, packed, scale, scale_f16,
                                        as_stream(stream));
}

LLMIK_API llmik_status llmik_pack_int4_along_k(const void* q, int K, int N, void* packed,
                                               void* stream) {
    if (K < 0 || N < 0) return invalid("negative dimension");
    if (K % 8 != 0) return invalid("K must be a multiple of 8");
    if ((long)K * N > 0 && (!q || !packed)) return invalid("null pointer");
    if (!aligned(packed, 4)) return set_error(LLMIK_ERR_ALIGNMENT, "packed must be 4-byte aligned");
    return launch_pack_int4_along_k(q, K, N, packed, as_stream(stream));
}

LLMIK_API llmik_status llmik_rmsnorm(const void* x, const void* weight, void* out, int rows,
                                     int hidden, float eps, void* stream) {
    if (rows < 0 || hidden < 0) return invalid("negative dimension");
    if (rows > 0 && hidden > 0 && (!x || !weight || !out)) return invalid("null pointer");
    if (hidden % 8 == 0 && (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, 16)))
        return set_error(LLMIK_ERR_ALIGNMENT, "rmsnorm tensors must be 16-byte aligned");
    return launch_rmsnorm(x, weight, out, rows, hidden, eps, as_stream(stream));
}

LLMIK_API llmik_status llmik_silu_mul(const void* gate, const void* up, void* out, long n,
                                      void* stream) {
    if (n < 0) return invalid("negative size");
    if (n > 0 && (!gate || !up || !out)) return invalid("null pointer");
    if (!aligned(gate, 16) || !aligned(up, 16) || !aligned(out, 16))
        return set_error(LLMIK_ERR_ALIGNMENT, "silu_mul tensors must be 16-byte aligned");
    return launch_silu_mul(gate, up, out, n, as_stream(stream));
}

LLMIK_API llmik_status llmik_rope(const void* x, const void* cos, const void* sin, void* out,
                                  int B, int H, int S, int D, void* stream) {
    if (B < 0 || H < 0 || S < 0 || D < 0) return invalid("negative dimension");
    if (D % 2 != 0) return invalid("head_dim must be even");
    if ((long)B * H * S * D > 0 && (!x || !cos || !sin || !out)) return invalid("null pointer");
    return launch_rope(x, cos, sin, out, B, H, S, D, as_stream(stream));
}

LLMIK_API llmik_status llmik_rope_qkv_append_f16(const void* qkv, const void* cos, const void* sin,
                                                 void* q_out, void* k_cache, void* v_cache, int batch,
                                                 int n_heads, int n_kv_heads, int head_dim, int max_len,
                                                 int pos, void* stream) {
    if (batch < 0 || n_heads < 0 || n_kv_heads < 0 || head_dim < 0 || max_len < 0)
        return invalid("negative dimension");
    if (head_dim % 2 != 0) return invalid("head_dim must be even");
    if (pos < 0 || pos >= max_len) return invalid("pos outside the cache");
    if ((long)batch * (n_heads + 2L * n_kv_heads) * head_dim > 0 &&
        (!qkv || !cos || !sin || !q_out || !k_cache || !v_cache))
        return invalid("null pointer");
    if ((long)batch * (n_heads + 2L * n_kv_heads) * (head_dim / 2) > 0xFFFFFFFFL * 256L)
        return invalid("too many heads");
    return launch_rope_qkv_append(qkv, cos, sin, q_out, k_cache, v_cache, batch, n_heads, n_kv_heads,
                                  head_dim, max_len, pos, as_stream(stream));
}

LLMIK_API llmik_status llmik_add_rmsnorm(const void* x, const void* residual, const void* weight,
                                         void* h_out, void* out, int rows, int hidden, float eps,
                                         void* stream) {
    if (rows < 0 || hidden < 0) return invalid("negative dimension");
    if (hidden % 8 != 0 || hidden > 8192) return invalid("hidden must be a multiple of 8 and at most 8192");
    if ((long)rows * hidden > 0 && (!x || !residual || !weight || !h_out || !out))
        return invalid("null pointer");
    if (!aligned(x, 16) || !aligned(residual, 16) || !aligned(weight, 16) || !aligned(h_out, 16) ||
        !aligned(out, 16))
        return set_error(LLMIK_ERR_ALIGNMENT, "add_rmsnorm tensors must be 16-byte aligned");
    return launch_add_rmsnorm(x, residual, weight, h_out, out, rows, hidden, eps, as_stream(stream));
}

LLMIK_API llmik_status llmik_silu_mul_halves(const void* gate_up, void* out, long rows, int cols,
                                             void* stream) {
    if (rows < 0 || cols < 0) return invalid("negative dimension");
    if (cols % 8 != 0) return invalid("cols must be a multiple of 8");
    if (rows * cols > 0 && (!gate_up || !out)) return invalid("null pointer");
    if ((rows * cols + 2047) / 2048 > 0xFFFFFFFFL) return invalid("too many values");
    if (!aligned(gate_up, 16) || !aligned(out, 16))
        return set_error(LLMIK_ERR_ALIGNMENT, "silu_mul_halves tensors must be 16-byte aligned");
    return launch_silu_mul_halves(gate_up, out, rows, cols, as_stream(stream));
}

}  // extern "C"
