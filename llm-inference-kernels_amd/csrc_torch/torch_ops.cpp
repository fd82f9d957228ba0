// llmik_cuda._C: the torch-facing half of the llmik_cuda ops in C++.
//
// The reference binds its ops with pybind11 in bindings/extension.cpp: each
// op validates with TORCH_CHECK, allocates its outputs with torch and
// enqueues the launcher on the current stream. These functions do the same
// over the C ABI of libllmik_hip.so (include/llmik.h), so an eager call
// costs one binding call instead of Python-side validation, a ctypes call
// and Python stream / device-guard lookups. The Python wrappers in
// llmik_cuda/__init__.py keep the reference's signatures and check that the
// inputs are device tensors; everything after that check is here, with the
// same messages. Split-K workspaces are cached per (device, stream); a
// replaced buffer is kept alive because HIP graphs captured earlier on that
// stream still address it.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/llmik.h"

namespace {

using at::Tensor;

inline void* ptr(const Tensor& t) { return t.data_ptr(); }

inline hipStream_t stream_of(const Tensor& t) {
    return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

inline void check(llmik_status st) {
    TORCH_CHECK(st == LLMIK_OK, "llmik: ", llmik_last_error(), " (status ", st, ")");
}

// ---- per-(device, stream) workspace ------------------------------------------
// The kernels need the workspace's completion counters to be zero when they
// start and leave them zero when they end. A buffer created eagerly is zeroed
// before any kernel can use it, and is cached for the stream. A buffer created
// while the stream is capturing a graph is zeroed only inside that graph (the
// fill is recorded, not run), so it is right for that graph's replays alone:
// it is kept alive for them but never cached, and a later call (eager, or in
// another capture) on the stream gets a buffer of its own.
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Tensor> g_ws;
std::vector<Tensor> g_ws_retired;
std::vector<Tensor> g_ws_captured;

bool stream_is_capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(s, &cs);
    TORCH_CHECK(e == hipSuccess, "llmik: hipStreamIsCapturing failed: ", hipGetErrorString(e));
    return cs != hipStreamCaptureStatusNone;
}

std::pair<void*, size_t> workspace(const Tensor& like, hipStream_t s, size_t nbytes) {
    if (nbytes == 0) return {nullptr, 0};
    const std::pair<int, hipStream_t> key{like.get_device(), s};
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find(key);
    if (it == g_ws.end() || (size_t)it->second.numel() < nbytes) {
        if (stream_is_capturing(s)) {
            Tensor ws = at::zeros({(int64_t)nbytes}, like.options().dtype(at::kByte));
            g_ws_captured.push_back(ws);
            return {ws.data_ptr(), nbytes};
        }
        size_t size = nbytes;
        if (it != g_ws.end()) {
            size = std::max(nbytes, (size_t)(2 * it->second.numel()));
            g_ws_retired.push_back(it->second);
        }
        Tensor ws = at::zeros({(int64_t)size}, like.options().dtype(at::kByte));
        g_ws[key] = ws;
        return {ws.data_ptr(), size};
    }
    return {it->second.data_ptr(), (size_t)it->second.numel()};
}

py::dict workspaces() {
    py::dict d;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    for (const auto& kv : g_ws)
        d[py::make_tuple(kv.first.first, (uintptr_t)kv.first.second)] = kv.second;
    return d;
}

// ---------------------------------------------------------------- attention

Tensor decode_attention(const Tensor& q, const Tensor& k, const Tensor& v, double softmax_scale,
                        int64_t seqlen) {
    TORCH_CHECK(q.scalar_type() == at::kHalf, "fp16 only for now");
    TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(), "inputs must be contiguous");
    TORCH_CHECK(k.scalar_type() == at::kHalf && v.scalar_type() == at::kHalf, "k and v must be fp16");
    TORCH_CHECK(q.dim() == 3 && k.dim() == 4 && v.dim() == 4,
                "q must be [batch, n_heads, head_dim] and k/v [batch, n_kv_heads, S, head_dim]");
    TORCH_CHECK(k.sizes() == v.sizes(), "k and v must have the same shape");
    const int batch = q.size(0), n_heads = q.size(1), head_dim = q.size(2);
    const int n_kv_heads = k.size(1), kv_buf_len = k.size(2);
    TORCH_CHECK(k.size(0) == batch && k.size(3) == head_dim, "q and k/v shapes disagree");
    const int s = seqlen > 0 ? (int)seqlen : kv_buf_len;
    TORCH_CHECK(s <= kv_buf_len, "seqlen exceeds allocated cache length");
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "q, k, v must be CUDA tensors");
    const c10::DeviceGuard guard(q.device());
    Tensor out = at::empty_like(q);
    const hipStream_t st = stream_of(q);
    auto ws = workspace(q, st, llmik_attention_workspace_size(batch, n_heads, n_kv_heads, s, head_dim));
    check(llmik_decode_attention_f16(ptr(q), ptr(k), ptr(v), ptr(out), batch, n_heads, n_kv_heads, s,
                                     head_dim, kv_buf_len, (float)softmax_scale, ws.first, ws.second, st));
    return out;
}

Tensor decode_attention_int8(const Tensor& q, const Tensor& k_q, const Tensor& k_scale, const Tensor& v_q,
                             const Tensor& v_scale, double softmax_scale, int64_t seqlen) {
    TORCH_CHECK(q.scalar_type() == at::kHalf, "q must be fp16");
    TORCH_CHECK(k_q.scalar_type() == at::kChar && v_q.scalar_type() == at::kChar, "k_q and v_q must be int8");
    TORCH_CHECK(k_scale.scalar_type() == at::kHalf && v_scale.scalar_type() == at::kHalf,
                "k_scale and v_scale must be fp16");
    TORCH_CHECK(q.is_contiguous() && k_q.is_contiguous() && k_scale.is_contiguous() && v_q.is_contiguous() &&
                    v_scale.is_contiguous(), "all tensors must be contiguous");
    TORCH_CHECK(q.dim() == 3 && k_q.dim() == 4 && k_q.sizes() == v_q.sizes(),
                "q must be [batch, n_heads, head_dim] and k_q/v_q [batch, n_kv_heads, S, head_dim]");
    const int batch = q.size(0), n_heads = q.size(1), head_dim = q.size(2);
    const int n_kv_heads = k_q.size(1), kv_buf_len = k_q.size(2);
    TORCH_CHECK(k_q.size(0) == batch && k_q.size(3) == head_dim, "q and k_q/v_q shapes disagree");
    TORCH_CHECK(k_scale.dim() == 3 && k_scale.size(0) == batch && k_scale.size(1) == n_kv_heads &&
                    k_scale.size(2) == kv_buf_len && k_scale.sizes() == v_scale.sizes(),
                "k_scale/v_scale must be [batch, n_kv_heads, S]");
    const int s = seqlen > 0 ? (int)seqlen : kv_buf_len;
    TORCH_CHECK(s <= kv_buf_len, "seqlen exceeds allocated cache length");
    TORCH_CHECK(q.is_cuda() && k_q.is_cuda() && v_q.is_cuda() && k_scale.is_cuda() && v_scale.is_cuda(),
                "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(q.device());
    Tensor out = at::empty_like(q);
    const hipStream_t st = stream_of(q);
    auto ws = workspace(q, st, llmik_attention_workspace_size(batch, n_heads, n_kv_heads, s, head_dim));
    check(llmik_decode_attention_int8(ptr(q), ptr(k_q), ptr(k_scale), ptr(v_q), ptr(v_scale), ptr(out), batch,
                                      n_heads, n_kv_heads, s, head_dim, kv_buf_len, (float)softmax_scale,
                                      ws.first, ws.second, st));
    return out;
}

Tensor decode_attention_int4(const Tensor& q, const Tensor& k_q, const Tensor& k_scale, const Tensor& v_q,
                             const Tensor& v_scale, int64_t group_size, double softmax_scale, int64_t seqlen) {
    TORCH_CHECK(q.scalar_type() == at::kHalf, "q must be fp16");
    TORCH_CHECK(k_q.scalar_type() == at::kChar && v_q.scalar_type() == at::kChar,
                "k_q and v_q must be int8 (packed int4)");
    TORCH_CHECK(k_scale.scalar_type() == at::kHalf && v_scale.scalar_type() == at::kHalf,
                "k_scale and v_scale must be fp16");
    TORCH_CHECK(q.is_contiguous() && k_q.is_contiguous() && k_scale.is_contiguous() && v_q.is_contiguous() &&
                    v_scale.is_contiguous(), "all tensors must be contiguous");
    TORCH_CHECK(q.dim() == 3 && k_q.dim() == 4 && k_q.sizes() == v_q.sizes() && k_scale.dim() == 4,
                "q must be [batch, n_heads, head_dim], k_q/v_q [batch, n_kv_heads, S, head_dim/2]");
    const int batch = q.size(0), n_heads = q.size(1), head_dim = q.size(2);
    const int n_kv_heads = k_q.size(1), kv_buf_len = k_q.size(2);
    TORCH_CHECK(k_q.size(0) == batch && 2 * k_q.size(3) == head_dim, "q and k_q/v_q shapes disagree");
    const int n_groups = k_scale.size(2);
    TORCH_CHECK(k_scale.size(0) == batch && k_scale.size(1) == n_kv_heads && k_scale.size(3) == head_dim,
                "k_scale must be [batch, n_kv_heads, n_groups, head_dim]");
    TORCH_CHECK(v_scale.dim() == 3 && v_scale.size(0) == batch && v_scale.size(1) == n_kv_heads &&
                    v_scale.size(2) == kv_buf_len, "v_scale must be [batch, n_kv_heads, S]");
    TORCH_CHECK(group_size > 0, "group_size must be positive");
    const int s = seqlen > 0 ? (int)seqlen : kv_buf_len;
    TORCH_CHECK(s <= kv_buf_len, "seqlen exceeds allocated cache length");
    TORCH_CHECK(q.is_cuda() && k_q.is_cuda() && v_q.is_cuda() && k_scale.is_cuda() && v_scale.is_cuda(),
                "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(q.device());
    Tensor out = at::empty_like(q);
    const hipStream_t st = stream_of(q);
    auto ws = workspace(q, st, llmik_attention_workspace_size(batch, n_heads, n_kv_heads, s, head_dim));
    check(llmik_decode_attention_int4(ptr(q), ptr(k_q), ptr(k_scale), ptr(v_q), ptr(v_scale), ptr(out), batch,
                                      n_heads, n_kv_heads, s, head_dim, kv_buf_len, (int)group_size, n_groups,
                                      (float)softmax_scale, ws.first, ws.second, st));
    return out;
}

// ---------------------------------------------------------------- KV writers

void check_writer_input(const Tensor& x) {
    TORCH_CHECK(x.scalar_type() == at::kHalf, "x must be fp16");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    TORCH_CHECK(x.dim() == 4, "x must be [batch, n_kv_heads, seqlen, head_dim]");
    TORCH_CHECK(x.size(3) == 128, "only head_dim=128 supported");
}

std::tuple<Tensor, Tensor> quantize_per_token(const Tensor& x) {
    check_writer_input(x);
    const int b = x.size(0), h = x.size(1), s = x.size(2), d = x.size(3);
    TORCH_CHECK(x.is_cuda(), "x must be CUDA");
    const c10::DeviceGuard guard(x.device());
    Tensor q = at::empty({b, h, s, d}, x.options().dtype(at::kChar));
    Tensor scale = at::empty({b, h, s}, x.options());
    check(llmik_quantize_per_token_int8(ptr(x), ptr(q), ptr(scale), b, h, s, d, stream_of(x)));
    return {q, scale};
}

std::tuple<Tensor, Tensor> quantize_k_per_channel_groupwise_int4(const Tensor& x, int64_t group_size) {
    check_writer_input(x);
    TORCH_CHECK(group_size > 0, "group_size must be positive");
    const int b = x.size(0), h = x.size(1), s = x.size(2), d = x.size(3);
    const int n_groups = (s + (int)group_size - 1) / (int)group_size;
    TORCH_CHECK(x.is_cuda(), "x must be CUDA");
    const c10::DeviceGuard guard(x.device());
    Tensor q = at::empty({b, h, s, d / 2}, x.options().dtype(at::kChar));
    Tensor scale = at::empty({b, h, n_groups, d}, x.options());
    check(llmik_quantize_k_per_channel_groupwise_int4(ptr(x), ptr(q), ptr(scale), b, h, s, d, (int)group_size,
                                                      stream_of(x)));
    return {q, scale};
}

std::tuple<Tensor, Tensor> quantize_v_per_token_int4(const Tensor& x) {
    check_writer_input(x);
    const int b = x.size(0), h = x.size(1), s = x.size(2), d = x.size(3);
    TORCH_CHECK(x.is_cuda(), "x must be CUDA");
    const c10::DeviceGuard guard(x.device());
    Tensor q = at::empty({b, h, s, d / 2}, x.options().dtype(at::kChar));
    Tensor scale = at::empty({b, h, s}, x.options());
    check(llmik_quantize_v_per_token_int4(ptr(x), ptr(q), ptr(scale), b, h, s, d, stream_of(x)));
    return {q, scale};
}

// Token stride of x's (batch, kv_head) rows, in tokens: x is contiguous or a
// token slice buf[:, :, a:b] of a contiguous 4-D buffer.
int token_rows(const Tensor& x) {
    const int64_t batch = x.size(0), n_kv_heads = x.size(1), n_tok = x.size(2), head_dim = x.size(3);
    TORCH_CHECK(x.stride(3) == 1 && (n_tok <= 1 || x.stride(2) == head_dim),
                "x must be contiguous within each (batch, kv_head) row");
    int64_t row;
    if (n_kv_heads > 1) {
        row = x.stride(1);
        TORCH_CHECK(batch <= 1 || x.stride(0) == n_kv_heads * row,
                    "x rows must be equally spaced (a token slice of a contiguous buffer)");
    } else if (batch > 1) {
        row = x.stride(0);
    } else {
        row = n_tok * head_dim;
    }
    TORCH_CHECK(row % head_dim == 0 && row >= n_tok * head_dim,
                "x rows must be equally spaced (a token slice of a contiguous buffer)");
    return (int)(row / head_dim);
}

struct IntoDims { int batch, n_kv_heads, n_tok, head_dim, cache_len, x_len; };

IntoDims check_into(const Tensor& x, const Tensor& q_cache, const Tensor& scale_cache, int64_t offset,
                    bool packed) {
    TORCH_CHECK(x.scalar_type() == at::kHalf, "x must be fp16");
    TORCH_CHECK(q_cache.scalar_type() == at::kChar && scale_cache.scalar_type() == at::kHalf,
                "q_cache must be int8 and scale_cache fp16");
    TORCH_CHECK(x.dim() == 4 && q_cache.dim() == 4, "x must be [batch, n_kv_heads, n, head_dim] and q_cache 4-D");
    IntoDims d{(int)x.size(0), (int)x.size(1), (int)x.size(2), (int)x.size(3), 0, 0};
    TORCH_CHECK(d.head_dim == 128, "only head_dim=128 supported");
    TORCH_CHECK(q_cache.is_contiguous() && scale_cache.is_contiguous(), "q_cache and scale_cache must be contiguous");
    d.cache_len = q_cache.size(2);
    const int width = packed ? d.head_dim / 2 : d.head_dim;
    TORCH_CHECK(q_cache.size(0) == d.batch && q_cache.size(1) == d.n_kv_heads && q_cache.size(3) == width,
                "q_cache must be [batch, n_kv_heads, cache_len, ", width, "]");
    TORCH_CHECK(0 <= offset && offset + d.n_tok <= d.cache_len, "offset + n exceeds the cache length");
    d.x_len = token_rows(x);
    return d;
}

void quantize_per_token_into(const Tensor& x, const Tensor& q_cache, const Tensor& scale_cache, int64_t offset) {
    const IntoDims d = check_into(x, q_cache, scale_cache, offset, false);
    TORCH_CHECK(scale_cache.dim() == 3 && scale_cache.size(0) == d.batch && scale_cache.size(1) == d.n_kv_heads &&
                    scale_cache.size(2) == d.cache_len, "scale_cache must be [batch, n_kv_heads, cache_len]");
    TORCH_CHECK(x.is_cuda() && q_cache.is_cuda() && scale_cache.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(x.device());
    check(llmik_quantize_per_token_int8_into(ptr(x), d.x_len, ptr(q_cache), ptr(scale_cache), d.batch,
                                             d.n_kv_heads, d.n_tok, d.head_dim, d.cache_len, (int)offset,
                                             stream_of(x)));
}

void quantize_v_per_token_int4_into(const Tensor& x, const Tensor& q_cache, const Tensor& scale_cache,
                                    int64_t offset) {
    const IntoDims d = check_into(x, q_cache, scale_cache, offset, true);
    TORCH_CHECK(scale_cache.dim() == 3 && scale_cache.size(0) == d.batch && scale_cache.size(1) == d.n_kv_heads &&
                    scale_cache.size(2) == d.cache_len, "scale_cache must be [batch, n_kv_heads, cache_len]");
    TORCH_CHECK(x.is_cuda() && q_cache.is_cuda() && scale_cache.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(x.device());
    check(llmik_quantize_v_per_token_int4_into(ptr(x), d.x_len, ptr(q_cache), ptr(scale_cache), d.batch,
                                               d.n_kv_heads, d.n_tok, d.head_dim, d.cache_len, (int)offset,
                                               stream_of(x)));
}

void quantize_k_per_channel_groupwise_int4_into(const Tensor& x, const Tensor& q_cache, const Tensor& scale_cache,
                                                int64_t offset, int64_t group_size) {
    TORCH_CHECK(group_size > 0, "group_size must be positive");
    TORCH_CHECK(offset % group_size == 0, "offset must be a multiple of group_size");
    const IntoDims d = check_into(x, q_cache, scale_cache, offset, true);
    const int n_groups = (d.cache_len + (int)group_size - 1) / (int)group_size;
    TORCH_CHECK(scale_cache.dim() == 4 && scale_cache.size(0) == d.batch && scale_cache.size(1) == d.n_kv_heads &&
                    scale_cache.size(2) == n_groups && scale_cache.size(3) == d.head_dim,
                "scale_cache must be [batch, n_kv_heads, ceil(cache_len/group_size), head_dim]");
    TORCH_CHECK(x.is_cuda() && q_cache.is_cuda() && scale_cache.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(x.device());
    check(llmik_quantize_k_per_channel_groupwise_int4_into(ptr(x), d.x_len, ptr(q_cache), ptr(scale_cache), d.batch,
                                                           d.n_kv_heads, d.n_tok, d.head_dim, d.cache_len,
                                                           (int)offset, (int)group_size, stream_of(x)));
}

void kivi_append_token_int4(const Tensor& k, const Tensor& v, const Tensor& k_open, const Tensor& k_q,
                            const Tensor& k_scale, const Tensor& v_q, const Tensor& v_scale, int64_t length,
                            int64_t group_size) {
    TORCH_CHECK(k.scalar_type() == at::kHalf && v.scalar_type() == at::kHalf && k_open.scalar_type() == at::kHalf,
                "k, v and k_open must be fp16");
    TORCH_CHECK(k.dim() == 4 && v.dim() == 4 && k.size(0) == v.size(0) && k.size(1) == v.size(1) &&
                    k.size(3) == 128 && v.size(3) == 128, "k and v must be [batch, n_kv_heads, n, 128]");
    TORCH_CHECK(group_size > 0, "group_size must be positive");
    const int batch = k.size(0), n_kv_heads = k.size(1);
    const int max_len = k_q.dim() == 4 ? (int)k_q.size(2) : 0;
    const int n_groups = (max_len + (int)group_size - 1) / (int)group_size;
    TORCH_CHECK(k_q.dim() == 4 && k_q.size(0) == batch && k_q.size(1) == n_kv_heads && k_q.size(3) == 64 &&
                    k_q.sizes() == v_q.sizes() && k_q.scalar_type() == at::kChar && v_q.scalar_type() == at::kChar,
                "k_q / v_q must be [batch, n_kv_heads, max_len, 64] int8");
    TORCH_CHECK(k_scale.dim() == 4 && k_scale.size(0) == batch && k_scale.size(1) == n_kv_heads &&
                    k_scale.size(2) == n_groups && k_scale.size(3) == 128 && v_scale.dim() == 3 &&
                    v_scale.size(0) == batch && v_scale.size(1) == n_kv_heads && v_scale.size(2) == max_len &&
                    k_scale.scalar_type() == at::kHalf && v_scale.scalar_type() == at::kHalf,
                "k_scale / v_scale must be fp16 and match the cache's shape");
    TORCH_CHECK(k_open.dim() == 4 && k_open.size(0) == batch && k_open.size(1) == n_kv_heads &&
                    k_open.size(2) == group_size && k_open.size(3) == 128,
                "k_open must be [batch, n_kv_heads, group_size, 128]");
    TORCH_CHECK(k_open.is_contiguous() && k_q.is_contiguous() && k_scale.is_contiguous() && v_q.is_contiguous() &&
                    v_scale.is_contiguous(), "cache tensors must be contiguous");
    const int k_len = token_rows(k), v_len = token_rows(v);
    TORCH_CHECK(k.is_cuda() && v.is_cuda() && k_open.is_cuda() && k_q.is_cuda() && k_scale.is_cuda() &&
                    v_q.is_cuda() && v_scale.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(k.device());
    check(llmik_kivi_append_token_int4(ptr(k), k_len, ptr(v), v_len, ptr(k_open), ptr(k_q), ptr(k_scale), ptr(v_q),
                                       ptr(v_scale), batch, n_kv_heads, 128, max_len, (int)group_size, (int)length,
                                       stream_of(k)));
}

// -------------------------------------------------------------------- W4A16

Tensor gemm(const Tensor& act, const Tensor& weight_packed, const Tensor& scale, int64_t group_size, bool f32) {
    TORCH_CHECK(act.scalar_type() == at::kHalf, "act must be fp16");
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt, "weight_packed must be int32 (uint32 bit pattern)");
    TORCH_CHECK(scale.scalar_type() == at::kHalf, "scale must be fp16");
    TORCH_CHECK(act.is_contiguous() && weight_packed.is_contiguous() && scale.is_contiguous(),
                "all tensors must be contiguous");
    TORCH_CHECK(act.dim() == 2 && weight_packed.dim() == 2 && scale.dim() == 2, "all inputs must be 2D");
    const int M = act.size(0), K = act.size(1);
    const int k_packs = weight_packed.size(0), N = weight_packed.size(1);
    const int n_groups = scale.size(0);
    TORCH_CHECK(K == k_packs * 8, "act.K must equal weight_packed.K_packs * 8");
    TORCH_CHECK(scale.size(1) == N, "scale and weight_packed N mismatch");
    TORCH_CHECK(group_size > 0 && group_size % 8 == 0, "group_size must be a positive multiple of 8");
    TORCH_CHECK(K == n_groups * group_size, "K must equal n_groups * group_size");
    TORCH_CHECK(act.is_cuda() && weight_packed.is_cuda() && scale.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(act.device());
    Tensor out = at::empty({M, N}, act.options().dtype(f32 ? at::kFloat : at::kHalf));
    if (M == 0 || N == 0) return out;
    if (K == 0) return out.zero_();
    const hipStream_t st = stream_of(act);
    auto ws = workspace(act, st, llmik_w4a16_workspace_size(M, N, K, (int)group_size));
    check((f32 ? llmik_w4a16_gemm_f32out : llmik_w4a16_gemm)(ptr(act), ptr(weight_packed), ptr(scale), ptr(out), M,
                                                             N, K, (int)group_size, ws.first, ws.second, st));
    return out;
}

Tensor w4a16_gemm(const Tensor& act, const Tensor& weight_packed, const Tensor& scale, int64_t group_size) {
    return gemm(act, weight_packed, scale, group_size, false);
}

Tensor w4a16_gemm_qkv_rope(const Tensor& act, const Tensor& weight_packed, const Tensor& scale, const Tensor& cos,
                          const Tensor& sin, const Tensor& k_cache, const Tensor& v_cache, int64_t pos,
                          int64_t n_heads, int64_t group_size) {
    TORCH_CHECK(act.scalar_type() == at::kHalf && scale.scalar_type() == at::kHalf && cos.scalar_type() == at::kHalf &&
                    sin.scalar_type() == at::kHalf && k_cache.scalar_type() == at::kHalf &&
                    v_cache.scalar_type() == at::kHalf,
                "act, scale, cos, sin and the caches must be fp16");
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt, "weight_packed must be int32 (uint32 bit pattern)");
    TORCH_CHECK(act.is_contiguous() && weight_packed.is_contiguous() && scale.is_contiguous() && cos.is_contiguous() &&
                    sin.is_contiguous() && k_cache.is_contiguous() && v_cache.is_contiguous(),
                "all tensors must be contiguous");
    TORCH_CHECK(act.dim() == 2 && weight_packed.dim() == 2 && scale.dim() == 2, "act and weights must be 2D");
    TORCH_CHECK(k_cache.dim() == 4 && k_cache.size(3) == 128 && v_cache.sizes() == k_cache.sizes(),
                "k_cache and v_cache must be [batch, n_kv_heads, max_len, 128] of one shape");
    TORCH_CHECK(cos.numel() == 128 && sin.numel() == 128, "cos and sin must be the position's 128 values");
    const int M = act.size(0), K = act.size(1);
    const int Hkv = k_cache.size(1), max_len = k_cache.size(2);
    TORCH_CHECK(k_cache.size(0) == M, "the caches' batch must equal act's rows");
    TORCH_CHECK(n_heads > 0 && n_heads % Hkv == 0, "n_heads must be a positive multiple of n_kv_heads");
    const int N = (n_heads + 2 * Hkv) * 128;
    TORCH_CHECK(weight_packed.size(1) == N && scale.size(1) == N, "weight N must be (n_heads + 2 n_kv_heads) * 128");
    TORCH_CHECK(K == weight_packed.size(0) * 8, "act.K must equal weight_packed.K_packs * 8");
    TORCH_CHECK(group_size > 0 && group_size % 8 == 0 && K == scale.size(0) * group_size,
                "K must equal n_groups * group_size");
    TORCH_CHECK(pos >= 0 && pos < max_len, "pos outside the cache");
    TORCH_CHECK(act.is_cuda() && weight_packed.is_cuda() && scale.is_cuda() && cos.is_cuda() && sin.is_cuda() &&
                    k_cache.is_cuda() && v_cache.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(act.device());
    Tensor q = at::empty({M, n_heads, 128}, act.options());
    if (M == 0) return q;
    const hipStream_t st = stream_of(act);
    auto ws = workspace(act, st, llmik_w4a16_qkv_rope_workspace_size(M, (int)n_heads, Hkv, K, (int)group_size));
    check(llmik_w4a16_gemm_qkv_rope_f16(ptr(act), ptr(weight_packed), ptr(scale), ptr(cos), ptr(sin), ptr(q),
                                        ptr(k_cache), ptr(v_cache), M, K, (int)group_size, (int)n_heads, Hkv,
                                        max_len, (int)pos, ws.first, ws.second, st));
    return q;
}

Tensor w4a16_gemm_swiglu(const Tensor& act, const Tensor& weight_packed, const Tensor& scale, int64_t group_size) {
    TORCH_CHECK(act.scalar_type() == at::kHalf, "act must be fp16");
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt, "weight_packed must be int32 (uint32 bit pattern)");
    TORCH_CHECK(scale.scalar_type() == at::kHalf, "scale must be fp16");
    TORCH_CHECK(act.is_contiguous() && weight_packed.is_contiguous() && scale.is_contiguous(),
                "all tensors must be contiguous");
    TORCH_CHECK(act.dim() == 2 && weight_packed.dim() == 2 && scale.dim() == 2, "all inputs must be 2D");
    const int M = act.size(0), K = act.size(1);
    const int N = weight_packed.size(1);
    TORCH_CHECK(K == weight_packed.size(0) * 8, "act.K must equal weight_packed.K_packs * 8");
    TORCH_CHECK(scale.size(1) == N, "scale and weight_packed N mismatch");
    TORCH_CHECK(group_size > 0 && group_size % 8 == 0, "group_size must be a positive multiple of 8");
    TORCH_CHECK(K == scale.size(0) * group_size, "K must equal n_groups * group_size");
    TORCH_CHECK(N % 64 == 0, "the interleaved gate|up weight needs N % 64 == 0");
    TORCH_CHECK(act.is_cuda() && weight_packed.is_cuda() && scale.is_cuda(), "all inputs must be CUDA tensors");
    const c10::DeviceGuard guard(act.device());
    Tensor out = at::empty({M, N / 2}, act.options());
    if (M == 0) return out;
    const hipStream_t st = stream_of(act);
    auto ws = workspace(act, st, llmik_w4a16_swiglu_workspace_size(M, N, K, (int)group_size));
    check(llmik_w4a16_gemm_swiglu(ptr(act), ptr(weight_packed), ptr(scale), ptr(out), M, N, K, (int)group_size,
                                  ws.first, ws.second, st));
    return out;
}

Tensor w4a16_gemm_f32out(const Tensor& act, const Tensor& weight_packed, const Tensor& scale, int64_t group_size) {
    return gemm(act, weight_packed, scale, group_size, true);
}

Tensor w4a16_dequantize(const Tensor& weight_packed, const Tensor& scale, int64_t group_size) {
    TORCH_CHECK(weight_packed.scalar_type() == at::kInt, "weight_packed int32");
    TORCH_CHECK(scale.scalar_type() == at::kHalf, "scale fp16");
    TORCH_CHECK(weight_packed.is_contiguous() && scale.is_contiguous(), "contiguous");
    TORCH_CHECK(weight_packed.dim() == 2 && scale.dim() == 2, "weight_packed and scale must be 2D");
    const int K = weight_packed.size(0) * 8, N = weight_packed.size(1);
    TORCH_CHECK(scale.size(1) == N, "scale/weight N mismatch");
    TORCH_CHECK(group_size > 0 && K % group_size == 0, "K must be a multiple of group_size");
    TORCH_CHECK(scale.size(0) * group_size == K, "scale must have K / group_size rows");
    TORCH_CHECK(weight_packed.is_cuda() && scale.is_cuda(), "inputs must be CUDA");
    const c10::DeviceGuard guard(scale.device());
    Tensor out = at::empty({K, N}, scale.options());
    check(llmik_w4a16_dequantize(ptr(weight_packed), ptr(scale), ptr(out), K, N, (int)group_size, stream_of(scale)));
    return out;
}

// ------------------------------------------------------ fused elementwise ops

Tensor rmsnorm(const Tensor& x, const Tensor& weight, double eps) {
    TORCH_CHECK(x.scalar_type() == at::kHalf && weight.scalar_type() == at::kHalf, "fp16 only");
    const int64_t H = x.size(-1);
    TORCH_CHECK(weight.numel() == H, "weight length must match x last dim");
    TORCH_CHECK(x.is_cuda() && weight.is_cuda(), "inputs must be CUDA");
    const c10::DeviceGuard guard(x.device());
    Tensor x2 = x.contiguous().reshape({-1, H});
    Tensor w = weight.contiguous();
    Tensor out = at::empty_like(x2);
    check(llmik_rmsnorm(ptr(x2), ptr(w), ptr(out), (int)x2.size(0), (int)H, (float)eps, stream_of(x)));
    return out.reshape(x.sizes());
}

Tensor silu_mul(const Tensor& gate, const Tensor& up) {
    TORCH_CHECK(gate.scalar_type() == at::kHalf && up.scalar_type() == at::kHalf, "fp16 only");
    TORCH_CHECK(gate.sizes() == up.sizes(), "gate and up must have the same shape");
    TORCH_CHECK(gate.is_cuda() && up.is_cuda(), "inputs must be CUDA");
    const c10::DeviceGuard guard(gate.device());
    Tensor g = gate.contiguous(), u = up.contiguous();
    Tensor out = at::empty_like(g);
    check(llmik_silu_mul(ptr(g), ptr(u), ptr(out), (long)g.numel(), stream_of(gate)));
    return out;
}

Tensor rope(const Tensor& x, const Tensor& cos, const Tensor& sin) {
    TORCH_CHECK(x.scalar_type() == at::kHalf, "fp16 only");
    TORCH_CHECK(x.dim() == 4, "x must be [B, H, S, D]");
    const int64_t B = x.size(0), H = x.size(1), S = x.size(2), D = x.size(3);
    TORCH_CHECK(D % 2 == 0, "head_dim must be even");
    TORCH_CHECK(cos.scalar_type() == at::kHalf && sin.scalar_type() == at::kHalf, "fp16 only");
    auto norm_cs = [&](const Tensor& t) {
        Tensor c = t.contiguous();
        if (c.numel() == B * S * D) return c.reshape({B, S, D});
        TORCH_CHECK(c.numel() == S * D, "cos/sin must be [B,S,D] or broadcastable [S,D]/[1,S,D]");
        return c.reshape({1, S, D}).expand({B, S, D}).contiguous();
    };
    Tensor cc = norm_cs(cos), sc = norm_cs(sin);
    TORCH_CHECK(x.is_cuda() && cos.is_cuda() && sin.is_cuda(), "inputs must be CUDA");
    const c10::DeviceGuard guard(x.device());
    Tensor xc = x.contiguous();
    Tensor out = at::empty_like(xc);
    check(llmik_rope(ptr(xc), ptr(cc), ptr(sc), ptr(out), (int)B, (int)H, (int)S, (int)D, stream_of(x)));
    return out;
}

// ------------------------------------------------------ decode-step merges

Tensor rope_qkv_append(const Tensor& qkv, const Tensor& cos, const Tensor& sin, const Tensor& k_cache,
                       const Tensor& v_cache, int64_t pos) {
    TORCH_CHECK(qkv.scalar_type() == at::kHalf && cos.scalar_type() == at::kHalf && sin.scalar_type() == at::kHalf &&
                    k_cache.scalar_type() == at::kHalf && v_cache.scalar_type() == at::kHalf, "fp16 only");
    TORCH_CHECK(k_cache.dim() == 4 && k_cache.sizes() == v_cache.sizes() && k_cache.is_contiguous() &&
                    v_cache.is_contiguous(), "caches must be contiguous [batch, n_kv_heads, max_len, head_dim]");
    const int64_t B = k_cache.size(0), Hkv = k_cache.size(1), max_len = k_cache.size(2), D = k_cache.size(3);
    TORCH_CHECK(D % 2 == 0, "head_dim must be even");
    TORCH_CHECK(cos.numel() == D && sin.numel() == D, "cos/sin must be one [head_dim] row");
    TORCH_CHECK(qkv.size(0) == B && qkv.numel() % (B * D) == 0, "qkv must be [batch, heads * head_dim]");
    const int64_t H = qkv.numel() / (B * D) - 2 * Hkv;
    TORCH_CHECK(H > 0, "qkv holds fewer than 2 n_kv_heads + 1 heads");
    TORCH_CHECK(0 <= pos && pos < max_len, "pos outside the cache");
    TORCH_CHECK(qkv.is_cuda() && cos.is_cuda() && sin.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda(),
                "inputs must be CUDA");
    const c10::DeviceGuard guard(qkv.device());
    Tensor x = qkv.contiguous(), cc = cos.contiguous(), sc = sin.contiguous();
    Tensor q = at::empty({B, H, D}, qkv.options());
    check(llmik_rope_qkv_append_f16(ptr(x), ptr(cc), ptr(sc), ptr(q), ptr(k_cache), ptr(v_cache), (int)B, (int)H,
                                    (int)Hkv, (int)D, (int)max_len, (int)pos, stream_of(qkv)));
    return q;
}

std::tuple<Tensor, Tensor> add_rmsnorm(const Tensor& x, const Tensor& residual, const Tensor& weight, double eps) {
    TORCH_CHECK(x.scalar_type() == at::kHalf && residual.scalar_type() == at::kHalf &&
                    weight.scalar_type() == at::kHalf, "fp16 only");
    TORCH_CHECK(x.sizes() == residual.sizes(), "x and residual must have the same shape");
    const int64_t Hd = x.size(-1);
    TORCH_CHECK(weight.numel() == Hd, "weight length must match x last dim");
    TORCH_CHECK(x.is_cuda() && residual.is_cuda() && weight.is_cuda(), "inputs must be CUDA");
    const c10::DeviceGuard guard(x.device());
    Tensor x2 = x.contiguous().reshape({-1, Hd}), r2 = residual.contiguous().reshape({-1, Hd});
    Tensor w = weight.contiguous();
    Tensor h = at::empty_like(x2), out = at::empty_like(x2);
    check(llmik_add_rmsnorm(ptr(x2), ptr(r2), ptr(w), ptr(h), ptr(out), (int)x2.size(0), (int)Hd, (float)eps,
                            stream_of(x)));
    return {h.reshape(x.sizes()), out.reshape(x.sizes())};
}

Tensor silu_mul_halves(const Tensor& gate_up) {
    TORCH_CHECK(gate_up.scalar_type() == at::kHalf, "fp16 only");
    TORCH_CHECK(gate_up.size(-1) % 16 == 0, "the last dim must be 2 * cols with cols a multiple of 8");
    TORCH_CHECK(gate_up.is_cuda(), "inputs must be CUDA");
    const c10::DeviceGuard guard(gate_up.device());
    const int64_t cols = gate_up.size(-1) / 2;
    Tensor gu = gate_up.contiguous();
    const int64_t rows = cols ? gu.numel() / (2 * cols) : 0;
    std::vector<int64_t> shape(gu.sizes().begin(), gu.sizes().end());
    shape.back() = cols;
    Tensor out = at::empty(shape, gu.options());
    check(llmik_silu_mul_halves(ptr(gu), ptr(out), (long)rows, (int)cols, stream_of(gate_up)));
    return out;
}

}  // namespace

PYBIND11_MODULE(_C, m) {
    m.doc() = "torch-facing half of the llmik_cuda ops (validation, outputs, stream) over libllmik_hip.so";
    m.def("decode_attention", &decode_attention);
    m.def("decode_attention_int8", &decode_attention_int8);
    m.def("decode_attention_int4", &decode_attention_int4);
    m.def("quantize_per_token", &quantize_per_token);
    m.def("quantize_k_per_channel_groupwise_int4", &quantize_k_per_channel_groupwise_int4);
    m.def("quantize_v_per_token_int4", &quantize_v_per_token_int4);
    m.def("quantize_per_token_into", &quantize_per_token_into);
    m.def("quantize_v_per_token_int4_into", &quantize_v_per_token_int4_into);
    m.def("quantize_k_per_channel_groupwise_int4_into", &quantize_k_per_channel_groupwise_int4_into);
    m.def("kivi_append_token_int4", &kivi_append_token_int4);
    m.def("w4a16_gemm", &w4a16_gemm);
    m.def("w4a16_gemm_f32out", &w4a16_gemm_f32out);
    m.def("w4a16_gemm_swiglu", &w4a16_gemm_swiglu);
    m.def("w4a16_gemm_qkv_rope", &w4a16_gemm_qkv_rope);
    m.def("w4a16_dequantize", &w4a16_dequantize);
    m.def("rmsnorm", &rmsnorm);
    m.def("silu_mul", &silu_mul);
    m.def("rope", &rope);
    m.def("rope_qkv_append", &rope_qkv_append);
    m.def("add_rmsnorm", &add_rmsnorm);
    m.def("silu_mul_halves", &silu_mul_halves);
    m.def("workspaces", &workspaces);
    m.def("token_rows", &token_rows);
}
