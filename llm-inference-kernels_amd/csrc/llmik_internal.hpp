// Host-side declarations shared by the kernel translation units and the
// C ABI layer (capi.cpp). Not part of the public interface.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/llmik.h"

namespace llmik {

constexpr int kMaxAttnSplits = 256;
// Completion counters live in a fixed region at the start of every
// workspace; split partials always start after it, so counters of one call
// never alias partials of another.
constexpr size_t kCounterBytes = LLMIK_WORKSPACE_COUNTER_BYTES;
constexpr long kMaxCounters = (long)(kCounterBytes / sizeof(uint32_t));

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const char* msg);
// Converts hipGetLastError() after a launch into an llmik_status.
int check_launch();
// Compute units of the current device (cached per device).
int device_cu_count();

// ---- attention -------------------------------------------------------------
struct AttnPlan {
    int hpw;             // query heads per workgroup
    int n_hchunks;       // head chunks per kv head
    int n_splits;        // KV splits per (batch, kv head, head chunk)
    int chunk;           // tokens per split (multiple of 32 * waves)
    int waves;           // waves per MFMA workgroup (4 or 8)
    long n_slot_groups;  // batch * n_kv_heads * n_hchunks
    size_t workspace_bytes;
    size_t off_ml, off_o;
};

AttnPlan plan_attention(int batch, int n_heads, int n_kv_heads, int seqlen);
// fp16 tile size knob (see llmik_attention_set_plan_override).
void set_attention_plan_override(int f16_half_tiles);
// W4A16 plan knobs (see llmik_w4a16_set_plan_override).
void set_w4a16_plan_override(int stream_mode, int stream_splits);

struct AttnLaunch {
    const void* q;
    const void* k;
    const void* v;
    const void* k_scale;
    const void* v_scale;
    void* out;
    int batch, n_heads, n_kv_heads, seqlen, kv_buf_len;
    int group_size, n_groups;
    float softmax_scale;
    void* workspace;
    size_t workspace_bytes;
};

int launch_attention_f16(const AttnLaunch& a, hipStream_t stream);
int launch_attention_i8(const AttnLaunch& a, hipStream_t stream);
int launch_attention_i4(const AttnLaunch& a, hipStream_t stream);

// ---- KV writers ------------------------------------------------------------
// rows = batch * n_kv_heads; tokens [0, n_tok) of each row of x (token
// stride src_len) go to cache positions dst_off + t (token stride dst_len).
int launch_quantize_per_token(const void* x, void* q, void* scale, int rows, int n_tok,
                              int src_len, int dst_len, int dst_off, int qmax, bool pack4,
                              hipStream_t stream);
// As above for K per channel, group-wise; dst_off % group_size == 0 and the
// scale cache holds dst_groups groups per row.
int launch_quantize_k_groupwise_int4(const void* x, void* q, void* scale, int rows, int n_tok,
                                     int src_len, int dst_len, int dst_off, int dst_groups,
                                     int group_size, hipStream_t stream);
int launch_kivi_append_token(const void* k, long k_stride, const void* v, long v_stride, void* k_open,
                             void* k_q, void* k_scale, void* v_q, void* v_scale, int rows, int r,
                             int pos, int group_size, int max_len, int n_groups, hipStream_t stream);

// ---- W4A16 -----------------------------------------------------------------
struct GemmPlan {
    int kind;          // 0: single-row VALU GEMV, 1: tiled multi-row VALU,
                       // 2: single-row MFMA GEMV, 3: multi-row MFMA GEMM,
                       // 4: MFMA GEMV over up to 16 rows,
                       // 5: streaming MFMA GEMV, 1 <= M <= 16, N % 64 == 0
                       // 6: 32x32x16 MFMA GEMM, M > 16, N % 128 == 0
                       // 7: 32x32x16 MFMA GEMM, both operands in LDS, M >= 256, N % 128 == 0, K % 64 == 0
    int cols_per_lane; // 4 (16-byte weight loads) or 1
    int tile_n;        // output columns per workgroup
    int tile_m;        // output rows per workgroup
    int n_tiles, m_tiles;
    int splits;        // K splits
    int kp_per_split;  // packed K rows (8 K each) per split
    int waves;         // kinds 5, 6: waves per workgroup
    int wave_steps;    // kinds 5, 6: 32-K steps per wave; kind 7: 64-K stages per split
    int full_tiles;    // kind 7: leading tiles computed unsplit
    int split_tiles;   // kind 7: tiles computed in `splits` K splits
    size_t workspace_bytes;
    size_t off_part;
};

GemmPlan plan_w4a16(int M, int N, int K, int group_size);
GemmPlan plan_w4a16_stream_forced(int M, int N, int K, int group_size);
int launch_w4a16_swiglu(const void* act, const void* w, const void* scale, void* out, int M, int N,
                        int K, int group_size, void* ws, size_t ws_bytes, hipStream_t stream);
int launch_w4a16_qkv_rope(const void* act, const void* w, const void* scale, const void* cs, const void* sn,
                          void* q_out, void* k_cache, void* v_cache, int M, int K, int group_size,
                          int n_heads, int n_kv_heads, int max_len, int pos, void* ws, size_t ws_bytes,
                          hipStream_t stream);
int launch_w4a16(const void* act, const void* w, const void* scale, void* out, bool f32_out,
                 int M, int N, int K, int group_size, void* ws, size_t ws_bytes,
                 hipStream_t stream);
int launch_w4a16_dequantize(const void* w, const void* scale, void* out, int K, int N,
                            int group_size, hipStream_t stream);
// Group-wise INT4 weight quantiser (any of q / packed / scale / scale_f16
// may be null; packed needs K % 8 == 0 and group_size % 8 == 0).
int launch_quantize_weights_int4(const void* W, bool w_fp16, int K, int N, int group_size, void* q,
                                 void* packed, void* scale, void* scale_f16, hipStream_t stream);
int launch_pack_int4_along_k(const void* q, int K, int N, void* packed, hipStream_t stream);

// ---- fused elementwise -----------------------------------------------------
int launch_rmsnorm(const void* x, const void* w, void* out, int rows, int hidden, float eps,
                   hipStream_t stream);
int launch_silu_mul(const void* g, const void* u, void* out, long n, hipStream_t stream);
int launch_rope(const void* x, const void* cs, const void* sn, void* out, int B, int H, int S,
                int D, hipStream_t stream);
// decode-step merges of the ops above
int launch_rope_qkv_append(const void* qkv, const void* cs, const void* sn, void* q_out, void* kbuf,
                           void* vbuf, int B, int H, int Hkv, int D, int max_len, int pos,
                           hipStream_t stream);
int launch_add_rmsnorm(const void* x, const void* r, const void* w, void* h_out, void* out, int rows,
                       int hidden, float eps, hipStream_t stream);
int launch_silu_mul_halves(const void* gu, void* out, long rows, int cols, hipStream_t stream);

}  // namespace llmik
