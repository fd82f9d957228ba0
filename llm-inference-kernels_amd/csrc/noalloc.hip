// Allocation-free form of the fp16 decode attention entry point, for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc). It runs the same kernels
// as llmik_decode_attention_f16, with the split-K workspace (completion
// counters and split partials) in a file-scope device array instead of a
// caller-supplied buffer.
//
// The array is `scratch` below. Its host-side name is only a stand-in for
// the symbol, not a device address, so host code never passes it anywhere:
// the first call on each device resolves the device copy's address with
// hipGetSymbolAddress (with that device current) and keeps it per device.
//
// Contents between calls: the counter region (the first
// LLMIK_WORKSPACE_COUNTER_BYTES) is zero when the code object loads (static
// storage) and every call leaves it zero again; the partials past it are
// overwritten before they are read. Calls on one device share one array, so
// calls that overlap on a device (different streams, or host threads without
// ordering) race and must not be issued.
#include <hip/hip_runtime.h>

#include <mutex>

#include "llmik_internal.hpp"

// 2 MiB: the largest attention workspace on a 256-CU MI355X is ~1.05 MiB
// (fewer than 2 x CUs split slots of up to 4 heads x 130 fp32, plus the
// counters); devices with more CUs keep the same margin up to ~480 CUs.
static_assert(LLMIK_NOALLOC_SCRATCH_BYTES == (2u << 20), "scratch size is part of the ABI");
static __device__ __align__(256) unsigned char scratch[LLMIK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices] = {};   // per device: the device address of `scratch`

// Device address of this device's copy of `scratch`, resolved once per device
// with that device current.
int scratch_for_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return llmik::set_error(static_cast<int>(e), "hipGetDevice failed");
    }
    if (dev < 0 || dev >= kMaxDevices)
        return llmik::set_error(LLMIK_ERR_UNSUPPORTED, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            (void)hipGetLastError();
            return llmik::set_error(e != hipSuccess ? static_cast<int>(e) : LLMIK_ERR_WORKSPACE,
                                    "hipGetSymbolAddress(scratch) failed");
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return LLMIK_OK;
}

}  // namespace

extern "C" {

LLMIK_API llmik_status llmik_decode_attention_f16_noalloc(
    const void* q, const void* k, const void* v, void* out, int batch, int n_heads,
    int n_kv_heads, int seqlen, int head_dim, int kv_buf_len, float softmax_scale, void* stream) {
    // Shape errors are reported by the shared entry point (a zero-size
    // query below returns 0 for them, and they are re-checked there).
    const size_t need = llmik_attention_workspace_size(batch, n_heads, n_kv_heads, seqlen, head_dim);
    if (need > LLMIK_NOALLOC_SCRATCH_BYTES) {
        return llmik::set_error(LLMIK_ERR_WORKSPACE,
                                "llmik_decode_attention_f16_noalloc: this call needs more split-K "
                                "workspace than the 2 MiB static scratch; use "
                                "llmik_decode_attention_f16 with a workspace");
    }
    void* ws = nullptr;
    if (need > 0) {
        const int st = scratch_for_current_device(&ws);
        if (st != LLMIK_OK) return st;
    }
    return llmik_decode_attention_f16(q, k, v, out, batch, n_heads, n_kv_heads, seqlen, head_dim,
                                      kv_buf_len, softmax_scale, ws, need > 0 ? LLMIK_NOALLOC_SCRATCH_BYTES : 0,
                                      stream);
}

}  // extern "C"
