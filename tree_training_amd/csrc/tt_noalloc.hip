// tt_attn_bwd_noalloc: the tree-attention backward for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). It runs exactly tt_attn_bwd, with the
// workspace taken from a file-scope device array instead of a caller argument.
//
// The array is a host-side stand-in in host code: its device address differs
// per GPU and is only known through hipGetSymbolAddress, looked up once per
// device (with that device current) on the first call there and cached. Only
// that address is ever handed to kernels.
#include <atomic>
#include <mutex>

#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr size_t kScratchBytes = (size_t)TT_NOALLOC_SCRATCH_MB << 20;

// One copy per GPU, held from module load until the process ends.
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch array.
int scratch_ptr(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TT_E_HIP;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* q = nullptr;
            if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return TT_E_HIP;
            g_scratch_ptr[dev].store(q, std::memory_order_release);
            p = q;
        }
    }
    *out = p;
    return TT_OK;
}

}  // namespace

extern "C" {

size_t tt_noalloc_scratch_bytes(void) { return kScratchBytes; }

int tt_attn_bwd_noalloc(const tt_attn_problem* p, const void* o, const float* lse, tt_tensor d_o, void* dq,
                        void* dk, void* dv, float* dk_past_acc, float* dv_past_acc, void* stream) {
    const size_t need = tt_attn_bwd_workspace_bytes(p);
    if (need == 0) return TT_E_ARG;
    if (need > kScratchBytes) return TT_E_WORKSPACE;
    void* ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc != TT_OK) return rc;
    // tt_attn_bwd validates everything else before its first launch; every
    // workspace word it reads was written earlier in the same call (delta by
    // the dQ or delta pass, the split-tile sums zeroed by a kernel before the
    // dK/dV pass), except delta across a split TT_BWD_* sequence of calls.
    return tt_attn_bwd(p, o, lse, d_o, dq, dk, dv, dk_past_acc, dv_past_acc, ws, need, stream);
}

}  // extern "C"
