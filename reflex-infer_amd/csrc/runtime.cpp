// runtime.cpp -- process-wide state of the library: the fp32 workspace of
// the split launches and the tuning overrides read from the environment.
//
// Workspace (split-K GEMM partials, small-batch K-split partials,
// decode-attention chunk partials):
// One buffer of kWorkspaceBytes per (device, stream), allocated the first
// time a split launch is enqueued on that stream and never resized or freed
// until the process ends.  Hence:
//   * a HIP graph captured on a stream keeps a valid workspace pointer for
//     the life of the process, whatever is launched later, on any stream;
//   * split launches on different streams never share memory; launches on
//     one stream are ordered by the stream itself;
//   * no entry point synchronises: the only runtime call is the one
//     hipMalloc per (device, stream), made with the calling thread's capture
//     mode set to relaxed so that it is also legal while the stream is
//     being captured (the allocation is not part of the graph).
// Every split launcher sizes its split count so that its partials fit.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "launch.h"

namespace rxq4 {

namespace {
std::mutex g_mutex;
std::map<std::pair<int, uintptr_t>, void *> *g_buffers = nullptr;  // never destroyed
}  // namespace

hipError_t stream_workspace(hipStream_t st, float **ws) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const auto key = std::make_pair(dev, reinterpret_cast<uintptr_t>(st));
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_buffers) g_buffers = new std::map<std::pair<int, uintptr_t>, void *>();
    auto it = g_buffers->find(key);
    if (it == g_buffers->end()) {
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        if ((e = hipThreadExchangeStreamCaptureMode(&mode)) != hipSuccess) return e;
        void *p = nullptr;
        e = hipMalloc(&p, kWorkspaceBytes);
        hipStreamCaptureMode back = mode;
        (void)hipThreadExchangeStreamCaptureMode(&back);
        if (e != hipSuccess) return e;
        it = g_buffers->emplace(key, p).first;
    }
    *ws = static_cast<float *>(it->second);
    return hipSuccess;
}

// Tuning overrides, read once (the first launch) and fixed for the process.
// Unset or non-positive values keep the launchers' own choices.
namespace {
int env_pos(const char *name) {
    const char *v = getenv(name);
    if (!v || !*v) return 0;
    const int r = atoi(v);
    return r > 0 ? r : 0;
}
bool env_off(const char *name) {
    const char *v = getenv(name);
    return v && v[0] == '0';
}
}  // namespace

const Tuning &tuning() {
    static const Tuning t = [] {
        Tuning r;
        r.gemm_splits = env_pos("RXQ4_GEMM_SPLITS");
        r.gemv_waves_per_cu = env_pos("RXQ4_GEMV_WAVES_PER_CU");
        r.gemv_lds_waves_per_cu = env_pos("RXQ4_GEMV_LDS_WAVES_PER_CU");
        r.attn_split = env_pos("RXQ4_ATTN_SPLIT");
        r.attn_mfma = !env_off("RXQ4_ATTN_MFMA");
        r.multi_token_gemv = env_off("RXQ4_MULTI_TOKEN_GEMV") ? 0
                             : env_pos("RXQ4_MULTI_TOKEN_GEMV") ? 1 : -1;
        r.gemm_tm = env_pos("RXQ4_GEMM_TM");
        r.gemm_order = env_pos("RXQ4_GEMM_ORDER");
        r.gemm_mixed = env_pos("RXQ4_GEMM_MIXED");
        r.tokens_waves = env_pos("RXQ4_TOKENS_WAVES");
        r.tokens_lds_split = env_pos("RXQ4_TOKENS_LDS_SPLIT");
        return r;
    }();
    return t;
}

int workspace_count() {
    std::lock_guard<std::mutex> lock(g_mutex);
    return g_buffers ? static_cast<int>(g_buffers->size()) : 0;
}

}  // namespace rxq4
