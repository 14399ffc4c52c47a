// runtime.cpp -- process-wide state of the library: the fp32 workspace of
// the split launches and the tuning overrides read from the environment.
//
// Workspace (split-K GEMM partials, small-batch K-split partials,
// decode-attention chunk partials):
// One buffer of kWorkspaceBytes per (device, stream), allocated the first
// time a split launch is enqueued on that stream and kept until
// rxq4_release_workspace frees it or the process ends.  Hence:
//   * a HIP graph captured on a stream keeps a valid workspace pointer for
//     as long as the buffer is not released, whatever is launched later;
//   * split launches on different streams never share memory; launches on
//     one stream are ordered by the stream itself.  hipStreamPerThread is one
//     handle value for many streams (each thread's own default stream), so
//     its buffers are kept per (device, thread); the legacy null stream is
//     one stream for all threads and serialises them, so it has one buffer;
//   * no launch synchronises: the only runtime call is the one hipMalloc per
//     (device, stream), made with the calling thread's capture mode set to
//     relaxed so that it is also legal while the stream is being captured
//     (the allocation is not part of the graph).
// Every split launcher sizes its split count so that its partials fit.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdlib>
#include <map>
#include <mutex>
#include <thread>
#include <tuple>
#include <utility>

#include "launch.h"

namespace rxq4 {

namespace {
std::mutex g_mutex;
// (device, stream handle, thread id or 0) -> buffer
using WsKey = std::tuple<int, uintptr_t, size_t>;
std::map<WsKey, void *> *g_buffers = nullptr;  // never destroyed

hipError_t workspace_key(hipStream_t st, WsKey *key) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const size_t tid = st == hipStreamPerThread
                           ? std::hash<std::thread::id>()(std::this_thread::get_id()) | 1u
                           : 0u;
    *key = WsKey(dev, reinterpret_cast<uintptr_t>(st), tid);
    return hipSuccess;
}
}  // namespace

hipError_t stream_workspace(hipStream_t st, float **ws) {
    WsKey key;
    hipError_t e = workspace_key(st, &key);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_buffers) g_buffers = new std::map<WsKey, void *>();
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

hipError_t release_stream_workspace(hipStream_t st, int *released) {
    *released = 0;
    WsKey key;
    hipError_t e = workspace_key(st, &key);
    if (e != hipSuccess) return e;
    void *p = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        if (!g_buffers) return hipSuccess;
        auto it = g_buffers->find(key);
        if (it == g_buffers->end()) return hipSuccess;
        p = it->second;
        g_buffers->erase(it);
    }
    // the stream's queued work may still use the buffer
    if ((e = hipStreamSynchronize(st)) != hipSuccess) return e;
    if ((e = hipFree(p)) != hipSuccess) return e;
    *released = 1;
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
        r.gemm_nw = env_pos("RXQ4_GEMM_NW");
        r.gemv_stream = env_off("RXQ4_GEMV_STREAM") ? -1 : env_pos("RXQ4_GEMV_STREAM");
        return r;
    }();
    return t;
}

int workspace_count() {
    std::lock_guard<std::mutex> lock(g_mutex);
    return g_buffers ? static_cast<int>(g_buffers->size()) : 0;
}

}  // namespace rxq4
