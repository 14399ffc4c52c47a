// dispatch_link_probe.cpp -- links the reference's own dispatcher
// (src/dispatch.cpp of FastCrest/reflex-infer, compiled from its sources into
// _ref/dispatch.o) against the MI355X kernel layer
// (reflex-infer_amd/lib/libreflex_infer_hip_kernels.so) and calls through it.
// Test infrastructure: it shows that the reference dispatcher binds to this
// build's reflex::infer::kernels::* seam without changes.  Only calls that the
// seam answers before touching a GPU are made, so it runs without one.
#include <cstdio>

#include "reflex/infer.h"

using namespace reflex::infer;

int main() {
    int fake_weights[4] = {0, 0, 0, 0};
    GemvQuantArgs g{};
    g.weights = fake_weights;
    g.weights_device = fake_weights;
    g.ggml_type = 15;  // Q8_K: not served (Q4_K, Q5_K and Q6_K are)
    g.M = 16;
    g.K = 256;
    const Status q8 = gemv_quant(g);
    g.ggml_type = 13;  // Q5_K passes the type check and fails the shape check
    g.K = 100;
    const Status q5 = gemv_quant(g);

    AttentionDecodeArgs a{};
    const Status attn = flash_attention_decode(a);

    const Q4Kernels reg = registered_q4_backend();
    const bool all_null = !reg.gemv_quant && !reg.gemv_quant_add && !reg.gemv_quant_pair &&
                          !reg.gemv_quant_triple && !reg.gemm_quant_batched &&
                          !reg.gemv_quant_f32 && !reg.dequant_embedding_row;
    std::printf("{\"gemv_quant_q8k\": %d, \"gemv_quant_q5k_bad_k\": %d, "
                "\"flash_attention_decode\": %d, \"registry_empty\": %d}\n",
                static_cast<int>(q8), static_cast<int>(q5), static_cast<int>(attn),
                all_null ? 1 : 0);
    return 0;
}
