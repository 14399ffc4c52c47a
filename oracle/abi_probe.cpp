// abi_probe.cpp -- prints the binary layout of the reflex::infer public API as
// JSON.  TEST INFRASTRUCTURE: the same source is compiled once against the
// reference checkout's include/reflex/infer.h and once against this
// repository's, and tests/test_abi.py requires the two outputs to be equal.
#include <cstddef>
#include <cstdio>
#include <type_traits>

#include "reflex/infer.h"

using namespace reflex::infer;

static bool first = true;

static void field(const char* type, const char* name, size_t off) {
    std::printf("%s\"%s.%s\": %zu", first ? "" : ",\n", type, name, off);
    first = false;
}

template <typename T>
static void shape(const char* type) {
    std::printf("%s\"%s.sizeof\": %zu,\n\"%s.alignof\": %zu", first ? "" : ",\n", type,
                sizeof(T), type, alignof(T));
    first = false;
}

#define F(T, m) field(#T, #m, offsetof(T, m))

int main() {
    std::printf("{\n");
    shape<Status>("Status");
    shape<QuantFormat>("QuantFormat");
    shape<DeviceClass>("DeviceClass");
    shape<ModelFamily>("ModelFamily");
    field("Status", "NotImplemented", (size_t)Status::NotImplemented);
    field("Status", "InvalidArgument", (size_t)Status::InvalidArgument);
    field("Status", "UnsupportedQuantFormat", (size_t)Status::UnsupportedQuantFormat);
    field("QuantFormat", "Unknown", (size_t)QuantFormat::Unknown);
    field("DeviceClass", "Unknown", (size_t)DeviceClass::Unknown);
    field("ModelFamily", "Unknown", (size_t)ModelFamily::Unknown);

    shape<HardwareProfile>("HardwareProfile");
    F(HardwareProfile, sm_count); F(HardwareProfile, total_memory_bytes);
    F(HardwareProfile, nominal_dram_gbps);
    shape<ModelShape>("ModelShape");
    F(ModelShape, vocab_size); F(ModelShape, max_context);
    shape<QuantDescriptor>("QuantDescriptor");
    F(QuantDescriptor, group_size); F(QuantDescriptor, kv_cache_int8);
    shape<KernelSupport>("KernelSupport");
    F(KernelSupport, kv_convert);

    shape<GemvQuantArgs>("GemvQuantArgs");
    F(GemvQuantArgs, y); F(GemvQuantArgs, weights); F(GemvQuantArgs, weights_device);
    F(GemvQuantArgs, ggml_type); F(GemvQuantArgs, x); F(GemvQuantArgs, M);
    F(GemvQuantArgs, K); F(GemvQuantArgs, stream);

    shape<GemvQuantAddArgs>("GemvQuantAddArgs");
    F(GemvQuantAddArgs, y); F(GemvQuantAddArgs, weights); F(GemvQuantAddArgs, weights_device);
    F(GemvQuantAddArgs, ggml_type); F(GemvQuantAddArgs, x); F(GemvQuantAddArgs, residual);
    F(GemvQuantAddArgs, M); F(GemvQuantAddArgs, K); F(GemvQuantAddArgs, stream);

    shape<GemvQuantPairArgs>("GemvQuantPairArgs");
    F(GemvQuantPairArgs, y0); F(GemvQuantPairArgs, weights0);
    F(GemvQuantPairArgs, weights0_device); F(GemvQuantPairArgs, ggml_type0);
    F(GemvQuantPairArgs, M0); F(GemvQuantPairArgs, y1); F(GemvQuantPairArgs, weights1);
    F(GemvQuantPairArgs, weights1_device); F(GemvQuantPairArgs, ggml_type1);
    F(GemvQuantPairArgs, M1); F(GemvQuantPairArgs, x); F(GemvQuantPairArgs, K);
    F(GemvQuantPairArgs, stream);

    shape<GemvQuantTripleArgs>("GemvQuantTripleArgs");
    F(GemvQuantTripleArgs, y0); F(GemvQuantTripleArgs, weights0);
    F(GemvQuantTripleArgs, weights0_device); F(GemvQuantTripleArgs, ggml_type0);
    F(GemvQuantTripleArgs, M0); F(GemvQuantTripleArgs, y1); F(GemvQuantTripleArgs, weights1);
    F(GemvQuantTripleArgs, weights1_device); F(GemvQuantTripleArgs, ggml_type1);
    F(GemvQuantTripleArgs, M1); F(GemvQuantTripleArgs, y2); F(GemvQuantTripleArgs, weights2);
    F(GemvQuantTripleArgs, weights2_device); F(GemvQuantTripleArgs, ggml_type2);
    F(GemvQuantTripleArgs, M2); F(GemvQuantTripleArgs, x); F(GemvQuantTripleArgs, K);
    F(GemvQuantTripleArgs, stream);

    shape<GemmQuantBatchedArgs>("GemmQuantBatchedArgs");
    F(GemmQuantBatchedArgs, y); F(GemmQuantBatchedArgs, weights);
    F(GemmQuantBatchedArgs, weights_device); F(GemmQuantBatchedArgs, ggml_type);
    F(GemmQuantBatchedArgs, x); F(GemmQuantBatchedArgs, M); F(GemmQuantBatchedArgs, N);
    F(GemmQuantBatchedArgs, K); F(GemmQuantBatchedArgs, stream);

    shape<GemvQuantF32Args>("GemvQuantF32Args");
    F(GemvQuantF32Args, y); F(GemvQuantF32Args, weights); F(GemvQuantF32Args, weights_device);
    F(GemvQuantF32Args, ggml_type); F(GemvQuantF32Args, x); F(GemvQuantF32Args, M);
    F(GemvQuantF32Args, K); F(GemvQuantF32Args, stream);

    shape<DequantEmbeddingRowArgs>("DequantEmbeddingRowArgs");
    F(DequantEmbeddingRowArgs, dst); F(DequantEmbeddingRowArgs, weights);
    F(DequantEmbeddingRowArgs, weights_device); F(DequantEmbeddingRowArgs, ggml_type);
    F(DequantEmbeddingRowArgs, token_id); F(DequantEmbeddingRowArgs, hidden_dim);
    F(DequantEmbeddingRowArgs, stream);

    shape<AttentionDecodeArgs>("AttentionDecodeArgs");
    F(AttentionDecodeArgs, scale); F(AttentionDecodeArgs, kv_int8);
    F(AttentionDecodeArgs, k_scales); F(AttentionDecodeArgs, stream);
    shape<AttentionPrefillBatchedArgs>("AttentionPrefillBatchedArgs");
    F(AttentionPrefillBatchedArgs, start_pos); F(AttentionPrefillBatchedArgs, kv_int8);
    F(AttentionPrefillBatchedArgs, v_scales); F(AttentionPrefillBatchedArgs, stream);

    shape<Q4Kernels>("Q4Kernels");
    F(Q4Kernels, gemv_quant); F(Q4Kernels, gemv_quant_add); F(Q4Kernels, gemv_quant_pair);
    F(Q4Kernels, gemv_quant_triple); F(Q4Kernels, gemm_quant_batched);
    F(Q4Kernels, gemv_quant_f32); F(Q4Kernels, dequant_embedding_row);

    constexpr HardwareProfile hp = orin_nano_8gb_sm87();
    field("orin_nano_8gb_sm87", "sm", (size_t)hp.sm);
    field("orin_nano_8gb_sm87", "shared_mem_per_block", hp.shared_mem_per_block);
    field("orin_nano_8gb_sm87", "dram_gbps_x10", (size_t)(hp.nominal_dram_gbps * 10.0f));
    std::printf(",\n\"version_string\": \"%s\"", version_string());
    std::printf("\n}\n");
    return 0;
}
