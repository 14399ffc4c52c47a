// dispatch.cpp -- the public reflex::infer entry points and the Q4 backend
// plug-in registry.
//
// Behaviour of the reference dispatcher (src/dispatch.cpp:6-108): one
// lock-free slot per Q4 operation; register_q4_backend() overwrites all seven
// slots (release stores; a null member restores the built-in path for that
// operation), every call loads its slot (acquire) and forwards to the
// registered function if set, else to reflex::infer::kernels::*.  Attention is
// not pluggable.  Implemented here as one array of atomic slots indexed by
// operation.
#include <atomic>

#include "reflex/infer.h"
#include "seam.h"

namespace reflex::infer {
namespace {

enum Op : int {
    kGemv, kGemvAdd, kGemvPair, kGemvTriple, kGemmBatched, kGemvF32, kEmbedRow, kOpCount
};

std::atomic<void (*)()> g_slots[kOpCount];

template <typename Fn>
void put(Op op, Fn fn) noexcept {
    g_slots[op].store(reinterpret_cast<void (*)()>(fn), std::memory_order_release);
}

template <typename Fn>
Fn get(Op op) noexcept {
    return reinterpret_cast<Fn>(g_slots[op].load(std::memory_order_acquire));
}

template <typename Fn, typename Args>
Status route(Op op, Status (*builtin)(const Args &), const Args &args) {
    if (Fn fn = get<Fn>(op)) return fn(args);
    return builtin(args);
}

}  // namespace

void register_q4_backend(const Q4Kernels &k) noexcept {
    put(kGemv, k.gemv_quant);
    put(kGemvAdd, k.gemv_quant_add);
    put(kGemvPair, k.gemv_quant_pair);
    put(kGemvTriple, k.gemv_quant_triple);
    put(kGemmBatched, k.gemm_quant_batched);
    put(kGemvF32, k.gemv_quant_f32);
    put(kEmbedRow, k.dequant_embedding_row);
}

Q4Kernels registered_q4_backend() noexcept {
    Q4Kernels k{};
    k.gemv_quant = get<GemvQuantFn>(kGemv);
    k.gemv_quant_add = get<GemvQuantAddFn>(kGemvAdd);
    k.gemv_quant_pair = get<GemvQuantPairFn>(kGemvPair);
    k.gemv_quant_triple = get<GemvQuantTripleFn>(kGemvTriple);
    k.gemm_quant_batched = get<GemmQuantBatchedFn>(kGemmBatched);
    k.gemv_quant_f32 = get<GemvQuantF32Fn>(kGemvF32);
    k.dequant_embedding_row = get<DequantEmbeddingRowFn>(kEmbedRow);
    return k;
}

Status gemv_quant(const GemvQuantArgs &a) {
    return route<GemvQuantFn>(kGemv, kernels::gemv_quant, a);
}
Status gemv_quant_add(const GemvQuantAddArgs &a) {
    return route<GemvQuantAddFn>(kGemvAdd, kernels::gemv_quant_add, a);
}
Status gemv_quant_pair(const GemvQuantPairArgs &a) {
    return route<GemvQuantPairFn>(kGemvPair, kernels::gemv_quant_pair, a);
}
Status gemv_quant_triple(const GemvQuantTripleArgs &a) {
    return route<GemvQuantTripleFn>(kGemvTriple, kernels::gemv_quant_triple, a);
}
Status gemm_quant_batched(const GemmQuantBatchedArgs &a) {
    return route<GemmQuantBatchedFn>(kGemmBatched, kernels::gemm_quant_batched, a);
}
Status gemv_quant_f32(const GemvQuantF32Args &a) {
    return route<GemvQuantF32Fn>(kGemvF32, kernels::gemv_quant_f32, a);
}
Status dequant_embedding_row(const DequantEmbeddingRowArgs &a) {
    return route<DequantEmbeddingRowFn>(kEmbedRow, kernels::dequant_embedding_row, a);
}

Status flash_attention_decode(const AttentionDecodeArgs &a) {
    return kernels::flash_attention_decode(a);
}
Status flash_attention_prefill_batched(const AttentionPrefillBatchedArgs &a) {
    return kernels::flash_attention_prefill_batched(a);
}

}  // namespace reflex::infer
