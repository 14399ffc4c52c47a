// floors.hip -- measurement kernels for bench.py (not part of the drop-in
// library): what a launch, a sustained read and a sustained write cost on
// the box, the floors against which the GEMV and gather kernels are judged.
//   rxq4_floor_empty(stream)                       an empty kernel (one wave)
//   rxq4_floor_stream(src, bytes, sink, blocks, unroll, nt, stream)    a
//       persistent grid-stride read: `blocks` workgroups of 256 threads
//       loop over the buffer, each lane keeping two batches of `unroll`
//       (4, 8 or 16) 16-byte loads in flight (load j of a batch at
//       i + j * threads, coalesced across the grid); nt = 1 marks the loads
//       nontemporal.  The read ceiling the GEMVs are compared with.
//   rxq4_floor_write(dst, bytes, blocks, nt, stream)    a grid-stride
//       16-byte store of zeros over `bytes` (nt = 1: nontemporal stores),
//       the write rate the embedding gathers are compared with.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ void floor_empty_kernel() {}

// Persistent grid-stride read, two batches of U 16-byte loads in flight per
// lane.  Loads are unconditional (indices past the end clamp to the last
// element, an L2 hit), only their use is predicated.
template <int U, bool NT>
__global__ __launch_bounds__(256) void floor_stream_kernel(const u32x4 *__restrict__ src,
                                                           int64_t n16, uint32_t *sink) {
    const int64_t threads = (int64_t)gridDim.x * 256;
    const int64_t step = threads * U;
    const int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    auto load = [&](u32x4 *v, int64_t base) {
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const u32x4 *p = src + min(base + j * threads, n16 - 1);
            v[j] = NT ? __builtin_nontemporal_load(p) : *p;
        }
    };
    uint32_t acc = 0;
    auto use = [&](const u32x4 *v, int64_t base) {
#pragma unroll
        for (int j = 0; j < U; ++j)
            acc ^= (base + j * threads < n16) ? (v[j].x ^ v[j].y ^ v[j].z ^ v[j].w) : 0u;
    };
    u32x4 a[U], b[U];
    load(a, i0);
    load(b, i0 + step);
    for (int64_t base = i0; base < n16; base += 2 * step) {
        use(a, base);
        load(a, base + 2 * step);
        use(b, base + step);
        load(b, base + 3 * step);
    }
    __shared__ uint32_t red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (int i = 0; i < 256; ++i) s ^= red[i];
        sink[blockIdx.x] = s;
    }
}

template <bool NT>
__global__ __launch_bounds__(256) void floor_write_kernel(u32x4 *__restrict__ dst, int64_t n16) {
    const int64_t threads = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += threads) {
        if (NT)
            __builtin_nontemporal_store(u32x4{0, 0, 0, 0}, dst + i);
        else
            dst[i] = u32x4{0, 0, 0, 0};
    }
}

extern "C" {

int rxq4_floor_empty(void *stream) {
    floor_empty_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>();
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

// sink: at least `blocks` dwords
int rxq4_floor_stream(const void *src, int64_t bytes, uint32_t *sink, int blocks, int unroll,
                      int nt, void *stream) {
    if (bytes <= 0 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(src) & 15) != 0) return 4;
    if (blocks <= 0 || blocks > 65536) return 4;
    const int64_t n16 = bytes / 16;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const u32x4 *s = static_cast<const u32x4 *>(src);
#define RXQ4_STREAM(U)                                                                  \
    (nt ? (floor_stream_kernel<U, true><<<blocks, 256, 0, st>>>(s, n16, sink), 0)       \
        : (floor_stream_kernel<U, false><<<blocks, 256, 0, st>>>(s, n16, sink), 0))
    switch (unroll) {
    case 4: RXQ4_STREAM(4); break;
    case 8: RXQ4_STREAM(8); break;
    case 16: RXQ4_STREAM(16); break;
    default: return 4;
    }
#undef RXQ4_STREAM
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

int rxq4_floor_write(void *dst, int64_t bytes, int blocks, int nt, void *stream) {
    if (bytes <= 0 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(dst) & 15) != 0) return 4;
    if (blocks <= 0 || blocks > 65536) return 4;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    u32x4 *d = static_cast<u32x4 *>(dst);
    if (nt)
        floor_write_kernel<true><<<blocks, 256, 0, st>>>(d, bytes / 16);
    else
        floor_write_kernel<false><<<blocks, 256, 0, st>>>(d, bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // extern "C"
