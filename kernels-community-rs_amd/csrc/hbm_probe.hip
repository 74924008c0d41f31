// Streaming probe: the HBM ceiling for the bandwidth-bound kernels. It uses the
// memory shape of the gated-activation kernel (16-byte non-temporal loads and
// stores, four block-contiguous vectors in flight per lane, a capped grid that
// strides over the rest) with no arithmetic, so its rate is what those kernels
// could reach if their arithmetic were free.
#include "common.h"
#include "../../include/kcr_probe.h"

namespace kcr {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;
constexpr uint64_t kProbeBlocks = 32768;

template <int READS>
__global__ void __launch_bounds__(kProbeThreads) hbm_stream_kernel(u32x4_t* __restrict__ dst,
                                                                   const u32x4_t* __restrict__ src,
                                                                   uint64_t words) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kProbeThreads * kProbeUnroll;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kProbeThreads * kProbeUnroll + threadIdx.x; i < words;
         i += stride) {
        u32x4_t a[kProbeUnroll], b[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kProbeThreads;
            if (j < words) {
                a[u] = __builtin_nontemporal_load(src + j);
                if constexpr (READS == 2) b[u] = __builtin_nontemporal_load(src + words + j);
            }
        }
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * kProbeThreads;
            if (j < words) {
                u32x4_t r = a[u];
                if constexpr (READS == 2) r ^= b[u];
                __builtin_nontemporal_store(r, dst + j);
            }
        }
    }
}

}  // namespace
}  // namespace kcr

extern "C" int32_t kcr_hbm_stream_probe(void* dst, const void* src, int64_t words, int32_t reads, void* stream) {
    using namespace kcr;
    return guarded([&] {
        if (words < 0) throw value_error("words must be non-negative");
        if (reads != 1 && reads != 2) throw value_error("reads must be 1 or 2");
        if ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15)
            throw value_error("src and dst must be 16-byte aligned");
        if (words == 0) return;
        if (!dst || !src) throw value_error("src and dst are required");
        const uint64_t per_block = static_cast<uint64_t>(kProbeThreads) * kProbeUnroll;
        const uint64_t need = (static_cast<uint64_t>(words) + per_block - 1) / per_block;
        const unsigned grid = static_cast<unsigned>(std::min<uint64_t>(need, kProbeBlocks));
        auto s = static_cast<hipStream_t>(stream);
        auto d = static_cast<u32x4_t*>(dst);
        auto x = static_cast<const u32x4_t*>(src);
        if (reads == 1)
            hbm_stream_kernel<1><<<grid, kProbeThreads, 0, s>>>(d, x, static_cast<uint64_t>(words));
        else
            hbm_stream_kernel<2><<<grid, kProbeThreads, 0, s>>>(d, x, static_cast<uint64_t>(words));
        check_launch("launch hbm_stream_kernel");
    });
}
