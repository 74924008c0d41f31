// Dropout RNG state from a generator descriptor: what flash-attn2-rs's
// `rng_state` export and the descriptor arities of `fwd` do
// (src/host/rng.rs:13-78, kernel src/device/rng.rs:1-26). The descriptor
// (seed, offset, intragraph, captured) is the Philox reservation of a CUDA
// generator: with captured = 0, seed and offset are the values; with
// captured = 1 (a reservation made under graph capture) they are device
// addresses of the seed and of the base offset, and the offset is the value
// read plus intragraph. A one-lane kernel on the call's stream writes
// [seed, offset] into the int64 [2] state tensor, so a captured graph resolves
// the values live at each replay.

#include "attention.h"

namespace kcr {
namespace attn {
namespace {

__global__ __launch_bounds__(64) void resolve_rng_state_kernel(int64_t* state, uint64_t seed, uint64_t offset,
                                                               uint64_t intragraph, int32_t captured) {
    if (threadIdx.x != 0) return;
    uint64_t s = seed, o = offset;
    if (captured) {
        s = *reinterpret_cast<const uint64_t*>(seed);
        o = *reinterpret_cast<const uint64_t*>(offset) + intragraph;
    }
    state[0] = static_cast<int64_t>(s);
    state[1] = static_cast<int64_t>(o);
}

}  // namespace

void resolve_rng_state(const kcr_tensor* state, uint64_t seed, uint64_t offset, uint64_t intragraph, int captured,
                       hipStream_t s) {
    if (!state || state->dtype != KCR_INT64 || state->ndim != 1 || state->shape[0] != 2 ||
        state->strides[0] != 1 || reinterpret_cast<uintptr_t>(state->data) % 8 != 0) {
        throw value_error("rng_state must be a contiguous CUDA int64 tensor of shape [2]");
    }
    require_device(state, "rng_state");
    if (captured && (seed == 0 || offset == 0 || seed % 8 != 0 || offset % 8 != 0)) {
        throw value_error("captured RNG descriptor requires aligned non-null CUDA pointers");
    }
    resolve_rng_state_kernel<<<1, 64, 0, s>>>(static_cast<int64_t*>(state->data), seed, offset, intragraph,
                                              captured ? 1 : 0);
    check_launch("launch resolve_rng_state");
}

}  // namespace attn
}  // namespace kcr

extern "C" int kcr_flash_rng_state(const kcr_tensor* state, uint64_t seed, uint64_t offset, uint64_t intragraph,
                                   int captured, void* stream) {
    return kcr::guarded([&] {
        kcr::attn::resolve_rng_state(state, seed, offset, intragraph, captured, static_cast<hipStream_t>(stream));
    });
}
