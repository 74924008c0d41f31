// Layout staging of attention tensors: the packed copies the kernels need for
// rows they cannot read as 16-byte vectors (flash-attn2-rs/src/host/layout.rs:
// 46-125, device/layout.rs:1-35), and the copy of an output written through a
// packed buffer (host/forward/mod.rs:349-376).
//
// Design: rows of (batch, sequence, head) copied with their own strides on
// both sides. When both sides' bases, strides and widths are whole 16-byte
// chunks (the zero-padded head-size copies, and staging of aligned layouts)
// each lane moves 16-byte chunks, LPR lanes per row and 64 / LPR rows per
// wave; otherwise one wave per row moves 2-byte elements, so any layout works
// (the staged side is always packed and aligned).
#include "attention.h"

#include <algorithm>
#include <utility>

namespace kcr {
namespace attn {

namespace {

constexpr int kCopyWaves = 4;

// rows = B * S * H rows: D elements copied, then the destination row zeroed
// up to DZ elements (DZ > D for a zero-padded copy). Row r = ((b * S) + s) * H + h.
__global__ void __launch_bounds__(64 * kCopyWaves) copy_rows_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, int64_t rows, int64_t S, int64_t H,
    int64_t D, int64_t DZ, int64_t sb, int64_t ss, int64_t sh, int64_t db, int64_t ds, int64_t dh) {
    const int lane = threadIdx.x & 63;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * kCopyWaves + (threadIdx.x >> 6); r < rows;
         r += static_cast<int64_t>(gridDim.x) * kCopyWaves) {
        const int64_t h = r % H;
        const int64_t bs = r / H;
        const int64_t s = bs % S;
        const int64_t b = bs / S;
        const uint16_t* from = src + b * sb + s * ss + h * sh;
        uint16_t* to = dst + b * db + s * ds + h * dh;
        for (int64_t c = lane; c < D; c += 64) to[c] = from[c];
        for (int64_t c = D + lane; c < DZ; c += 64) to[c] = 0;
    }
}

// The 16-byte chunk form: CD chunks copied, then zero chunks up to CZ. Row r
// of rows < 2^31 is ((b * S) + s) * H + h.
template <int LPR>
__global__ void __launch_bounds__(64 * kCopyWaves) copy_rows_vec_kernel(
    uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, uint32_t rows, uint32_t S, uint32_t H,
    int CD, int CZ, int64_t sb, int64_t ss, int64_t sh, int64_t db, int64_t ds, int64_t dh) {
    constexpr int RPW = 64 / LPR;  // rows per wave
    const int lane = threadIdx.x & 63;
    const int c0 = lane % LPR;
    const uint32_t step = gridDim.x * kCopyWaves * RPW;
    for (uint32_t r = (blockIdx.x * kCopyWaves + (threadIdx.x >> 6)) * RPW + lane / LPR; r < rows; r += step) {
        const uint32_t h = r % H;
        const uint32_t bs = r / H;
        const uint32_t sq = bs % S;
        const uint32_t b = bs / S;
        const uint16_t* from = src + b * sb + sq * ss + h * sh;
        uint16_t* to = dst + b * db + sq * ds + h * dh;
        for (int c = c0; c < CZ; c += LPR) {
            const u32x4 v = c < CD ? *reinterpret_cast<const u32x4*>(from + 8 * c) : u32x4{0, 0, 0, 0};
            *reinterpret_cast<u32x4*>(to + 8 * c) = v;
        }
    }
}

// The tensor as [B, S, H, D] (packed 3-D tensors are [1, T, H, D]).
struct Dims4 {
    int64_t shape[4];
    int64_t stride[4];
};

Dims4 dims4(const kcr_tensor& t) {
    Dims4 d{};
    const int off = 4 - t.ndim;
    for (int i = 0; i < 4; ++i) {
        d.shape[i] = i < off ? 1 : t.shape[i - off];
        d.stride[i] = i < off ? 0 : t.strides[i - off];
    }
    return d;
}

// Copies the rows of `src` into `dst` (same outer shape): the first
// min(widths) elements of each row, the rest of a wider destination row zeroed.
void copy_rows(const kcr_tensor& dst, const kcr_tensor& src, hipStream_t s) {
    const Dims4 a = dims4(dst), b = dims4(src);
    const int64_t rows = a.shape[0] * a.shape[1] * a.shape[2];
    if (rows == 0 || a.shape[3] == 0) return;
    const int64_t width = std::min(a.shape[3], b.shape[3]);
    bool vec = width % 8 == 0 && a.shape[3] % 8 == 0 && rows < (int64_t{1} << 31) &&
               reinterpret_cast<uintptr_t>(dst.data) % 16 == 0 && reinterpret_cast<uintptr_t>(src.data) % 16 == 0 &&
               a.stride[3] == 1 && b.stride[3] == 1;
    for (int i = 0; i < 3; ++i) {
        vec = vec && (a.shape[i] == 1 || (a.stride[i] % 8 == 0 && b.stride[i] % 8 == 0));
    }
    if (vec) {
        const int CZ = static_cast<int>(a.shape[3] / 8), CD = static_cast<int>(width / 8);
        auto go = [&](auto lpr) {
            constexpr int LPR = decltype(lpr)::value;
            constexpr int RPB = kCopyWaves * (64 / LPR);  // rows per block
            const int64_t blocks = std::min<int64_t>((rows + RPB - 1) / RPB, 65536);
            copy_rows_vec_kernel<LPR><<<static_cast<unsigned>(blocks), 64 * kCopyWaves, 0, s>>>(
                static_cast<uint16_t*>(dst.data), static_cast<const uint16_t*>(src.data),
                static_cast<uint32_t>(rows), static_cast<uint32_t>(a.shape[1]), static_cast<uint32_t>(a.shape[2]),
                CD, CZ, b.stride[0], b.stride[1], b.stride[2], a.stride[0], a.stride[1], a.stride[2]);
        };
        if (CZ <= 4) {
            go(std::integral_constant<int, 4>{});
        } else if (CZ <= 8) {
            go(std::integral_constant<int, 8>{});
        } else if (CZ <= 16) {
            go(std::integral_constant<int, 16>{});
        } else if (CZ <= 32) {
            go(std::integral_constant<int, 32>{});
        } else {
            go(std::integral_constant<int, 64>{});
        }
        check_launch("launch copy_rows");
        return;
    }
    const int64_t blocks = std::min<int64_t>((rows + kCopyWaves - 1) / kCopyWaves, 65536);
    copy_rows_kernel<<<static_cast<unsigned>(blocks), 64 * kCopyWaves, 0, s>>>(
        static_cast<uint16_t*>(dst.data), static_cast<const uint16_t*>(src.data), rows, a.shape[1],
        a.shape[2], std::min(a.shape[3], b.shape[3]), a.shape[3], b.stride[0], b.stride[1], b.stride[2],
        a.stride[0], a.stride[1], a.stride[2]);
    check_launch("launch copy_rows");
}

int64_t span_elems(const kcr_tensor& t) {
    int64_t span = 1;
    for (int i = 0; i < t.ndim; ++i) {
        if (t.shape[i] == 0) return 0;
        span += (t.shape[i] - 1) * t.strides[i];
    }
    return span;
}

}  // namespace

bool spans_overlap(const kcr_tensor* a, const kcr_tensor* b) {
    if (!a || !b) return false;
    const int64_t na = span_elems(*a), nb = span_elems(*b);
    if (na == 0 || nb == 0) return false;
    const auto pa = reinterpret_cast<uintptr_t>(a->data), pb = reinterpret_cast<uintptr_t>(b->data);
    const uintptr_t ea = pa + static_cast<uintptr_t>(na) * element_size(a->dtype);
    const uintptr_t eb = pb + static_cast<uintptr_t>(nb) * element_size(b->dtype);
    return pa < eb && pb < ea;
}

bool nonoverlapping_layout(const kcr_tensor* t) {
    std::pair<int64_t, int64_t> dims[KCR_MAX_DIMS];  // (stride, size) of each dimension of size > 1
    int n = 0;
    for (int i = 0; i < t->ndim; ++i) {
        if (t->shape[i] == 0) return true;
        if (t->shape[i] == 1) continue;
        if (t->strides[i] < 0) return false;
        dims[n++] = {t->strides[i], t->shape[i]};
    }
    std::sort(dims, dims + n);
    int64_t reach = 0;  // largest offset reachable with the dimensions so far
    for (int i = 0; i < n; ++i) {
        if (dims[i].first <= reach) return false;
        reach += dims[i].first * (dims[i].second - 1);
    }
    return true;
}

Staged::Staged(const kcr_tensor* t, hipStream_t s, bool copy_in, int seq_dim, int64_t d,
               std::initializer_list<const kcr_tensor*> must_not_overlap)
    : src_(t), stream_(s) {
    if (!t) return;
    int64_t count = 1;
    for (int i = 0; i < t->ndim; ++i) count *= t->shape[i];
    if (count == 0) return;
    for (int i = 0; i < t->ndim; ++i) {
        if (t->shape[i] > 1 && t->strides[i] < 0) {
            throw value_error("attention tensors must have non-negative strides");
        }
    }
    bool pack = !rows_aligned16(t);
    if (seq_dim >= 0 && t->shape[seq_dim] > 1) {
        const int64_t st = t->strides[seq_dim];
        pack |= st < d || st > (int64_t{1} << 23);
    }
    for (const kcr_tensor* other : must_not_overlap) pack |= spans_overlap(t, other);
    if (!pack) return;
    packed_ = *t;
    int64_t stride = 1;
    for (int i = t->ndim - 1; i >= 0; --i) {
        packed_.strides[i] = stride;
        stride *= t->shape[i];
    }
    const size_t bytes = static_cast<size_t>(count) * element_size(t->dtype);
    check_hip(hipMallocAsync(&buffer_, bytes, s), "hipMallocAsync (packed attention tensor)");
    packed_.data = buffer_;
    if (copy_in) copy_rows(packed_, *t, s);
}

void Staged::copy_out() {
    if (buffer_) copy_rows(*src_, packed_, stream_);
}

Staged::~Staged() {
    if (buffer_) (void)hipFreeAsync(buffer_, stream_);
}

Padded::Padded(const kcr_tensor* t, int64_t width, hipStream_t s, bool copy_in) : src_(t), stream_(s) {
    if (!t) return;
    if (t->ndim < 1 || t->ndim > 4 || width < t->shape[t->ndim - 1]) {
        throw value_error("padded attention tensors are 1-4 dimensional and only widen the last dimension");
    }
    padded_ = *t;
    padded_.shape[t->ndim - 1] = width;
    int64_t count = 1;
    for (int i = t->ndim - 1; i >= 0; --i) {
        padded_.strides[i] = count;
        count *= padded_.shape[i];
    }
    if (count > 0) {
        const size_t bytes = static_cast<size_t>(count) * element_size(t->dtype);
        check_hip(hipMallocAsync(&buffer_, bytes, s), "hipMallocAsync (padded attention tensor)");
    }
    padded_.data = buffer_;
    if (copy_in && buffer_) copy_rows(padded_, *t, s);
}

void Padded::copy_out() {
    if (buffer_) copy_rows(*src_, padded_, stream_);
}

Padded::~Padded() {
    if (buffer_) (void)hipFreeAsync(buffer_, stream_);
}

}  // namespace attn
}  // namespace kcr
