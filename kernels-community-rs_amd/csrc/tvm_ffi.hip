// tvm-ffi packed-function exports: the symbols the reference's kernel-builder
// `_ops` module binds (`int32_t __tvm_ffi_<name>(void* handle, const TVMFFIAny*
// args, int32_t num_args, TVMFFIAny* result)`, flash-attn2-rs/src/host/forward/
// mod.rs:815-853, activation-rs/src/ops.rs:255-265, rmsnorm/src/ops.rs:442-444),
// as thin adapters over the C ABI of this library (include/kcr_hip.h).
//
// ABI followed: tvm-ffi 0.1.14 (the version the reference pins), whose public C
// header fixes
//   * TVMFFIAny: {int32 type_index; uint32 small_str_len / zero padding;
//     8-byte value union} (reference binding: flash-attn2-rs/src/host/mod.rs:59-66);
//   * the type indices used below (None 0, Int 1, Bool 2, Float 3, DLTensor
//     pointer 7, raw C string 8, byte-array pointer 9, small string 11, String
//     object 65, Tensor object 70);
//   * an object header of 24 bytes (ref count, type index, deleter) that a
//     Tensor object's DLTensor and a String object's byte array follow.
// DLTensor / DLDataType / DLDevice are DLPack's, restated here.
//
// The runtime side of tvm-ffi (the caller's current stream, the environment
// tensor allocator that the reference uses for the outputs it returns, error
// raising, and the `ffi.Array` constructor for multi-tensor results) lives in
// the tvm-ffi runtime library of the calling process. These adapters resolve
// those entry points from the process at call time (dlsym on RTLD_DEFAULT):
//   TVMFFIEnvGetStream, TVMFFIEnvTensorAlloc, TVMFFIErrorSetRaisedFromCStr,
//   TVMFFIFunctionGetGlobal, TVMFFIFunctionCall, TVMFFIObjectDecRef.
// Without a runtime, ops that only write caller-provided tensors run on the
// null stream; ops that must allocate their results fail with a RuntimeError.
// Errors always also leave the message in kcr_last_error().
#include "common.h"

#include <dlfcn.h>

#include <cstring>

namespace kcr {
namespace ffi {
namespace {

struct DLDataType {
    uint8_t code;
    uint8_t bits;
    uint16_t lanes;
};
struct DLDevice {
    int32_t device_type;
    int32_t device_id;
};
struct DLTensor {
    void* data;
    DLDevice device;
    int32_t ndim;
    DLDataType dtype;
    int64_t* shape;
    int64_t* strides;
    uint64_t byte_offset;
};
struct ObjectHeader {
    uint64_t combined_ref_count;
    int32_t type_index;
    uint32_t padding;
    void* deleter;
};
static_assert(sizeof(ObjectHeader) == 24, "tvm-ffi object header");
struct ByteArray {
    const char* data;
    size_t size;
};

}  // namespace
}  // namespace ffi
}  // namespace kcr

extern "C" {
typedef struct TVMFFIAny {
    int32_t type_index;
    uint32_t small_str_len;
    union {
        int64_t v_int64;
        double v_float64;
        void* v_ptr;
        const char* v_c_str;
        char v_bytes[8];
    };
} TVMFFIAny;
}
static_assert(sizeof(TVMFFIAny) == 16, "TVMFFIAny is 16 bytes");

namespace kcr {
namespace ffi {
namespace {

constexpr int32_t kNone = 0, kInt = 1, kBool = 2, kFloat = 3, kDLTensorPtr = 7, kRawStr = 8, kByteArrayPtr = 9,
                  kSmallStr = 11, kStr = 65, kFunction = 68, kShape = 69, kTensor = 70;
constexpr int32_t kDLCPU = 1, kDLCUDA = 2, kDLROCM = 10;

// Runtime entry points of the calling process's tvm-ffi runtime (or null),
// looked up on every call: a runtime loaded after the first call is found.
template <typename F>
F runtime_fn(const char* name) {
    return reinterpret_cast<F>(dlsym(RTLD_DEFAULT, name));
}
using GetStreamFn = void* (*)(int32_t, int32_t);
using TensorAllocFn = int (*)(DLTensor*, void**);
using SetRaisedFn = void (*)(const char*, const char*);
using GetGlobalFn = int (*)(const ByteArray*, void**);
using FunctionCallFn = int (*)(void*, TVMFFIAny*, int32_t, TVMFFIAny*);
using DecRefFn = int (*)(void*);

struct Args {
    const char* op;
    const TVMFFIAny* a;
    int32_t n;

    const TVMFFIAny& at(int i) const { return a[i]; }
    bool none(int i) const { return a[i].type_index == kNone; }

    [[noreturn]] void bad(int i, const char* want) const {
        throw type_error(std::string(op) + " argument #" + std::to_string(i) + ": expected " + want +
                         ", got type index " + std::to_string(a[i].type_index));
    }
    const DLTensor* dltensor(int i) const {
        const TVMFFIAny& x = a[i];
        if (x.type_index == kDLTensorPtr) return static_cast<const DLTensor*>(x.v_ptr);
        if (x.type_index == kTensor) {
            return reinterpret_cast<const DLTensor*>(static_cast<const char*>(x.v_ptr) + sizeof(ObjectHeader));
        }
        bad(i, "a Tensor");
    }
    const DLTensor* opt_dltensor(int i) const { return none(i) ? nullptr : dltensor(i); }
    double f64(int i) const {
        const TVMFFIAny& x = a[i];
        if (x.type_index == kFloat) return x.v_float64;
        if (x.type_index == kInt || x.type_index == kBool) return static_cast<double>(x.v_int64);
        bad(i, "a float");
    }
    int64_t i64(int i) const {
        const TVMFFIAny& x = a[i];
        if (x.type_index == kInt || x.type_index == kBool) return x.v_int64;
        bad(i, "an int");
    }
    bool boolean(int i) const {
        const TVMFFIAny& x = a[i];
        if (x.type_index == kBool || x.type_index == kInt) return x.v_int64 != 0;
        bad(i, "a bool");
    }
    std::string str(int i) const {
        const TVMFFIAny& x = a[i];
        switch (x.type_index) {
            case kRawStr: return std::string(x.v_c_str);
            case kSmallStr: return std::string(x.v_bytes, std::min<uint32_t>(x.small_str_len, 8));
            case kByteArrayPtr: {
                const auto* b = static_cast<const ByteArray*>(x.v_ptr);
                return std::string(b->data, b->size);
            }
            case kStr: {
                const auto* b = reinterpret_cast<const ByteArray*>(static_cast<const char*>(x.v_ptr) +
                                                                   sizeof(ObjectHeader));
                return std::string(b->data, b->size);
            }
            default: bad(i, "a string");
        }
    }
};

// DLPack (code, bits) -> kcr dtype.
int32_t dtype_of(const DLDataType& t) {
    if (t.lanes != 1) return KCR_DTYPE_OTHER;
    if (t.code == 2 && t.bits == 16) return KCR_FLOAT16;
    if (t.code == 2 && t.bits == 32) return KCR_FLOAT32;
    if (t.code == 2 && t.bits == 64) return KCR_FLOAT64;
    if (t.code == 4 && t.bits == 16) return KCR_BFLOAT16;
    if (t.code == 0 && t.bits == 32) return KCR_INT32;
    if (t.code == 0 && t.bits == 64) return KCR_INT64;
    return KCR_DTYPE_OTHER;
}

// A kcr_tensor view of a DLTensor (null strides mean compact row-major).
struct View {
    kcr_tensor t{};
    bool present = false;
    const kcr_tensor* ptr() const { return present ? &t : nullptr; }
};
View view_of(const DLTensor* d, const char* op) {
    View v;
    if (!d) return v;
    if (d->ndim < 0 || d->ndim > KCR_MAX_DIMS) {
        throw value_error(std::string(op) + ": tensors of rank " + std::to_string(d->ndim) +
                          " are not supported (at most 8)");
    }
    v.present = true;
    v.t.data = static_cast<char*>(d->data) + d->byte_offset;
    v.t.dtype = dtype_of(d->dtype);
    v.t.ndim = d->ndim;
    v.t.device = (d->device.device_type == kDLCUDA || d->device.device_type == kDLROCM) ? d->device.device_id : -1;
    int64_t stride = 1;
    for (int i = d->ndim - 1; i >= 0; --i) {
        v.t.shape[i] = d->shape[i];
        v.t.strides[i] = d->strides ? d->strides[i] : stride;
        stride *= d->shape[i];
    }
    return v;
}

// The caller's current stream on the tensor's device (TVMFFIEnvGetStream), or
// the null stream without a runtime.
void* stream_for(const DLTensor* d) {
    const GetStreamFn get = runtime_fn<GetStreamFn>("TVMFFIEnvGetStream");
    if (!get || !d) return nullptr;
    return get(d->device.device_type, d->device.device_id);
}

void check_status(int status) {
    if (status != KCR_OK) {
        const std::string m = kcr_last_error();
        switch (status) {
            case KCR_VALUE_ERROR: throw value_error(m);
            case KCR_TYPE_ERROR: throw type_error(m);
            default: throw runtime_error(m);
        }
    }
}

// An owned tensor result from the environment allocator (host/mod.rs:42-74).
struct Owned {
    void* handle = nullptr;
    DLTensor* dl = nullptr;
    Owned() = default;
    Owned(const Owned&) = delete;
    Owned& operator=(const Owned&) = delete;
    Owned(Owned&& o) noexcept : handle(o.handle), dl(o.dl) { o.handle = nullptr; }
    Owned& operator=(Owned&& o) noexcept {
        if (this != &o) {
            drop();
            handle = o.handle;
            dl = o.dl;
            o.handle = nullptr;
        }
        return *this;
    }
    ~Owned() { drop(); }
    void drop() {
        if (handle) {
            const DecRefFn dec = runtime_fn<DecRefFn>("TVMFFIObjectDecRef");
            if (dec) dec(handle);
            handle = nullptr;
        }
    }
    void* release() {
        void* h = handle;
        handle = nullptr;
        return h;
    }
};
Owned alloc(std::vector<int64_t> shape, DLDataType dtype, DLDevice device) {
    const TensorAllocFn fn = runtime_fn<TensorAllocFn>("TVMFFIEnvTensorAlloc");
    if (!fn) {
        throw runtime_error("this op returns tensors it allocates, which needs the tvm-ffi runtime "
                            "(TVMFFIEnvTensorAlloc) loaded in the process");
    }
    DLTensor proto{};
    proto.device = device;
    proto.ndim = static_cast<int32_t>(shape.size());
    proto.dtype = dtype;
    proto.shape = shape.data();
    Owned o;
    if (fn(&proto, &o.handle) != 0 || !o.handle) {
        o.handle = nullptr;
        throw runtime_error("environment tensor allocator failed");
    }
    o.dl = reinterpret_cast<DLTensor*>(static_cast<char*>(o.handle) + sizeof(ObjectHeader));
    return o;
}
constexpr DLDataType kF32{2, 32, 1};

void set_none(TVMFFIAny* r) {
    r->type_index = kNone;
    r->small_str_len = 0;
    r->v_int64 = 0;
}
void set_tensor(TVMFFIAny* r, Owned& t) {
    r->type_index = kTensor;
    r->small_str_len = 0;
    r->v_ptr = t.release();
}
// Array[Tensor] through the runtime's `ffi.Array` constructor.
void set_array(TVMFFIAny* r, std::vector<Owned>& items) {
    const GetGlobalFn get = runtime_fn<GetGlobalFn>("TVMFFIFunctionGetGlobal");
    const FunctionCallFn call = runtime_fn<FunctionCallFn>("TVMFFIFunctionCall");
    const DecRefFn dec = runtime_fn<DecRefFn>("TVMFFIObjectDecRef");
    if (!get || !call) throw runtime_error("returning an Array needs the tvm-ffi runtime (ffi.Array)");
    const ByteArray name{"ffi.Array", 9};
    void* fn = nullptr;
    if (get(&name, &fn) != 0 || !fn) throw runtime_error("the tvm-ffi runtime has no ffi.Array");
    std::vector<TVMFFIAny> args(items.size());
    for (size_t i = 0; i < items.size(); ++i) {
        args[i].type_index = kTensor;
        args[i].small_str_len = 0;
        args[i].v_ptr = items[i].handle;
    }
    TVMFFIAny out{};
    const int rc = call(fn, args.data(), static_cast<int32_t>(args.size()), &out);
    if (dec) dec(fn);
    if (rc != 0) throw runtime_error("ffi.Array failed");
    *r = out;  // the array holds its own references; `items` release theirs
}

// Runs `body`, mapping failures to -1 with the error raised in the runtime (as
// Error::set_raised does, host/forward/mod.rs:828-831) and kept locally.
template <typename F>
int32_t packed(const char* op, const TVMFFIAny* args, int32_t n, TVMFFIAny* result, F&& body) {
    Args a{op, args, n};
    const int status = guarded([&] { body(a, result); });
    if (status == KCR_OK) return 0;
    const SetRaisedFn raise = runtime_fn<SetRaisedFn>("TVMFFIErrorSetRaisedFromCStr");
    if (raise) {
        const char* kind = status == KCR_VALUE_ERROR ? "ValueError" : status == KCR_TYPE_ERROR ? "TypeError"
                                                                                              : "RuntimeError";
        raise(kind, kcr_last_error());
    }
    return -1;
}

void need(const Args& a, int count, const char* sig) {
    if (a.n != count) {
        throw value_error(std::string(a.op) + " expects " + std::to_string(count) + " arguments " + sig + ", got " +
                          std::to_string(a.n));
    }
}

// ---------------------------------------------------------------------------
// Activations (activation-rs/src/ops.rs:198-265): (out, input) -> None.
// ---------------------------------------------------------------------------
using ActFn = int (*)(const kcr_tensor*, const kcr_tensor*, void*);
int32_t activation(const char* op, ActFn fn, const TVMFFIAny* args, int32_t n, TVMFFIAny* r) {
    return packed(op, args, n, r, [&](const Args& a, TVMFFIAny* res) {
        need(a, 2, "(out, input)");
        const DLTensor* out = a.dltensor(0);
        const View vo = view_of(out, a.op), vi = view_of(a.dltensor(1), a.op);
        check_status(fn(vo.ptr(), vi.ptr(), stream_for(out)));
        set_none(res);
    });
}

// The dropout arguments of the forward: p, then seed (int) or a device RNG
// state tensor, then offset (host/forward/mod.rs:73-131).
struct Drop {
    kcr_dropout d{};
    View state;
    bool on = false;
    const kcr_dropout* ptr() const { return on ? &d : nullptr; }
};
Drop dropout_of(const Args& a, int ip, int iseed, int ioff, bool seed_is_state) {
    Drop r;
    const double p = a.f64(ip);
    if (!(p >= 0.0 && p < 1.0) || static_cast<float>(p) >= 1.0f) {
        throw value_error("p_dropout must be finite and in [0, 1) as float32");
    }
    if (!(static_cast<float>(p) > 0.0f)) return r;
    r.on = true;
    r.d.p = p;
    if (iseed >= 0) {
        const TVMFFIAny& s = a.at(iseed);
        if (seed_is_state || s.type_index == kDLTensorPtr || s.type_index == kTensor) {
            if (a.none(iseed)) throw value_error("dropout requires RNG state");
            r.state = view_of(a.dltensor(iseed), a.op);
            r.d.rng_state = r.state.ptr();
        } else {
            r.d.seed = static_cast<uint64_t>(a.i64(iseed));
        }
    }
    if (ioff >= 0) r.d.offset = static_cast<uint64_t>(a.i64(ioff));
    return r;
}

void scale_of(const Args& a, int i, int& has, double& v) {
    has = a.none(i) ? 0 : 1;
    v = has ? a.f64(i) : 0.0;
}

}  // namespace
}  // namespace ffi
}  // namespace kcr

using kcr::ffi::Args;
using kcr::ffi::Owned;
using kcr::ffi::View;

#define KCR_ACT_EXPORT(name)                                                                          \
    extern "C" int32_t __tvm_ffi_##name(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) { \
        return kcr::ffi::activation(#name, kcr_##name, args, n, result);                               \
    }
KCR_ACT_EXPORT(silu_and_mul)
KCR_ACT_EXPORT(mul_and_silu)
KCR_ACT_EXPORT(gelu_and_mul)
KCR_ACT_EXPORT(gelu_tanh_and_mul)
KCR_ACT_EXPORT(gelu)
KCR_ACT_EXPORT(gelu_tanh)
KCR_ACT_EXPORT(gelu_new)
KCR_ACT_EXPORT(gelu_fast)
KCR_ACT_EXPORT(gelu_quick)
KCR_ACT_EXPORT(silu)
#undef KCR_ACT_EXPORT

extern "C" int32_t __tvm_ffi_fatrelu_and_mul(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("fatrelu_and_mul", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        kcr::ffi::need(a, 3, "(out, input, threshold)");
        const auto* out = a.dltensor(0);
        const View vo = kcr::ffi::view_of(out, a.op), vi = kcr::ffi::view_of(a.dltensor(1), a.op);
        kcr::ffi::check_status(kcr_fatrelu_and_mul(vo.ptr(), vi.ptr(), a.f64(2), kcr::ffi::stream_for(out)));
        kcr::ffi::set_none(r);
    });
}

// RMSNorm (rmsnorm/src/ops.rs:237-440).
extern "C" int32_t __tvm_ffi_rms_norm_forward(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("rms_norm_forward", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        kcr::ffi::need(a, 7, "(y, rstd, x, weight, eps, offset, casting_mode)");
        const auto* x = a.dltensor(2);
        const View y = kcr::ffi::view_of(a.dltensor(0), a.op), rs = kcr::ffi::view_of(a.dltensor(1), a.op),
                   vx = kcr::ffi::view_of(x, a.op), w = kcr::ffi::view_of(a.opt_dltensor(3), a.op);
        const std::string mode = a.str(6);
        kcr::ffi::check_status(kcr_rms_norm_forward(y.ptr(), rs.ptr(), vx.ptr(), w.ptr(), a.f64(4), a.f64(5),
                                                    mode.c_str(), kcr::ffi::stream_for(x)));
        kcr::ffi::set_none(r);
    });
}

extern "C" int32_t __tvm_ffi_rms_norm_backward(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("rms_norm_backward", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        kcr::ffi::need(a, 8, "(dx, dw_partial, dy, x, weight, rstd, offset, casting_mode)");
        const auto* x = a.dltensor(3);
        const View dx = kcr::ffi::view_of(a.dltensor(0), a.op), dwp = kcr::ffi::view_of(a.opt_dltensor(1), a.op),
                   dy = kcr::ffi::view_of(a.opt_dltensor(2), a.op), vx = kcr::ffi::view_of(x, a.op),
                   w = kcr::ffi::view_of(a.opt_dltensor(4), a.op), rs = kcr::ffi::view_of(a.dltensor(5), a.op);
        const std::string mode = a.str(7);
        kcr::ffi::check_status(kcr_rms_norm_backward(dx.ptr(), dwp.ptr(), dy.ptr(), vx.ptr(), w.ptr(), rs.ptr(),
                                                     a.f64(6), mode.c_str(), kcr::ffi::stream_for(x)));
        kcr::ffi::set_none(r);
    });
}

extern "C" int32_t __tvm_ffi_rms_norm_reduce_weight_grad(void*, const TVMFFIAny* args, int32_t n,
                                                         TVMFFIAny* result) {
    return kcr::ffi::packed("rms_norm_reduce_weight_grad", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        kcr::ffi::need(a, 2, "(dw, dw_partial)");
        const auto* dw = a.dltensor(0);
        const View vdw = kcr::ffi::view_of(dw, a.op), vp = kcr::ffi::view_of(a.dltensor(1), a.op);
        kcr::ffi::check_status(kcr_rms_norm_reduce_weight_grad(vdw.ptr(), vp.ptr(), kcr::ffi::stream_for(dw)));
        kcr::ffi::set_none(r);
    });
}

// ---------------------------------------------------------------------------
// FlashAttention-2 (flash-attn2-rs/src/host).
// ---------------------------------------------------------------------------
namespace kcr {
namespace ffi {
namespace {

// The generator descriptor of fwd at arity 16 (reserve(generator, device,
// B * H * 32) returning a 4-element Shape) or 18 (four arguments), resolved
// into the state tensor on the call's stream (host/forward/mod.rs:132-178,
// 492-523).
void resolve_descriptor(const Args& a, const DLTensor* q, const DLTensor* k, const Drop& drop,
                        bool return_softmax) {
    const bool native = a.n == 16;
    if (native) {
        if (!drop.on || !drop.d.rng_state) throw value_error("native reservation requires dropout and a state tensor");
    } else {
        if (!drop.on || q->ndim != 4 || k->ndim != 4 || !drop.d.rng_state || q->shape[3] != 64 || q->shape[1] == 0 ||
            k->shape[1] == 0) {
            throw value_error("RNG descriptor requires nonempty D64 dropout");
        }
        if (return_softmax) throw value_error("RNG descriptor does not support diagnostic probabilities");
    }
    uint64_t desc[3];
    int captured;
    if (native) {
        if (a.at(14).type_index != kFunction) a.bad(14, "a Function (reserve)");
        const FunctionCallFn call = runtime_fn<FunctionCallFn>("TVMFFIFunctionCall");
        const DecRefFn dec = runtime_fn<DecRefFn>("TVMFFIObjectDecRef");
        if (!call) throw runtime_error("native reservation needs the tvm-ffi runtime (TVMFFIFunctionCall)");
        TVMFFIAny args[3]{};
        args[0].type_index = kInt;
        args[0].v_int64 = a.i64(15);
        args[1].type_index = kInt;
        args[1].v_int64 = q->device.device_id;
        args[2].type_index = kInt;
        args[2].v_int64 = q->shape[0] * q->shape[2] * 32;
        TVMFFIAny out{};
        if (call(a.at(14).v_ptr, args, 3, &out) != 0) throw runtime_error("reserve failed");
        if (out.type_index != kShape) {
            if (out.type_index >= kStr && dec) dec(out.v_ptr);
            throw type_error("reserve must return a Shape descriptor");
        }
        // ShapeObj: the object header, then {const int64_t* data; int64_t size}.
        const char* body = static_cast<const char*>(out.v_ptr) + sizeof(ObjectHeader);
        const int64_t* values = *reinterpret_cast<const int64_t* const*>(body);
        const int64_t size = *reinterpret_cast<const int64_t*>(body + sizeof(void*));
        const bool ok = size == 4 && (values[3] == 0 || values[3] == 1);
        if (ok) {
            for (int i = 0; i < 3; ++i) desc[i] = static_cast<uint64_t>(values[i]);
            captured = static_cast<int>(values[3]);
        }
        if (dec) dec(out.v_ptr);
        if (!ok) throw value_error("invalid reserved RNG descriptor");
    } else {
        for (int i = 0; i < 3; ++i) desc[i] = static_cast<uint64_t>(a.i64(14 + i));
        captured = a.boolean(17) ? 1 : 0;
    }
    if (captured && (desc[0] == 0 || desc[1] == 0 || desc[0] % 8 != 0 || desc[1] % 8 != 0)) {
        throw value_error(native ? "invalid reserved capture pointers" : "invalid capture descriptor pointers");
    }
    check_status(kcr_flash_rng_state(drop.d.rng_state, desc[0], desc[1], desc[2], captured, stream_for(q)));
}

// fwd / fwd_lse (host/forward/mod.rs:52-61, 815-853): 9 base arguments, then
// optionally (p, seed | state, offset) and/or the output tensor; arity 14 is
// (..., p, state, offset, out | None, return_softmax) and returns
// [out, lse, probabilities] (mod.rs:133-199, 382-398); arities 16 and 18 add a
// generator descriptor.
void fwd_impl(const Args& a, TVMFFIAny* r, bool lse_only) {
    const int n = a.n;
    if (n != 9 && n != 10 && n != 12 && n != 13 && n != 14 && n != 16 && n != 18) {
        throw value_error("fwd expects 9 positional arguments (q, k, v, alibi_slopes, softmax_scale, is_causal, "
                          "window_size_left, window_size_right, softcap), optionally followed by p_dropout, "
                          "seed, offset, and/or an output tensor; got " +
                          std::to_string(n));
    }
    const DLTensor* q = a.dltensor(0);
    if (q->ndim != 4) throw value_error("q must have 4 dimensions [B, S, H, D]");
    const bool wide = n == 14 || n == 16 || n == 18;
    const int out_idx = wide ? 12 : n - 1;
    const bool supplied = n == 10 || n == 13 || (wide && !a.none(12));
    const bool return_softmax = wide && a.boolean(13);
    if (lse_only && !supplied) throw value_error("LSE-only forward requires a supplied output");
    if (lse_only && return_softmax) throw value_error("LSE-only forward cannot return diagnostic probabilities");
    const Drop drop = n >= 12 ? dropout_of(a, 9, 10, 11, false) : Drop{};
    if (drop.d.rng_state && drop.d.offset != 0) {
        throw value_error("offset must be zero when seed is an RNG-state tensor");
    }
    if (n == 16 || n == 18) resolve_descriptor(a, q, a.dltensor(1), drop, return_softmax);
    if (return_softmax && (!drop.on || !drop.d.rng_state)) {
        throw value_error("return_softmax requires nonzero dropout and a CUDA RNG-state tensor");
    }
    int has_scale;
    double scale;
    scale_of(a, 4, has_scale, scale);
    const View vq = view_of(q, a.op), vk = view_of(a.dltensor(1), a.op), vv = view_of(a.dltensor(2), a.op),
               al = view_of(a.opt_dltensor(3), a.op);
    Owned out_o;
    const DLTensor* out = supplied ? a.dltensor(out_idx) : nullptr;
    if (!supplied) {
        out_o = alloc({q->shape[0], q->shape[1], q->shape[2], q->shape[3]}, q->dtype, q->device);
        out = out_o.dl;
    }
    Owned lse = alloc({q->shape[0], q->shape[2], q->shape[1]}, kF32, q->device);
    const View vo = view_of(out, a.op), vl = view_of(lse.dl, a.op);
    Owned probs;
    if (return_softmax) {
        const auto round128 = [](int64_t x) { return (x + 127) / 128 * 128; };
        probs = alloc({q->shape[0], q->shape[2], round128(q->shape[1]), round128(a.dltensor(1)->shape[1])},
                      q->dtype, q->device);
        const View vp = view_of(probs.dl, a.op);
        check_status(kcr_flash_fwd_softmax(vq.ptr(), vk.ptr(), vv.ptr(), al.ptr(), has_scale, scale,
                                           a.boolean(5) ? 1 : 0, a.i64(6), a.i64(7), a.f64(8), drop.ptr(),
                                           vo.ptr(), vl.ptr(), vp.ptr(), stream_for(q)));
    } else {
        check_status(kcr_flash_fwd(vq.ptr(), vk.ptr(), vv.ptr(), al.ptr(), has_scale, scale,
                                   a.boolean(5) ? 1 : 0, a.i64(6), a.i64(7), a.f64(8), drop.ptr(), vo.ptr(),
                                   vl.ptr(), stream_for(q)));
        if (wide) probs = alloc({0}, q->dtype, q->device);
    }
    if (lse_only) {
        set_tensor(r, lse);
        return;
    }
    std::vector<Owned> items;
    if (supplied) {
        // The supplied output is the caller's tensor: the array needs it as an
        // owned object only when it was passed as one.
        if (a.at(out_idx).type_index != kTensor) {
            throw runtime_error("fwd with a supplied output returns [out, lse] and needs `out` as a Tensor object");
        }
        const auto inc = runtime_fn<int (*)(void*)>("TVMFFIObjectIncRef");
        if (!inc) throw runtime_error("returning an Array needs the tvm-ffi runtime (TVMFFIObjectIncRef)");
        Owned o;
        o.handle = a.at(out_idx).v_ptr;
        inc(o.handle);
        items.push_back(std::move(o));
    } else {
        items.push_back(std::move(out_o));
    }
    items.push_back(std::move(lse));
    if (wide) items.push_back(std::move(probs));
    set_array(r, items);
}

void check_p(double p, double softcap) {
    if (!(p >= 0.0 && p < 1.0) || static_cast<float>(p) >= 1.0f ||
        (static_cast<float>(p) > 0.0f && softcap > 0.0)) {
        throw value_error("invalid dropout or dropout combined with softcap");
    }
}

// bwd_dq / bwd_dkv / bwd_all (host/backward.rs:14-626): 14 arguments.
void bwd_impl(const Args& a, TVMFFIAny* r, bool want_q, bool want_kv) {
    if (a.n != 14) {
        throw value_error("backward component expects q, k, v, dout, lse, delta, alibi, scale, causal, left, "
                          "right, softcap, dropout, rng_state");
    }
    const DLTensor* q = a.dltensor(0);
    const DLTensor* k = a.dltensor(1);
    const DLTensor* v = a.dltensor(2);
    if (q->ndim != 4 || k->ndim != 4 || v->ndim != 4) throw value_error("q, k and v must be [B, S, H, D]");
    const double p = a.f64(12);
    check_p(p, a.f64(11));
    Drop drop;
    if (static_cast<float>(p) > 0.0f) {
        if (a.none(13)) throw value_error("dropout backward requires saved RNG state");
        drop = dropout_of(a, 12, 13, -1, true);
    }
    int has_scale;
    double scale;
    scale_of(a, 7, has_scale, scale);
    Owned dq, dk, dv;
    if (want_q) dq = alloc({q->shape[0], q->shape[1], q->shape[2], q->shape[3]}, q->dtype, q->device);
    if (want_kv) {
        dk = alloc({k->shape[0], k->shape[1], k->shape[2], k->shape[3]}, k->dtype, k->device);
        dv = alloc({v->shape[0], v->shape[1], v->shape[2], v->shape[3]}, v->dtype, v->device);
    }
    const View vq = view_of(q, a.op), vk = view_of(k, a.op), vv = view_of(v, a.op),
               vdo = view_of(a.dltensor(3), a.op), vl = view_of(a.dltensor(4), a.op),
               vd = view_of(a.dltensor(5), a.op), al = view_of(a.opt_dltensor(6), a.op), vdq = view_of(dq.dl, a.op),
               vdk = view_of(dk.dl, a.op), vdv = view_of(dv.dl, a.op);
    check_status(kcr_flash_bwd(vq.ptr(), vk.ptr(), vv.ptr(), vdo.ptr(), vl.ptr(), vd.ptr(), al.ptr(), has_scale,
                               scale, a.boolean(8) ? 1 : 0, a.i64(9), a.i64(10), a.f64(11), drop.ptr(), vdq.ptr(),
                               vdk.ptr(), vdv.ptr(), nullptr, 0, stream_for(q)));
    if (want_q && !want_kv) {
        set_tensor(r, dq);
        return;
    }
    std::vector<Owned> items;
    if (want_q) items.push_back(std::move(dq));
    items.push_back(std::move(dk));
    items.push_back(std::move(dv));
    set_array(r, items);
}

}  // namespace
}  // namespace ffi
}  // namespace kcr

extern "C" int32_t __tvm_ffi_fwd(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("fwd", args, n, result,
                            [&](const Args& a, TVMFFIAny* r) { kcr::ffi::fwd_impl(a, r, false); });
}

extern "C" int32_t __tvm_ffi_rng_state(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("rng_state", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        if (a.n != 5) throw kcr::value_error("rng_state expects reference, seed, offset, intragraph, captured");
        const auto* ref = a.dltensor(0);
        if (ref->device.device_type != kcr::ffi::kDLCUDA && ref->device.device_type != kcr::ffi::kDLROCM) {
            throw kcr::value_error("RNG state requires a CUDA reference tensor");
        }
        const uint64_t seed = static_cast<uint64_t>(a.i64(1)), offset = static_cast<uint64_t>(a.i64(2));
        const uint64_t intragraph = static_cast<uint64_t>(a.i64(3));
        const int captured = a.boolean(4) ? 1 : 0;
        if (captured && (seed == 0 || offset == 0 || seed % 8 != 0 || offset % 8 != 0)) {
            throw kcr::value_error("captured RNG descriptor requires aligned non-null CUDA pointers");
        }
        Owned state = kcr::ffi::alloc({2}, kcr::ffi::DLDataType{0, 64, 1}, ref->device);
        const View vs = kcr::ffi::view_of(state.dl, a.op);
        kcr::ffi::check_status(kcr_flash_rng_state(vs.ptr(), seed, offset, intragraph, captured,
                                                   kcr::ffi::stream_for(ref)));
        kcr::ffi::set_tensor(r, state);
    });
}

extern "C" int32_t __tvm_ffi_fwd_lse(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("fwd_lse", args, n, result,
                            [&](const Args& a, TVMFFIAny* r) { kcr::ffi::fwd_impl(a, r, true); });
}

extern "C" int32_t __tvm_ffi_bwd_preprocess(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("bwd_preprocess", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        kcr::ffi::need(a, 3, "(dout, out, p_dropout)");
        const auto* out = a.dltensor(1);
        if (out->ndim != 4) throw kcr::value_error("dout and out must share shape, dtype and device");
        const double p = a.f64(2);
        if (!(p >= 0.0 && p < 1.0) || static_cast<float>(p) >= 1.0f) {
            throw kcr::value_error("p_dropout must be in [0, 1) as float32");
        }
        const int64_t rounded = (out->shape[1] + 127) / 128 * 128;
        Owned delta = kcr::ffi::alloc({out->shape[0], out->shape[2], rounded}, kcr::ffi::kF32, out->device);
        const View vdo = kcr::ffi::view_of(a.dltensor(0), a.op), vo = kcr::ffi::view_of(out, a.op),
                   vd = kcr::ffi::view_of(delta.dl, a.op);
        kcr::ffi::check_status(kcr_flash_bwd_preprocess(vdo.ptr(), vo.ptr(), p, vd.ptr(), kcr::ffi::stream_for(out)));
        kcr::ffi::set_tensor(r, delta);
    });
}

extern "C" int32_t __tvm_ffi_bwd_dq(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("bwd_dq", args, n, result,
                            [&](const Args& a, TVMFFIAny* r) { kcr::ffi::bwd_impl(a, r, true, false); });
}

extern "C" int32_t __tvm_ffi_bwd_dkv(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("bwd_dkv", args, n, result,
                            [&](const Args& a, TVMFFIAny* r) { kcr::ffi::bwd_impl(a, r, false, true); });
}

extern "C" int32_t __tvm_ffi_bwd_all(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("bwd_all", args, n, result,
                            [&](const Args& a, TVMFFIAny* r) { kcr::ffi::bwd_impl(a, r, true, true); });
}

// varlen_fwd_explicit (host/varlen/mod.rs:21-670): 19 arguments (20 with a
// block table, which this adapter does not take) -> [out, lse, probabilities].
extern "C" int32_t __tvm_ffi_varlen_fwd_explicit(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("varlen_fwd_explicit", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        if (a.n == 20 && !a.none(19)) {
            throw kcr::value_error("varlen_fwd_explicit with a block table is served by the Python ops module");
        }
        if (a.n != 19 && a.n != 20) kcr::ffi::need(a, 19, "(q, k, v, cu_seqlens_q, cu_seqlens_k, ...)");
        const auto* q = a.dltensor(0);
        if (q->ndim != 3) throw kcr::value_error("q must be [total_q, H, D]");
        const double p = a.f64(13);
        if (!(p >= 0.0 && p < 1.0) || static_cast<float>(p) >= 1.0f ||
            (static_cast<float>(p) > 0.0f && a.f64(12) > 0.0) ||
            (a.boolean(17) && !(static_cast<float>(p) > 0.0f))) {
            throw kcr::value_error("invalid dropout, softcap, or probability request");
        }
        kcr::ffi::Drop drop;
        if (static_cast<float>(p) > 0.0f) {
            if (a.none(14)) throw kcr::value_error("dropout requires RNG state");
            drop = kcr::ffi::dropout_of(a, 13, 14, -1, true);
        }
        int has_scale;
        double scale;
        kcr::ffi::scale_of(a, 8, has_scale, scale);
        Owned out = kcr::ffi::alloc({q->shape[0], q->shape[1], q->shape[2]}, q->dtype, q->device);
        Owned lse = kcr::ffi::alloc({q->shape[1], q->shape[0]}, kcr::ffi::kF32, q->device);
        const bool return_softmax = a.boolean(17);
        if (return_softmax && (a.dltensor(3)->ndim != 1 || a.dltensor(3)->shape[0] < 2 || a.i64(15) < 0 ||
                               a.i64(16) < 0 || a.i64(15) > INT32_MAX - 256 || a.i64(16) > INT32_MAX - 256)) {
            throw kcr::value_error("unsupported packed attention dimensions");
        }
        const auto round128 = [](int64_t x) { return (x + 127) / 128 * 128; };
        Owned probs = return_softmax
                          ? kcr::ffi::alloc({a.dltensor(3)->shape[0] - 1, q->shape[1], round128(a.i64(15)),
                                             round128(a.i64(16))},
                                            q->dtype, q->device)
                          : kcr::ffi::alloc({0}, q->dtype, q->device);
        const View vq = kcr::ffi::view_of(q, a.op), vk = kcr::ffi::view_of(a.dltensor(1), a.op),
                   vv = kcr::ffi::view_of(a.dltensor(2), a.op), cq = kcr::ffi::view_of(a.dltensor(3), a.op),
                   ck = kcr::ffi::view_of(a.dltensor(4), a.op), su = kcr::ffi::view_of(a.opt_dltensor(5), a.op),
                   lp = kcr::ffi::view_of(a.opt_dltensor(6), a.op), al = kcr::ffi::view_of(a.opt_dltensor(7), a.op),
                   vo = kcr::ffi::view_of(out.dl, a.op), vl = kcr::ffi::view_of(lse.dl, a.op);
        if (return_softmax) {
            const View vp = kcr::ffi::view_of(probs.dl, a.op);
            kcr::ffi::check_status(kcr_flash_varlen_fwd_softmax(
                vq.ptr(), vk.ptr(), vv.ptr(), cq.ptr(), ck.ptr(), su.ptr(), lp.ptr(), al.ptr(), has_scale, scale,
                a.boolean(9) ? 1 : 0, a.i64(10), a.i64(11), a.f64(12), drop.ptr(), a.i64(15), a.i64(16),
                a.boolean(18) ? 1 : 0, vo.ptr(), vl.ptr(), vp.ptr(), kcr::ffi::stream_for(q)));
        } else {
            kcr::ffi::check_status(kcr_flash_varlen_fwd(
                vq.ptr(), vk.ptr(), vv.ptr(), cq.ptr(), ck.ptr(), su.ptr(), lp.ptr(), al.ptr(), has_scale, scale,
                a.boolean(9) ? 1 : 0, a.i64(10), a.i64(11), a.f64(12), drop.ptr(), a.i64(15), a.i64(16),
                a.boolean(18) ? 1 : 0, vo.ptr(), vl.ptr(), kcr::ffi::stream_for(q)));
        }
        std::vector<Owned> items;
        items.push_back(std::move(out));
        items.push_back(std::move(lse));
        items.push_back(std::move(probs));
        kcr::ffi::set_array(r, items);
    });
}

// varlen_bwd_explicit (host/varlen/backward.rs:15-546): 19 arguments ->
// [dq, dk, dv, delta] with delta [H, total_q + 128 * batch].
extern "C" int32_t __tvm_ffi_varlen_bwd_explicit(void*, const TVMFFIAny* args, int32_t n, TVMFFIAny* result) {
    return kcr::ffi::packed("varlen_bwd_explicit", args, n, result, [&](const Args& a, TVMFFIAny* r) {
        kcr::ffi::need(a, 19, "(q, k, v, dout, out, lse, cu_seqlens_q, cu_seqlens_k, alibi, scale, causal, "
                              "left, right, softcap, p, state, max_q, max_k, zero_tensors)");
        const auto* q = a.dltensor(0);
        const auto* k = a.dltensor(1);
        const auto* v = a.dltensor(2);
        const auto* cu = a.dltensor(6);
        if (q->ndim != 3 || k->ndim != 3 || v->ndim != 3 || cu->ndim != 1) {
            throw kcr::value_error("q, k, v must be [total, H, D] and cu_seqlens one-dimensional");
        }
        const double p = a.f64(14);
        kcr::ffi::check_p(p, a.f64(13));
        kcr::ffi::Drop drop;
        if (static_cast<float>(p) > 0.0f) {
            if (a.none(15)) throw kcr::value_error("dropout backward requires saved RNG state");
            drop = kcr::ffi::dropout_of(a, 14, 15, -1, true);
        }
        int has_scale;
        double scale;
        kcr::ffi::scale_of(a, 9, has_scale, scale);
        const int64_t batch = cu->shape[0] - 1;
        Owned dq = kcr::ffi::alloc({q->shape[0], q->shape[1], q->shape[2]}, q->dtype, q->device);
        Owned dk = kcr::ffi::alloc({k->shape[0], k->shape[1], k->shape[2]}, k->dtype, k->device);
        Owned dv = kcr::ffi::alloc({v->shape[0], v->shape[1], v->shape[2]}, v->dtype, v->device);
        Owned delta = kcr::ffi::alloc({q->shape[1], q->shape[0] + 128 * batch}, kcr::ffi::kF32, q->device);
        const View vq = kcr::ffi::view_of(q, a.op), vk = kcr::ffi::view_of(k, a.op), vv = kcr::ffi::view_of(v, a.op),
                   vdo = kcr::ffi::view_of(a.dltensor(3), a.op), vo = kcr::ffi::view_of(a.dltensor(4), a.op),
                   vl = kcr::ffi::view_of(a.dltensor(5), a.op), cq = kcr::ffi::view_of(cu, a.op),
                   ck = kcr::ffi::view_of(a.dltensor(7), a.op), al = kcr::ffi::view_of(a.opt_dltensor(8), a.op),
                   vdq = kcr::ffi::view_of(dq.dl, a.op), vdk = kcr::ffi::view_of(dk.dl, a.op),
                   vdv = kcr::ffi::view_of(dv.dl, a.op), vd = kcr::ffi::view_of(delta.dl, a.op);
        kcr::ffi::check_status(kcr_flash_varlen_bwd(
            vq.ptr(), vk.ptr(), vv.ptr(), vdo.ptr(), vo.ptr(), vl.ptr(), cq.ptr(), ck.ptr(), al.ptr(), has_scale,
            scale, a.boolean(10) ? 1 : 0, a.i64(11), a.i64(12), a.f64(13), drop.ptr(), a.i64(16), a.i64(17),
            a.boolean(18) ? 1 : 0, vdq.ptr(), vdk.ptr(), vdv.ptr(), vd.ptr(), nullptr, 0, kcr::ffi::stream_for(q)));
        std::vector<Owned> items;
        items.push_back(std::move(dq));
        items.push_back(std::move(dk));
        items.push_back(std::move(dv));
        items.push_back(std::move(delta));
        kcr::ffi::set_array(r, items);
    });
}
