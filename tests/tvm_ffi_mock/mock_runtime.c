/* A stand-in for the few tvm-ffi runtime entry points that libkcr_hip.so's
 * __tvm_ffi_* adapters call, for tests only: the process has no tvm-ffi
 * runtime. Device memory comes from a callback the test installs (torch's
 * allocator); objects are reference counted like tvm-ffi's (a 24-byte header,
 * a Tensor's DLTensor right after it). */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct { uint8_t code, bits; uint16_t lanes; } DLDataType;
typedef struct { int32_t device_type, device_id; } DLDevice;
typedef struct {
    void* data; DLDevice device; int32_t ndim; DLDataType dtype;
    int64_t* shape; int64_t* strides; uint64_t byte_offset;
} DLTensor;
typedef struct { uint64_t refs; int32_t type_index; uint32_t pad; void (*deleter)(void*, int); } Header;
typedef struct { const char* data; size_t size; } ByteArray;
typedef struct { int32_t type_index; uint32_t small; union { int64_t i; double f; void* p; }; } Any;

typedef struct { Header h; DLTensor dl; int64_t shape[8]; } Tensor;
typedef struct { Header h; int64_t size; void* items[16]; } Array;
typedef struct { Header h; } Function;
typedef struct { Header h; const int64_t* data; int64_t size; int64_t values[8]; } Shape;
/* A reserve function: returns a Shape of its stored values, records its call. */
typedef struct { Header h; int64_t size; int64_t values[8]; int64_t last_args[3]; int64_t calls; } Reserve;

static void* (*g_alloc)(int64_t bytes, int32_t device_id);
static void* g_stream;
static char g_kind[64], g_msg[4096];
static int64_t g_live;
static Function g_array_fn = {{1u << 30, 68, 0, 0}};

void mock_set_alloc(void* (*fn)(int64_t, int32_t)) { g_alloc = fn; }
void mock_set_stream(void* s) { g_stream = s; }
const char* mock_error_kind(void) { return g_kind; }
const char* mock_error_message(void) { return g_msg; }
int64_t mock_live_objects(void) { return g_live; }
int64_t mock_array_size(void* a) { return ((Array*)a)->size; }
void* mock_array_item(void* a, int64_t i) { return ((Array*)a)->items[i]; }
DLTensor* mock_tensor(void* t) { return &((Tensor*)t)->dl; }
uint64_t mock_refs(void* o) { return ((Header*)o)->refs; }

void* mock_make_reserve(const int64_t* values, int64_t size) {
    Reserve* r = (Reserve*)calloc(1, sizeof(Reserve));
    r->h.refs = 1;
    r->h.type_index = 68;
    r->size = size > 8 ? 8 : size;
    memcpy(r->values, values, sizeof(int64_t) * r->size);
    return r;
}
int64_t mock_reserve_calls(void* r) { return ((Reserve*)r)->calls; }
int64_t mock_reserve_arg(void* r, int i) { return ((Reserve*)r)->last_args[i]; }

void* TVMFFIEnvGetStream(int32_t device_type, int32_t device_id) {
    (void)device_type; (void)device_id;
    return g_stream;
}

void TVMFFIErrorSetRaisedFromCStr(const char* kind, const char* message) {
    strncpy(g_kind, kind, sizeof g_kind - 1);
    strncpy(g_msg, message, sizeof g_msg - 1);
}

int TVMFFIObjectIncRef(void* obj) {
    ((Header*)obj)->refs++;
    return 0;
}

int TVMFFIObjectDecRef(void* obj) {
    Header* h = (Header*)obj;
    if (--h->refs == 0) {
        if (h->type_index == 71) {
            Array* a = (Array*)obj;
            for (int64_t i = 0; i < a->size; ++i) TVMFFIObjectDecRef(a->items[i]);
        }
        if (h->type_index == 70 || h->type_index == 71 || h->type_index == 69) {
            g_live--;
            free(obj);  /* device memory stays with the test's allocator */
        }
    }
    return 0;
}

int TVMFFIEnvTensorAlloc(DLTensor* proto, void** out) {
    if (!g_alloc || proto->ndim > 8) return -1;
    int64_t n = 1;
    for (int i = 0; i < proto->ndim; ++i) n *= proto->shape[i];
    Tensor* t = (Tensor*)calloc(1, sizeof(Tensor));
    t->h.refs = 1;
    t->h.type_index = 70;
    t->dl = *proto;
    memcpy(t->shape, proto->shape, sizeof(int64_t) * proto->ndim);
    t->dl.shape = t->shape;
    t->dl.strides = NULL;
    t->dl.byte_offset = 0;
    t->dl.data = g_alloc(n * proto->dtype.bits / 8, proto->device.device_id);
    if (!t->dl.data && n > 0) {
        free(t);
        return -1;
    }
    g_live++;
    *out = t;
    return 0;
}

int TVMFFIFunctionGetGlobal(const ByteArray* name, void** out) {
    if (name->size == 9 && memcmp(name->data, "ffi.Array", 9) == 0) {
        *out = &g_array_fn;
        return 0;
    }
    *out = NULL;
    return -1;
}

int TVMFFIFunctionCall(void* fn, Any* args, int32_t n, Any* result) {
    if (fn != &g_array_fn) {
        Reserve* r = (Reserve*)fn;
        if (n != 3) return -1;
        for (int i = 0; i < 3; ++i) r->last_args[i] = args[i].i;
        r->calls++;
        Shape* sh = (Shape*)calloc(1, sizeof(Shape));
        sh->h.refs = 1;
        sh->h.type_index = 69;
        memcpy(sh->values, r->values, sizeof(int64_t) * r->size);
        sh->data = sh->values;
        sh->size = r->size;
        g_live++;
        result->type_index = 69;
        result->small = 0;
        result->p = sh;
        return 0;
    }
    if (n > 16) return -1;
    Array* a = (Array*)calloc(1, sizeof(Array));
    a->h.refs = 1;
    a->h.type_index = 71;
    a->size = n;
    for (int32_t i = 0; i < n; ++i) {
        a->items[i] = args[i].p;
        TVMFFIObjectIncRef(args[i].p);
    }
    g_live++;
    result->type_index = 71;
    result->small = 0;
    result->p = a;
    return 0;
}
