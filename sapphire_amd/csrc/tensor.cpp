// tensor.cpp - tensor_t of include/tensor.h, with a device-resident weight copy.
//
// Host-side semantics follow the reference src/tensor/tensor.c (create, view, clone,
// refcount, accessors, the Q4_0 numel/2 allocation, view nbytes = numel * elem size).
// The private struct adds the device copy used by the GEMV entry points: quantized
// weights are uploaded once and repacked into the PACKED (or, for the LM head, TILED)
// layout, F32/BF16 uploaded as is; batched calls add a TILED copy. The copies are freed
// with the tensor.
#include <atomic>
#include <cstdlib>
#include <cstring>

#include "../../include/tensor.h"
#include "internal.h"
#include "tensor_impl.h"

using namespace sapphire;

static size_t shape_product(int ndim, const int *shape) {
    size_t p = 1;
    for (int i = 0; i < ndim; ++i) p *= (size_t)shape[i];
    return p;
}

static uint64_t next_serial() {
    static std::atomic<uint64_t> counter{0};
    return ++counter;
}

extern "C" {

size_t dtype_element_size(tensor_dtype_t dtype) {
    switch (dtype) {
        case DTYPE_F32: return 4;
        case DTYPE_BF16: return 2;
        case DTYPE_F16: return 2;
        case DTYPE_Q4_0: return 1;
        case DTYPE_Q8_0: return 1;
        default: return 0;
    }
}

const char *dtype_name(tensor_dtype_t dtype) {
    switch (dtype) {
        case DTYPE_F32: return "F32";
        case DTYPE_BF16: return "BF16";
        case DTYPE_F16: return "F16";
        case DTYPE_Q4_0: return "Q4_0";
        case DTYPE_Q8_0: return "Q8_0";
        default: return "UNKNOWN";
    }
}

tensor_t *tensor_create(int ndim, const int *shape, tensor_dtype_t dtype) {
    if (ndim < 1 || ndim > 8 || !shape) {
        set_error("tensor_create invalid ndim=%d or null shape", ndim);
        return nullptr;
    }
    tensor_t *t = new (std::nothrow) tensor_t();
    if (!t) return nullptr;
    t->ndim = ndim;
    t->dtype = dtype;
    t->layout = LAYOUT_ROW_MAJOR;
    memcpy(t->shape, shape, sizeof(int) * (size_t)ndim);
    const size_t numel = shape_product(ndim, shape);
    t->nbytes = dtype == DTYPE_Q4_0 ? (numel + 1) / 2 : numel * dtype_element_size(dtype);
    t->data = calloc(t->nbytes ? t->nbytes : 1, 1);
    if (!t->data) {
        delete t;
        return nullptr;
    }
    t->ref_count = 1;
    t->is_external = 0;
    t->serial = next_serial();
    return t;
}

tensor_t *tensor_create_view(tensor_dtype_t dtype, int ndim, const int *shape, void *data) {
    if (ndim < 1 || ndim > 8 || !shape) return nullptr;
    tensor_t *t = new (std::nothrow) tensor_t();
    if (!t) return nullptr;
    t->data = data;
    t->ndim = ndim;
    t->dtype = dtype;
    t->layout = LAYOUT_ROW_MAJOR;
    t->ref_count = 1;
    t->is_external = 1;
    memcpy(t->shape, shape, sizeof(int) * (size_t)ndim);
    t->nbytes = shape_product(ndim, shape) * dtype_element_size(dtype);
    t->serial = next_serial();
    return t;
}

tensor_t *tensor_clone(const tensor_t *src) {
    if (!src) return nullptr;
    tensor_t *c = tensor_create(src->ndim, src->shape, src->dtype);
    if (!c) return nullptr;
    c->layout = src->layout;
    memcpy(c->data, src->data, src->nbytes);
    return c;
}

int tensor_transpose(const tensor_t *src, tensor_t **dst) {
    if (!src || !dst || src->ndim != 2 || src->dtype != DTYPE_F32) return -1;
    const int m = src->shape[0], n = src->shape[1];
    const int dims[2] = {n, m};
    tensor_t *t = tensor_create(2, dims, DTYPE_F32);
    if (!t) return -1;
    const float *s = static_cast<const float *>(src->data);
    float *d = static_cast<float *>(t->data);
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) d[(size_t)j * m + i] = s[(size_t)i * n + j];
    *dst = t;
    return 0;
}

size_t tensor_numel(const tensor_t *t) { return t ? shape_product(t->ndim, t->shape) : 0; }

float tensor_get_f32(const tensor_t *t, size_t idx) {
    if (!t || idx >= tensor_numel(t)) return 0.0f;
    if (t->dtype == DTYPE_F32) return static_cast<const float *>(t->data)[idx];
    return 0.0f;  // quantized element access is not provided (tensor.c:238-243)
}

// The reference reads a tensor's host data on every GEMV; here the device copy is marked stale
// so the next GPU use uploads the new values. (Writes through tensor_data_mutable /
// tensor_data_f32 bypass this: their callers invalidate with sapphire_tensor_invalidate.)
int tensor_set_f32(tensor_t *t, size_t idx, float val) {
    if (!t || idx >= tensor_numel(t) || t->dtype != DTYPE_F32) return -1;
    static_cast<float *>(t->data)[idx] = val;
    std::lock_guard<std::mutex> g(t->dev_mu);
    t->dev_stale = t->dev != nullptr || t->dev_tiled != nullptr;
    t->gen.fetch_add(1, std::memory_order_acq_rel);
    return 0;
}

void tensor_ref_inc(tensor_t *t) {
    if (t) t->ref_count++;
}

void tensor_release(tensor_t *t) {
    if (!t) return;
    if (--t->ref_count > 0) return;
    transformer_tensor_released(t->serial);
    if (t->data && !t->is_external) free(t->data);
    tensor_drop_device(t);
    delete t;
}

void tensor_print_info(const tensor_t *t) {
    if (!t) {
        fprintf(stderr, "Tensor: NULL\n");
        return;
    }
    fprintf(stderr, "Tensor shape=[");
    for (int i = 0; i < t->ndim; ++i) fprintf(stderr, i ? ",%d" : "%d", t->shape[i]);
    fprintf(stderr, "] dtype=%s layout=%s %zu bytes ref_count=%d\n", dtype_name(t->dtype),
            t->layout == LAYOUT_ROW_MAJOR ? "row-major" : "col-major", t->nbytes, t->ref_count);
}

int tensor_ndim(const tensor_t *t) { return t ? t->ndim : 0; }
const int *tensor_shape(const tensor_t *t) { return t ? t->shape : nullptr; }
const void *tensor_data(const tensor_t *t) { return t ? t->data : nullptr; }
float *tensor_data_f32(const tensor_t *t) {
    if (!t || t->dtype != DTYPE_F32) return nullptr;
    return static_cast<float *>(t->data);
}
void *tensor_data_mutable(const tensor_t *t) { return t ? t->data : nullptr; }
tensor_dtype_t tensor_dtype(const tensor_t *t) { return t ? t->dtype : DTYPE_F32; }
size_t tensor_nbytes(const tensor_t *t) { return t ? t->nbytes : 0; }
int tensor_ref_count(const tensor_t *t) { return t ? t->ref_count : 0; }

}  // extern "C"

namespace sapphire {

namespace {

// Frees the device copies; the caller holds t->dev_mu.
void drop_device_locked(tensor_t *t) {
    if (t->dev || t->dev_tiled) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(t->dev_device);
        if (t->dev) (void)hipFree(t->dev);
        if (t->dev_tiled) (void)hipFree(t->dev_tiled);
        (void)hipSetDevice(cur);
    }
    t->dev = nullptr;
    t->dev_tiled = nullptr;
    t->dev_bytes = 0;
    t->dev_stale = false;
    t->gen.fetch_add(1, std::memory_order_acq_rel);
}

// Uploads the AoS blocks of a quantized tensor and converts them to `lay` on the device.
void *upload_quant(const tensor_t *t, int lay, hipStream_t s) {
    const int M = t->shape[0], K = t->shape[t->ndim - 1];
    const size_t aos = q_aos_bytes(t->dtype, M, K);
    const size_t bytes = lay == LAYOUT_TILED ? q_tiled_bytes(t->dtype, M, K) : q_packed_bytes(t->dtype, M, K);
    void *dst = nullptr, *tmp = nullptr;
    if (!hip_ok(hipMalloc(&dst, bytes), "hipMalloc(weights)")) return nullptr;
    if (!hip_ok(hipMalloc(&tmp, aos), "hipMalloc(staging)")) { (void)hipFree(dst); return nullptr; }
    bool ok = hip_ok(hipMemcpyAsync(tmp, t->data, aos, hipMemcpyHostToDevice, s), "upload weights") &&
              (lay == LAYOUT_TILED ? launch_to_tiled(t->dtype, tmp, M, K, dst, s)
                                   : launch_repack(t->dtype, tmp, M, K, dst, s)) == 0 &&
              hip_ok(hipStreamSynchronize(s), "repack sync");
    (void)hipFree(tmp);
    if (!ok) { (void)hipFree(dst); return nullptr; }
    return dst;
}

}  // namespace

void tensor_drop_device(tensor_t *t) {
    std::lock_guard<std::mutex> g(t->dev_mu);
    drop_device_locked(t);
}

const void *tensor_device_weights(const tensor_t *tc, int *layout, hipStream_t s) {
    tensor_t *t = const_cast<tensor_t *>(tc);
    std::lock_guard<std::mutex> g(t->dev_mu);
    if (t->dev_stale) drop_device_locked(t);
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (t->dev && t->dev_device == dev) {
        *layout = t->dev_layout;
        return t->dev;
    }
    if (t->dev) {
        set_error("tensor is resident on device %d, current device is %d", t->dev_device, dev);
        return nullptr;
    }
    const int M = t->shape[0], K = t->shape[t->ndim - 1];
    void *dst = nullptr;
    if (is_quant(t->dtype)) {
        // Long matrices (the LM head) go to the matrix-core TILED layout, the rest to PACKED.
        const int lay = (M >= kTiledMinRows && tiled_supported(t->dtype, M, K)) ? LAYOUT_TILED : LAYOUT_PACKED;
        dst = upload_quant(t, lay, s);
        if (!dst) return nullptr;
        t->dev_layout = lay;
        t->dev_bytes = lay == LAYOUT_TILED ? q_tiled_bytes(t->dtype, M, K) : q_packed_bytes(t->dtype, M, K);
    } else {
        const size_t bytes = (size_t)M * (size_t)K * dtype_element_size(t->dtype);
        if (!hip_ok(hipMalloc(&dst, bytes), "hipMalloc(weights)")) return nullptr;
        if (!hip_ok(hipMemcpyAsync(dst, t->data, bytes, hipMemcpyHostToDevice, s), "upload weights") ||
            !hip_ok(hipStreamSynchronize(s), "upload sync")) {
            (void)hipFree(dst);
            return nullptr;
        }
        t->dev_layout = LAYOUT_AOS;
        t->dev_bytes = bytes;
    }
    t->dev = dst;
    t->dev_device = dev;
    *layout = t->dev_layout;
    return dst;
}

const void *tensor_device_tiled(const tensor_t *tc, hipStream_t s) {
    int layout = 0;
    const void *w = tensor_device_weights(tc, &layout, s);
    if (!w) return nullptr;
    if (layout == LAYOUT_TILED) return w;
    tensor_t *t = const_cast<tensor_t *>(tc);
    const int M = t->shape[0], K = t->shape[t->ndim - 1];
    if (!is_quant(t->dtype) || !tiled_layout_ok(t->dtype, M, K)) {
        set_error("no TILED layout for this tensor (dtype %d, K=%d)", (int)t->dtype, K);
        return nullptr;
    }
    std::lock_guard<std::mutex> g(t->dev_mu);
    if (!t->dev_tiled) t->dev_tiled = upload_quant(t, LAYOUT_TILED, s);
    return t->dev_tiled;
}

}  // namespace sapphire

extern "C" int sapphire_tensor_invalidate(tensor_t *t) {
    if (!t) return -1;
    tensor_drop_device(t);
    return 0;
}

extern "C" const void *sapphire_tensor_device_data(const tensor_t *t, int *layout, void *stream) {
    if (!t || !layout) return nullptr;
    return tensor_device_weights(t, layout, as_stream(stream));
}
