// dispatch.cpp - the host-pointer API of include/kernels.h on the GPU.
//
// Replaces src/kernels/pool.c + dispatch.c (and the vector primitives of
// normalization.c, activations.c, utils.c): same names, argument meanings and return
// codes; each call stages its host vectors through pinned buffers, enqueues the HIP
// kernels on the context's stream and waits, so callers see the same synchronous
// behaviour as the reference's pthread pool.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>
#include <unistd.h>
#include <vector>

#include <cmath>

#include "../../include/kernels.h"
#include "../../include/quantize.h"
#include "../../include/rope.h"
#include "internal.h"
#include "tensor_impl.h"

using namespace sapphire;

struct sapphire_context {
    int num_threads = 1;
    int chunk_size = 16;
    int initialized = 0;
    int device = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;                     // one call in flight per context (pool.c:324,359)
    // pinned host staging and device buffers, grown on demand
    void *h_stage = nullptr;
    size_t h_bytes = 0;
    void *d_stage = nullptr;
    size_t d_bytes = 0;
};

namespace {

// Grow-only staging. Layout per call is chosen by the caller as byte offsets.
bool ensure_staging(kernel_context_t *c, size_t host_bytes, size_t dev_bytes) {
    if (host_bytes > c->h_bytes) {
        if (c->h_stage) (void)hipHostFree(c->h_stage);
        c->h_stage = nullptr;
        c->h_bytes = 0;
        const size_t want = std::max(host_bytes, size_t(1) << 20);
        if (!hip_ok(hipHostMalloc(&c->h_stage, want, hipHostMallocDefault), "hipHostMalloc")) return false;
        c->h_bytes = want;
    }
    if (dev_bytes > c->d_bytes) {
        if (c->d_stage) (void)hipFree(c->d_stage);
        c->d_stage = nullptr;
        c->d_bytes = 0;
        const size_t want = std::max(dev_bytes, size_t(1) << 20);
        if (!hip_ok(hipMalloc(&c->d_stage, want), "hipMalloc(staging)")) return false;
        c->d_bytes = want;
    }
    return true;
}

inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// The context used where the reference API has none (row kernels, vector primitives,
// NULL-context F32/BF16 GEMV).
kernel_context_t *default_ctx() {
    static std::once_flag once;
    static kernel_context_t *ctx = nullptr;
    std::call_once(once, [] {
        kernel_context_t *c = kernel_ctx_create(1, 16);
        if (c && kernel_ctx_init(c) == 0) ctx = c;
        else if (c) kernel_ctx_destroy(c);
    });
    return ctx;
}

// Runs f(stream) with n_in host arrays uploaded and n_out host arrays downloaded.
struct HostVec { const void *h; void *out_h; size_t bytes; };

template <class F>
int run_staged(kernel_context_t *c, std::initializer_list<HostVec> ins, std::initializer_list<HostVec> outs, F &&f) {
    std::lock_guard<std::mutex> g(c->mu);
    size_t total = 0;
    for (const auto &v : ins) total += align256(v.bytes);
    for (const auto &v : outs) total += align256(v.bytes);
    if (!ensure_staging(c, total, total)) return -1;
    if (!hip_ok(hipSetDevice(c->device), "hipSetDevice")) return -1;
    char *hb = static_cast<char *>(c->h_stage);
    char *db = static_cast<char *>(c->d_stage);
    std::vector<void *> dev_in, dev_out;
    size_t off = 0;
    for (const auto &v : ins) {
        memcpy(hb + off, v.h, v.bytes);
        if (!hip_ok(hipMemcpyAsync(db + off, hb + off, v.bytes, hipMemcpyHostToDevice, c->stream), "H2D"))
            return -1;
        dev_in.push_back(db + off);
        off += align256(v.bytes);
    }
    const size_t out_off = off;
    for (const auto &v : outs) {
        dev_out.push_back(db + off);
        off += align256(v.bytes);
    }
    if (f(dev_in, dev_out, c->stream) != 0) return -1;
    off = out_off;
    for (const auto &v : outs) {
        if (!hip_ok(hipMemcpyAsync(hb + off, db + off, v.bytes, hipMemcpyDeviceToHost, c->stream), "D2H"))
            return -1;
        off += align256(v.bytes);
    }
    if (!hip_ok(hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return -1;
    off = out_off;
    for (const auto &v : outs) {
        memcpy(v.out_h, hb + off, v.bytes);
        off += align256(v.bytes);
    }
    return 0;
}

// GEMV/GEMM core: Y[b*M + r] = A[r,:] . X[b*K ...] for b < batch.
int gemv_exec(kernel_context_t *c, const tensor_t *A, const float *X, float *Y, int batch) {
    if (!c || !c->initialized) {
        set_error("kernel context not initialized");
        return -1;
    }
    const int M = A->shape[0], K = A->shape[A->ndim - 1];
    const int dt = A->dtype;
    if (dt != DT_F32 && dt != DT_BF16 && !is_quant(dt)) {
        set_error("kernel_backend_exec: unsupported dtype %d", dt);
        return -1;
    }
    if (!A->data) return -1;
    // Quantized rows hold ceil(K/32) whole blocks; the activation is zero-padded to match.
    const int Kp = is_quant(dt) ? (K + 31) / 32 * 32 : K;
    std::lock_guard<std::mutex> g(c->mu);
    if (!hip_ok(hipSetDevice(c->device), "hipSetDevice")) return -1;
    int layout = 0;
    // batches of quantized rows run on the matrix cores from a TILED copy when K allows it
    const bool mm = is_quant(dt) && batch > 1 && tiled_layout_ok(dt, M, Kp);
    const void *w = mm ? tensor_device_tiled(A, c->stream) : tensor_device_weights(A, &layout, c->stream);
    if (!w) return -1;
    const size_t xb = (size_t)batch * Kp * sizeof(float), yb = (size_t)batch * M * sizeof(float);
    const size_t wsb = mm ? gemm_workspace_bytes(M, Kp) : 0;
    if (!ensure_staging(c, align256(xb) + align256(yb), align256(xb) + align256(yb) + wsb)) return -1;
    char *hb = static_cast<char *>(c->h_stage);
    char *db = static_cast<char *>(c->d_stage);
    float *hx = reinterpret_cast<float *>(hb), *hy = reinterpret_cast<float *>(hb + align256(xb));
    float *dx = reinterpret_cast<float *>(db), *dy = reinterpret_cast<float *>(db + align256(xb));
    for (int b = 0; b < batch; ++b) {
        memcpy(hx + (size_t)b * Kp, X + (size_t)b * K, sizeof(float) * (size_t)K);
        if (Kp > K) memset(hx + (size_t)b * Kp + K, 0, sizeof(float) * (size_t)(Kp - K));
    }
    if (!hip_ok(hipMemcpyAsync(dx, hx, xb, hipMemcpyHostToDevice, c->stream), "H2D x")) return -1;
    int rc;
    if (is_quant(dt)) {
        if (mm)
            rc = launch_gemm_tiled(dt, w, M, Kp, dx, batch, dy, db + align256(xb) + align256(yb), c->stream);
        else
            rc = batch == 1 ? launch_gemv_q(dt, layout, w, M, Kp, dx, dy, c->stream)
                            : launch_gemm_q(dt, layout, w, M, Kp, dx, dy, batch, c->stream);
    } else if (dt == DT_BF16 && batch > 1 && gemm_bf16_supported(w, M, K)) {
        rc = launch_gemm_bf16(w, M, K, dx, K, batch, dy, M, c->stream);   // weights read once per 16
    } else {
        rc = 0;
        for (int b = 0; b < batch && rc == 0; ++b)
            rc = launch_gemv_f(dt, w, M, K, dx + (size_t)b * K, dy + (size_t)b * M, c->stream);
    }
    if (rc != 0) return -1;
    if (!hip_ok(hipMemcpyAsync(hy, dy, yb, hipMemcpyDeviceToHost, c->stream), "D2H y")) return -1;
    if (!hip_ok(hipStreamSynchronize(c->stream), "hipStreamSynchronize")) return -1;
    memcpy(Y, hy, yb);
    return 0;
}

bool valid_matrix(const tensor_t *A, const char *who) {
    if (tensor_ndim(A) != 2) {
        set_error("%s weight must be 2D", who);
        return false;
    }
    const int *shape = tensor_shape(A);
    if (!shape || shape[0] <= 0 || shape[1] <= 0) {
        set_error("%s invalid shape", who);
        return false;
    }
    return true;
}

float row_dot(int dt, const void *W_row, const float *x, int block_count, int block_size) {
    if (block_size != 32 || !W_row || !x || block_count <= 0) return 0.0f;
    kernel_context_t *c = default_ctx();
    if (!c) return 0.0f;
    const int K = block_count * 32;
    float y = 0.0f;
    const size_t wb = q_aos_bytes(dt, 1, K);
    const int rc = run_staged(c, {HostVec{W_row, nullptr, wb}, HostVec{x, nullptr, sizeof(float) * (size_t)K}},
                              {HostVec{nullptr, &y, sizeof(float)}},
                              [&](std::vector<void *> &in, std::vector<void *> &out, hipStream_t s) {
                                  return launch_gemv_q(dt, LAYOUT_AOS, in[0], 1, K, static_cast<float *>(in[1]),
                                                       static_cast<float *>(out[0]), s);
                              });
    return rc == 0 ? y : 0.0f;
}

int unary_host(float *x, int n, int op, float a) {
    if (!x || n <= 0) return -1;
    kernel_context_t *c = default_ctx();
    if (!c) return -1;
    const size_t b = sizeof(float) * (size_t)n;
    return run_staged(c, {HostVec{x, nullptr, b}}, {HostVec{nullptr, x, b}},
                      [&](std::vector<void *> &in, std::vector<void *> &out, hipStream_t s) {
                          if (launch_unary(static_cast<float *>(in[0]), n, op, a, s) != 0) return -1;
                          return hip_ok(hipMemcpyAsync(out[0], in[0], b, hipMemcpyDeviceToDevice, s), "D2D") ? 0
                                                                                                              : -1;
                      });
}

int norm_host(float *out, const float *in, const float *w, float eps, int dim, int batch, bool delta) {
    if (!out || !in || !w || dim <= 0 || batch <= 0 || eps < 0.0f) return -1;
    kernel_context_t *c = default_ctx();
    if (!c) return -1;
    const size_t b = sizeof(float) * (size_t)dim * (size_t)batch, wb = sizeof(float) * (size_t)dim;
    return run_staged(c, {HostVec{in, nullptr, b}, HostVec{w, nullptr, wb}}, {HostVec{nullptr, out, b}},
                      [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                          return launch_rmsnorm(static_cast<float *>(o[0]), static_cast<float *>(i[0]),
                                                static_cast<float *>(i[1]), eps, dim, batch, delta, s);
                      });
}

// One F32 / BF16 row of cols elements dotted with x (the row kernels of f32_avx.c / bf16_avx.c)
// as a one-row GEMV.
float f_row_dot(int dt, const void *W_row, const float *x, int block_count, int block_size) {
    if (!W_row || !x) return 0.0f;
    const long cols = block_size == 1 ? (long)block_count : (long)block_count * (long)block_size;
    if (cols <= 0 || cols > (1L << 28)) return 0.0f;
    kernel_context_t *c = default_ctx();
    if (!c) return 0.0f;
    const int K = (int)cols;
    const size_t es = dt == DT_F32 ? 4 : 2;
    float y = 0.0f;
    const int rc = run_staged(c, {HostVec{W_row, nullptr, es * (size_t)K}, HostVec{x, nullptr, sizeof(float) * (size_t)K}},
                              {HostVec{nullptr, &y, sizeof(float)}},
                              [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                                  return launch_gemv_f(dt, i[0], 1, K, static_cast<float *>(i[1]),
                                                       static_cast<float *>(o[0]), s);
                              });
    return rc == 0 ? y : 0.0f;
}

// One weight row times a batch (kernel_gemm_{f32,bf16}_avx2): Y[b * out_stride] = w . X[b].
// Computed as the GEMV of the batch matrix X [batch][d_model] with w as the vector (the same
// products; BF16 weights widen exactly to fp32 first).
void gemm_row(int dt, const gemm_args_t *a) {
    if (!a || !a->w_row || !a->X || !a->Y || a->batch_size <= 0 || a->d_model <= 0) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    const int B = a->batch_size, K = a->d_model;
    const size_t es = dt == DT_F32 ? 4 : 2;
    std::vector<float> y((size_t)B), wf((size_t)K);
    const int rc = run_staged(
        c, {HostVec{a->w_row, nullptr, es * (size_t)K}, HostVec{a->X, nullptr, sizeof(float) * (size_t)B * K}},
        {HostVec{nullptr, y.data(), sizeof(float) * (size_t)B}, HostVec{nullptr, wf.data(), sizeof(float) * (size_t)K}},
        [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
            float *w = static_cast<float *>(i[0]);
            if (dt == DT_BF16) {
                w = static_cast<float *>(o[1]);
                if (launch_bf16_to_f32(w, static_cast<uint16_t *>(i[0]), K, s) != 0) return -1;
            }
            return launch_gemv_f(DT_F32, i[1], B, K, w, static_cast<float *>(o[0]), s);
        });
    if (rc != 0) return;
    for (int b = 0; b < B; ++b) a->Y[(size_t)b * (size_t)a->out_stride] = y[(size_t)b];
}

}  // namespace

extern "C" {

kernel_context_t *kernel_ctx_create(int num_threads, int chunk_size) {
    if (num_threads <= 0) {
        num_threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
        if (num_threads <= 0) num_threads = 1;
    }
    if (chunk_size <= 0) chunk_size = 16;
    kernel_context_t *c = new (std::nothrow) kernel_context_t();
    if (!c) return nullptr;
    c->num_threads = num_threads;
    c->chunk_size = chunk_size;
    return c;
}

int kernel_ctx_init(kernel_context_t *c) {
    if (!c) {
        set_error("kernel_ctx_init: context is NULL");
        return -1;
    }
    if (c->initialized) return 0;
    if (!hip_ok(hipGetDevice(&c->device), "hipGetDevice")) return -1;
    if (!hip_ok(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate")) return -1;
    c->initialized = 1;
    return 0;
}

void kernel_ctx_destroy(kernel_context_t *c) {
    if (!c) return;
    if (c->initialized) {
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
        (void)hipStreamDestroy(c->stream);
    }
    if (c->h_stage) (void)hipHostFree(c->h_stage);
    if (c->d_stage) (void)hipFree(c->d_stage);
    delete c;
}

int kernel_parallel_for(kernel_context_t *c, parallel_for_fn_t fn, void *arg, int n) {
    if (!c || !fn || n <= 0) return -1;
    std::lock_guard<std::mutex> g(c->mu);
    const int nt = std::min(c->num_threads, n);
    if (nt <= 1) {
        for (int i = 0; i < n; ++i) fn(arg, i);
        return 0;
    }
    std::atomic<int> next{0};
    auto worker = [&] {
        for (int i = next.fetch_add(1); i < n; i = next.fetch_add(1)) fn(arg, i);
    };
    std::vector<std::thread> th;
    th.reserve((size_t)nt - 1);
    for (int t = 1; t < nt; ++t) th.emplace_back(worker);
    worker();
    for (auto &t : th) t.join();
    return 0;
}

float quantized_gemv_q4_0_aligned(const void *W, const float *x, int nb, int bs) { return row_dot(DT_Q4_0, W, x, nb, bs); }
float quantized_gemv_q4_0_unaligned(const void *W, const float *x, int nb, int bs) { return row_dot(DT_Q4_0, W, x, nb, bs); }
float quantized_gemv_q8_0_aligned(const void *W, const float *x, int nb, int bs) { return row_dot(DT_Q8_0, W, x, nb, bs); }
float quantized_gemv_q8_0_unaligned(const void *W, const float *x, int nb, int bs) { return row_dot(DT_Q8_0, W, x, nb, bs); }
float quantized_gemv_bf16_avx2(const void *W, const float *x, int nb, int bs) { return f_row_dot(DT_BF16, W, x, nb, bs); }
float quantized_gemv_bf16_scalar(const void *W, const float *x, int nb, int bs) { return f_row_dot(DT_BF16, W, x, nb, bs); }
float quantized_gemv_f32_avx2(const void *W, const float *x, int nb, int bs) { return f_row_dot(DT_F32, W, x, nb, bs); }
float quantized_gemv_f32_scalar(const void *W, const float *x, int nb, int bs) { return f_row_dot(DT_F32, W, x, nb, bs); }
void kernel_gemm_f32_avx2(const gemm_args_t *args) { gemm_row(DT_F32, args); }
void kernel_gemm_bf16_avx2(const gemm_args_t *args) { gemm_row(DT_BF16, args); }

int kernel_gemv(kernel_context_t *ctx, float *y, const tensor_t *A, const float *x) {
    if (!y || !A || !x) {
        set_error("kernel_gemv null pointer");
        return -1;
    }
    if (!valid_matrix(A, "kernel_gemv")) return -1;
    switch (tensor_dtype(A)) {
        case DTYPE_F32:
        case DTYPE_BF16:
        case DTYPE_Q4_0:
        case DTYPE_Q8_0:
            if (!ctx) {
                if (tensor_dtype(A) == DTYPE_F32 || tensor_dtype(A) == DTYPE_BF16) ctx = default_ctx();
                else {
                    set_error("kernel_gemv requires non-NULL context for quantized weights");
                    return -1;
                }
            }
            return gemv_exec(ctx, A, x, y, 1) == 0 ? 0 : -1;
        default:
            set_error("kernel_gemv unsupported dtype %d", (int)tensor_dtype(A));
            return -1;
    }
}

int kernel_quantize(kernel_context_t *ctx, void *blocks, tensor_dtype_t dtype, const tensor_t *src) {
    if (!blocks || !src || !src->data) {
        set_error("kernel_quantize null pointer");
        return -1;
    }
    if (tensor_ndim(src) != 2 || (tensor_dtype(src) != DTYPE_F32 && tensor_dtype(src) != DTYPE_BF16) ||
        (dtype != DTYPE_Q4_0 && dtype != DTYPE_Q8_0)) {
        set_error("kernel_quantize: source must be a 2-D F32 or BF16 tensor, destination Q4_0 or Q8_0");
        return -1;
    }
    const int M = tensor_shape(src)[0], K = tensor_shape(src)[1];
    if (M <= 0 || K <= 0) {
        set_error("kernel_quantize: non-positive shape");
        return -1;
    }
    kernel_context_t *c = ctx ? ctx : default_ctx();
    if (!c || !c->initialized) {
        set_error("kernel context not initialized");
        return -1;
    }
    const int sdt = tensor_dtype(src);
    const size_t sb = (size_t)M * K * (sdt == DTYPE_F32 ? 4 : 2);
    const size_t ob = q_aos_bytes(dtype, M, K);
    return run_staged(c, {HostVec{src->data, nullptr, sb}}, {HostVec{nullptr, blocks, ob}},
                      [&](std::vector<void *> &in, std::vector<void *> &out, hipStream_t s) {
                          return launch_quantize(dtype, sdt, in[0], M, K, out[0], s);
                      });
}

int kernel_gemm(kernel_context_t *ctx, float *Y, const tensor_t *A, const float *X, int batch_size, int out_stride) {
    (void)out_stride;
    if (!Y || !A || !X || batch_size <= 0) {
        set_error("kernel_gemm invalid arguments");
        return -1;
    }
    if (!ctx) {
        set_error("kernel_gemm requires non-NULL context");
        return -1;
    }
    if (!valid_matrix(A, "kernel_gemm")) return -1;
    return gemv_exec(ctx, A, X, Y, batch_size) == 0 ? 0 : -1;
}

int kernel_gemv_tensor(kernel_context_t *ctx, const tensor_t *y, const tensor_t *A, const tensor_t *x) {
    if (!y || !A || !x) {
        set_error("kernel_gemv_tensor null pointer");
        return -1;
    }
    if (tensor_ndim(y) != 1 || tensor_dtype(y) != DTYPE_F32) {
        set_error("kernel_gemv_tensor output must be 1D F32 tensor");
        return -1;
    }
    if (tensor_ndim(x) != 1 || tensor_dtype(x) != DTYPE_F32) {
        set_error("kernel_gemv_tensor input must be 1D F32 tensor");
        return -1;
    }
    const int *sa = tensor_shape(A), *sx = tensor_shape(x), *sy = tensor_shape(y);
    if (!sa || !sx || !sy || tensor_ndim(A) < 2) {
        set_error("kernel_gemv_tensor shapes invalid");
        return -1;
    }
    if (sa[1] != sx[0] || sy[0] != sa[0]) {
        set_error("kernel_gemv_tensor shape mismatch");
        return -1;
    }
    return kernel_gemv(ctx, tensor_data_f32(y), A, static_cast<const float *>(tensor_data(x)));
}

int kernel_gemv_add(kernel_context_t *ctx, float *y, const tensor_t *A, const float *x, float alpha) {
    if (!y || !A || !x) {
        set_error("kernel_gemv_add null pointer");
        return -1;
    }
    if (tensor_ndim(A) != 2) {
        set_error("kernel_gemv_add weight must be 2D");
        return -1;
    }
    const int m = tensor_shape(A)[0];
    std::vector<float> tmp((size_t)std::max(m, 0));
    if (kernel_gemv(ctx, tmp.data(), A, x) != 0) return -1;
    kernel_context_t *c = default_ctx();
    if (!c) return -1;
    const size_t b = sizeof(float) * (size_t)m;
    return run_staged(c, {HostVec{y, nullptr, b}, HostVec{tmp.data(), nullptr, b}}, {HostVec{nullptr, y, b}},
                      [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                          if (launch_axpy(static_cast<float *>(i[0]), static_cast<float *>(i[1]), m, alpha, true, s))
                              return -1;
                          return hip_ok(hipMemcpyAsync(o[0], i[0], b, hipMemcpyDeviceToDevice, s), "D2D") ? 0 : -1;
                      });
}

int kernel_gemv_batch(kernel_context_t *ctx, float *Y, const tensor_t *A, const float *X, int batch_size) {
    if (!Y || !A || !X || batch_size <= 0) {
        set_error("kernel_gemv_batch invalid arguments");
        return -1;
    }
    if (tensor_ndim(A) != 2) {
        set_error("kernel_gemv_batch weight must be 2D");
        return -1;
    }
    if (batch_size > 1 && ctx) return gemv_exec(ctx, A, X, Y, batch_size) == 0 ? 0 : -1;
    const int m = tensor_shape(A)[0], n = tensor_shape(A)[1];
    for (int k = 0; k < batch_size; ++k)
        if (kernel_gemv(ctx, Y + (size_t)k * m, A, X + (size_t)k * n) != 0) return -1;
    return 0;
}

int kernel_get_simd_lane_count(tensor_dtype_t dtype) {
    switch (dtype) {
        case DTYPE_F32:
        case DTYPE_BF16:
        case DTYPE_F16:
        case DTYPE_Q4_0:
        case DTYPE_Q8_0:
            return 8;
        default:
            return 1;
    }
}

void gelu_inplace(float *x, int n) { (void)unary_host(x, n, UOP_GELU, 0.f); }
void silu_inplace(float *x, int n) { (void)unary_host(x, n, UOP_SILU, 0.f); }
void relu_inplace(float *x, int n) { (void)unary_host(x, n, UOP_RELU, 0.f); }

// Scalar activations (activations.c:16-105): one value's host arithmetic with libm, written
// with the fused multiply-add the reference build contracts x + 0.044715 x^3 into.
float silu(float x) {
    const float sigmoid = 1.0f / (1.0f + expf(-x));
    return x * sigmoid;
}
float relu(float x) { return x > 0.0f ? x : 0.0f; }
float gelu(float x) {
    const float y = 0.7978845608f * fmaf((0.044715f * x) * x, x, x);
    return 0.5f * x * (1.0f + tanhf(y));
}
float geglu(float x, float y) { return x * gelu(y); }

// rope.c:41-63 on the host with libm, the same formula and rounding as the reference.
int rope_precompute_freqs(float *freqs_cos, float *freqs_sin, int d_k, int max_context_len, float rope_base) {
    if (!freqs_cos || !freqs_sin) return -1;
    const int half = d_k / 2;
    for (int pos = 0; pos < max_context_len; ++pos)
        for (int m = 0; m < half; ++m) {
            const float freq = 1.0f / powf(rope_base, 2.0f * (float)m / (float)d_k);
            const float angle = (float)pos * freq;
            const float cv = cosf(angle), sv = sinf(angle);
            const size_t at = (size_t)pos * (size_t)d_k + (size_t)m;
            freqs_cos[at] = freqs_cos[at + half] = cv;
            freqs_sin[at] = freqs_sin[at + half] = sv;
        }
    return 0;
}

// rope.c:99-117: the half-split rotation of one head on the GPU, with table row pos.
void rope_apply_fast(float *x, int pos, int head_dim, const float *freqs_cos, const float *freqs_sin) {
    if (!x || !freqs_cos || !freqs_sin || head_dim < 2 || pos < 0) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    const int half = head_dim / 2;
    const size_t row = (size_t)pos * (size_t)head_dim, xb = sizeof(float) * (size_t)head_dim;
    (void)run_staged(c,
                     {HostVec{x, nullptr, xb}, HostVec{freqs_cos + row, nullptr, sizeof(float) * (size_t)half},
                      HostVec{freqs_sin + row, nullptr, sizeof(float) * (size_t)half}},
                     {HostVec{nullptr, x, xb}},
                     [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                         if (launch_rope(static_cast<float *>(i[0]), 1, head_dim, 0, static_cast<float *>(i[1]),
                                         static_cast<float *>(i[2]), s) != 0)
                             return -1;
                         return hip_ok(hipMemcpyAsync(o[0], i[0], xb, hipMemcpyDeviceToDevice, s), "D2D") ? 0 : -1;
                     });
}

// rope.c:17-25 with positional_encoding.c:16-40,76-104: pair p = (x[2p], x[2p+1]) for
// 2p + 1 < head_dim is rotated by theta_p = pos * powf(1/base, 2p/head_dim). The angles are
// host libm values, the rotation runs on the GPU.
void apply_rope(float *x, int pos, int head_dim, float base) {
    if (!x || head_dim < 2) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    const int np = head_dim / 2;
    std::vector<float> cs((size_t)np), sn((size_t)np);
    for (int p = 0; p < np; ++p) {
        const float inv_freq = powf(1.0f / base, 2.0f * (float)p / (float)head_dim);
        const float theta = (float)pos * inv_freq;
        cs[(size_t)p] = cosf(theta);
        sn[(size_t)p] = sinf(theta);
    }
    const size_t xb = sizeof(float) * (size_t)head_dim, tb = sizeof(float) * (size_t)np;
    (void)run_staged(c, {HostVec{x, nullptr, xb}, HostVec{cs.data(), nullptr, tb}, HostVec{sn.data(), nullptr, tb}},
                     {HostVec{nullptr, x, xb}},
                     [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                         if (launch_rope_pairs(static_cast<float *>(i[0]), np, static_cast<float *>(i[1]),
                                               static_cast<float *>(i[2]), s) != 0)
                             return -1;
                         return hip_ok(hipMemcpyAsync(o[0], i[0], xb, hipMemcpyDeviceToDevice, s), "D2D") ? 0 : -1;
                     });
}

void apply_rope_default(float *x, int pos, int head_dim) { apply_rope(x, pos, head_dim, 1000000.0f); }

void vec_scale(float *x, float s, int n) {
    if (s == 1.0f) return;  // utils.c:88
    (void)unary_host(x, n, UOP_SCALE, s);
}

void vec_softcap(float *x, int n, float cap) {
    if (cap <= 0.0f) return;  // utils.c:120
    (void)unary_host(x, n, UOP_SOFTCAP, cap);
}

int sapphire_geglu(float *output, const float *input, size_t size) {
    if (!output || !input || size == 0 || (size % 2) != 0) return -1;
    kernel_context_t *c = default_ctx();
    if (!c) return -1;
    const int n = (int)(size / 2);
    return run_staged(c, {HostVec{input, nullptr, sizeof(float) * size}},
                      {HostVec{nullptr, output, sizeof(float) * (size_t)n}},
                      [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                          return launch_geglu_split(static_cast<float *>(o[0]), static_cast<float *>(i[0]), n, s);
                      });
}

int rmsnorm(float *out, const float *in, const float *w, float eps, int dim) {
    return norm_host(out, in, w, eps, dim, 1, false);
}

int rmsnorm_delta(float *out, const float *in, const float *w, float eps, int dim) {
    return norm_host(out, in, w, eps, dim, 1, true);
}

int rmsnorm_batch(float *out, const float *in, const float *w, float eps, int batch, int dim) {
    return norm_host(out, in, w, eps, dim, batch, false);
}

void softmax(float *scores, int n) {
    if (n <= 0 || !scores) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    const size_t b = sizeof(float) * (size_t)n;
    (void)run_staged(c, {HostVec{scores, nullptr, b}}, {HostVec{nullptr, scores, b}},
                     [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                         float *scratch = softmax_partials_scratch();   // the current device's
                         if (!scratch) return -1;
                         return launch_softmax_argmax(static_cast<float *>(i[0]), n, static_cast<float *>(o[0]),
                                                      nullptr, scratch, s);
                     });
}

void vec_add(float *dst, const float *src, int n) {
    if (!dst || !src || n <= 0) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    const size_t b = sizeof(float) * (size_t)n;
    (void)run_staged(c, {HostVec{dst, nullptr, b}, HostVec{src, nullptr, b}}, {HostVec{nullptr, dst, b}},
                     [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                         if (launch_axpy(static_cast<float *>(i[0]), static_cast<float *>(i[1]), n, 1.f, false, s))
                             return -1;
                         return hip_ok(hipMemcpyAsync(o[0], i[0], b, hipMemcpyDeviceToDevice, s), "D2D") ? 0 : -1;
                     });
}

void vec_copy(float *dst, const float *src, int n) {
    if (!dst || !src || n <= 0) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    const size_t b = sizeof(float) * (size_t)n;
    (void)run_staged(c, {HostVec{src, nullptr, b}}, {HostVec{nullptr, dst, b}},
                     [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                         return hip_ok(hipMemcpyAsync(o[0], i[0], b, hipMemcpyDeviceToDevice, s), "D2D") ? 0 : -1;
                     });
}

float vec_dot(const float *a, const float *b, int n) {
    if (!a || !b || n <= 0) return 0.0f;
    kernel_context_t *c = default_ctx();
    if (!c) return 0.0f;
    float r = 0.0f;
    const size_t bytes = sizeof(float) * (size_t)n;
    const int rc = run_staged(c, {HostVec{a, nullptr, bytes}, HostVec{b, nullptr, bytes}},
                              {HostVec{nullptr, &r, sizeof(float)}},
                              [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                                  return launch_dot_ref(static_cast<float *>(i[0]), static_cast<float *>(i[1]), n,
                                                        static_cast<float *>(o[0]), s);
                              });
    return rc == 0 ? r : 0.0f;
}

void bf16_to_f32_vec(float *dst, const uint16_t *src, int n) {
    if (!dst || !src || n <= 0) return;
    kernel_context_t *c = default_ctx();
    if (!c) return;
    (void)run_staged(c, {HostVec{src, nullptr, sizeof(uint16_t) * (size_t)n}},
                     {HostVec{nullptr, dst, sizeof(float) * (size_t)n}},
                     [&](std::vector<void *> &i, std::vector<void *> &o, hipStream_t s) {
                         return launch_bf16_to_f32(static_cast<float *>(o[0]), static_cast<uint16_t *>(i[0]), n, s);
                     });
}

const float *get_norm_weights(const tensor_t *weight, float *scratch, int n) {
    if (!weight) return nullptr;
    if (tensor_dtype(weight) == DTYPE_BF16) {
        bf16_to_f32_vec(scratch, static_cast<const uint16_t *>(tensor_data(weight)), n);
        return scratch;
    }
    return static_cast<const float *>(tensor_data(weight));
}

}  // extern "C"
