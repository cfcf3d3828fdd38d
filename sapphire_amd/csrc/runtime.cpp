// runtime.cpp - error reporting, device-memory/stream/event wrappers and the
// device-pointer entry points of sapphire_hip.h.
#include <cstdarg>
#include <cstring>
#include <mutex>

#include "../../include/quantize.h"
#include "../../include/sapphire_hip.h"
#include "internal.h"

namespace sapphire {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "[sapphire-hip] %s\n", g_err);
}

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_error("%s: %s", what, hipGetErrorString(e));
    return false;
}

}  // namespace sapphire

using namespace sapphire;

namespace {

bool valid_quant_args(int dtype, const void *w, int M, int K) {
    if (!is_quant(dtype)) { set_error("dtype %d is not Q4_0/Q8_0", dtype); return false; }
    if (!w || M <= 0 || K <= 0) { set_error("bad quantized matrix arguments (w=%p M=%d K=%d)", w, M, K); return false; }
    if ((reinterpret_cast<uintptr_t>(w) & 3u) != 0) { set_error("weights must be 4-byte aligned"); return false; }
    return true;
}

}  // namespace

extern "C" {

const char *sapphire_last_error(void) { return g_err; }
const char *sapphire_version(void) { return "sapphire-hip 0.1 (gfx950)"; }

int sapphire_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int sapphire_set_device(int device) { SPH_CHECK(hipSetDevice(device)); return 0; }

void *sapphire_malloc(size_t bytes) {
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc")) return nullptr;
    return p;
}

int sapphire_free(void *p) { SPH_CHECK(hipFree(p)); return 0; }

int sapphire_memcpy_h2d(void *dst, const void *src, size_t n) {
    SPH_CHECK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice));
    return 0;
}

int sapphire_memcpy_d2h(void *dst, const void *src, size_t n) {
    SPH_CHECK(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost));
    return 0;
}

int sapphire_memcpy_d2d(void *dst, const void *src, size_t n, void *stream) {
    SPH_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, as_stream(stream)));
    return 0;
}

// Blocking: the fill is complete on return, so work on any stream (non-blocking ones
// included) sees it.
int sapphire_memset(void *p, int v, size_t n) {
    SPH_CHECK(hipMemset(p, v, n));
    SPH_CHECK(hipDeviceSynchronize());
    return 0;
}
int sapphire_synchronize(void) { SPH_CHECK(hipDeviceSynchronize()); return 0; }

void *sapphire_stream_create(void) {
    hipStream_t s = nullptr;
    if (!hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate")) return nullptr;
    return s;
}

int sapphire_stream_destroy(void *s) { SPH_CHECK(hipStreamDestroy(as_stream(s))); return 0; }
int sapphire_stream_synchronize(void *s) { SPH_CHECK(hipStreamSynchronize(as_stream(s))); return 0; }

void *sapphire_event_create(void) {
    hipEvent_t e = nullptr;
    if (!hip_ok(hipEventCreate(&e), "hipEventCreate")) return nullptr;
    return e;
}

int sapphire_event_destroy(void *e) { SPH_CHECK(hipEventDestroy(reinterpret_cast<hipEvent_t>(e))); return 0; }

int sapphire_event_record(void *e, void *s) {
    SPH_CHECK(hipEventRecord(reinterpret_cast<hipEvent_t>(e), as_stream(s)));
    return 0;
}

int sapphire_event_synchronize(void *e) {
    SPH_CHECK(hipEventSynchronize(reinterpret_cast<hipEvent_t>(e)));
    return 0;
}

float sapphire_event_elapsed_ms(void *a, void *b) {
    float ms = -1.f;
    if (!hip_ok(hipEventElapsedTime(&ms, reinterpret_cast<hipEvent_t>(a), reinterpret_cast<hipEvent_t>(b)),
                "hipEventElapsedTime"))
        return -1.f;
    return ms;
}

size_t sapphire_q_aos_bytes(int dt, int M, int K) { return is_quant(dt) ? q_aos_bytes(dt, M, K) : 0; }
size_t sapphire_q_packed_bytes(int dt, int M, int K) { return is_quant(dt) ? q_packed_bytes(dt, M, K) : 0; }
size_t sapphire_q_scales_offset(int dt, int M, int K) { return is_quant(dt) ? q_scales_offset(dt, M, K) : 0; }

int sapphire_q_repack_dev(int dt, const void *w_aos, int M, int K, void *w_packed, void *stream) {
    if (!valid_quant_args(dt, w_aos, M, K) || !w_packed) return -1;
    return launch_repack(dt, w_aos, M, K, w_packed, as_stream(stream));
}

size_t sapphire_q_layout_bytes(int dt, int layout, int M, int K) {
    if (!is_quant(dt) || M <= 0 || K <= 0) return 0;
    if (layout == LAYOUT_AOS) return q_aos_bytes(dt, M, K);
    if (layout == LAYOUT_PACKED) return q_packed_bytes(dt, M, K);
    if (layout == LAYOUT_TILED && tiled_layout_ok(dt, M, K)) return q_tiled_bytes(dt, M, K);
    return 0;
}

int sapphire_q_convert_dev(int dt, const void *w_aos, int M, int K, int layout, void *out, void *stream) {
    if (!valid_quant_args(dt, w_aos, M, K) || !out) return -1;
    if (layout == LAYOUT_PACKED) return launch_repack(dt, w_aos, M, K, out, as_stream(stream));
    if (layout == LAYOUT_TILED) {
        if (!tiled_layout_ok(dt, M, K)) {
            set_error("TILED layout needs K to be a multiple of 128 (K=%d)", K);
            return -1;
        }
        return launch_to_tiled(dt, w_aos, M, K, out, as_stream(stream));
    }
    set_error("bad target layout %d", layout);
    return -1;
}

static bool valid_layout(int dt, int layout, int M, int K) {
    if (layout == LAYOUT_AOS || layout == LAYOUT_PACKED) return true;
    if (layout == LAYOUT_TILED && tiled_layout_ok(dt, M, K)) return true;
    set_error("layout %d is not valid for a %d x %d matrix", layout, M, K);
    return false;
}

int sapphire_q_unpack_ints_dev(int dt, int layout, const void *w, int M, int K, int8_t *out, void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !out || !valid_layout(dt, layout, M, K)) return -1;
    return launch_unpack_ints(dt, layout, w, M, K, out, as_stream(stream));
}

int sapphire_q_dequant_dev(int dt, int layout, const void *w, int M, int K, float *out, void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !out || !valid_layout(dt, layout, M, K)) return -1;
    return launch_dequant(dt, layout, w, M, K, out, as_stream(stream));
}

int sapphire_gemv_q_dev(int dt, int layout, const void *w, int M, int K, const float *x, float *y, void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !x || !y) return -1;
    if (K % kBlock != 0) { set_error("K=%d is not a multiple of 32", K); return -1; }
    if (!valid_layout(dt, layout, M, K)) return -1;
    return launch_gemv_q(dt, layout, w, M, K, x, y, as_stream(stream));
}

size_t sapphire_gemm_workspace_bytes(int dt, int M, int K) {
    if (!is_quant(dt) || M <= 0 || K <= 0 || K % kBlock != 0) return 0;
    return gemm_workspace_bytes(M, K);
}

int sapphire_gemm_q_dev(int dt, int layout, const void *w, int M, int K, const float *X, int batch, float *Y,
                        void *ws, void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !X || !Y || batch <= 0) {
        if (batch <= 0) set_error("batch must be positive (got %d)", batch);
        return -1;
    }
    if (K % kBlock != 0) { set_error("K=%d is not a multiple of 32", K); return -1; }
    if (!valid_layout(dt, layout, M, K)) return -1;
    hipStream_t s = as_stream(stream);
    if (layout != LAYOUT_TILED) return launch_gemm_q(dt, layout, w, M, K, X, Y, batch, s);
    if (!ws) { set_error("the TILED GEMM needs a workspace"); return -1; }
    return launch_gemm_tiled(dt, w, M, K, X, batch, Y, ws, s);
}

int sapphire_gemm_q_greedy_dev(int dt, const void *w, int M, int K, const float *X, int batch, int *tokens, void *ws,
                               void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !X || !tokens || !ws || batch <= 0 || batch > 16) {
        if (batch <= 0 || batch > 16) set_error("greedy GEMM: batch must be 1..16 (got %d)", batch);
        else if (!ws) set_error("greedy GEMM: needs a workspace");
        return -1;
    }
    if (!tiled_layout_ok(dt, M, K) || gemm_splits(K) != 1) {
        set_error("greedy GEMM: TILED weights with K a multiple of 128 and at most 1152 (K=%d)", K);
        return -1;
    }
    GemmIn gi;
    gi.x = X;
    gi.ldx = K;
    GemmOut go;
    go.tokens = tokens;
    return launch_gemm_tiled_ex(dt, w, M, K, batch, gi, go, ws, as_stream(stream));
}

int sapphire_gemm_splits(int K) { return K > 0 && K % kBlock == 0 ? gemm_splits(K) : 0; }

int sapphire_gemm_q_fused_dev(int dt, const void *w, int M, int K, int batch, const sapphire_gemm_input_t *in,
                              const sapphire_gemm_output_t *out, void *ws, void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !in || !out) return -1;
    if (!tiled_layout_ok(dt, M, K)) {
        set_error("the fused GEMM takes TILED weights (K a multiple of 128; K=%d)", K);
        return -1;
    }
    GemmIn gi;
    gi.x = in->x;
    gi.ldx = in->ldx;
    gi.parts = in->parts;
    gi.nparts = in->nparts;
    gi.ldp = in->ldp;
    gi.part_stride = in->part_stride;
    gi.w_delta = in->w_delta;
    gi.resid_out = in->resid_out;
    gi.ldr = in->ldr;
    gi.w_norm = in->w_norm;
    gi.eps = in->eps;
    gi.x_blocked = in->x_blocked != 0;
    GemmOut go;
    go.y = out->y;
    go.ldy = out->ldy;
    go.parts = out->parts;
    go.geglu = out->geglu != 0;
    go.y_blocked = out->y_blocked != 0;
    return launch_gemm_tiled_ex(dt, w, M, K, batch, gi, go, ws, as_stream(stream));
}

int sapphire_quantize_dev(int dst_dtype, int src_dtype, const void *src, int M, int K, void *blocks, void *stream) {
    return launch_quantize(dst_dtype, src_dtype, src, M, K, blocks, as_stream(stream));
}

int sapphire_gemm_bf16_dev(const void *w, int M, int K, const float *x, int ldx, int batch, float *y, int ldy,
                           void *stream) {
    return launch_gemm_bf16(w, M, K, x, ldx, batch, y, ldy, as_stream(stream));
}

int sapphire_gemv_f_dev(int dt, const void *w, int M, int K, const float *x, float *y, void *stream) {
    if ((dt != DT_F32 && dt != DT_BF16) || !w || !x || !y || M <= 0 || K <= 0) {
        set_error("bad F32/BF16 GEMV arguments");
        return -1;
    }
    return launch_gemv_f(dt, w, M, K, x, y, as_stream(stream));
}

}  // extern "C"

namespace {

// Per-device scratch for reduction partials (softmax/argmax), allocated and zeroed once
// per device on first use and kept until the process ends. Calls that overlap on one
// device share it. The fused GEMV epilogue owns the first half, the standalone softmax
// the second.
constexpr size_t kPartialBytes = 256 * 1024;
constexpr size_t kFusedBytes = kPartialBytes / 2;

void *partial_scratch() {
    static std::mutex mu;
    static void *scratch[64] = {nullptr};
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= 64) { set_error("device index %d out of range", dev); return nullptr; }
    std::lock_guard<std::mutex> g(mu);
    if (!scratch[dev]) {
        void *p = nullptr;
        if (!hip_ok(hipMalloc(&p, kPartialBytes), "hipMalloc(partials)")) return nullptr;
        // complete before any (possibly non-blocking) stream uses the buffer
        if (!hip_ok(hipMemset(p, 0, kPartialBytes), "hipMemset(partials)") ||
            !hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize")) {
            (void)hipFree(p);
            return nullptr;
        }
        scratch[dev] = p;
    }
    return scratch[dev];
}

float *standalone_part(void *scratch) { return reinterpret_cast<float *>(static_cast<char *>(scratch) + kFusedBytes); }

}  // namespace

namespace sapphire {
float *softmax_partials_scratch() {
    void *s = partial_scratch();
    return s ? standalone_part(s) : nullptr;
}
}  // namespace sapphire

extern "C" {

int sapphire_softmax_argmax_dev(const float *logits, int n, float *probs, int *argmax, void *stream) {
    if (!logits || n <= 0 || (!probs && !argmax)) { set_error("bad softmax arguments"); return -1; }
    void *scratch = partial_scratch();
    if (!scratch) return -1;
    return launch_softmax_argmax(logits, n, probs, argmax, standalone_part(scratch), as_stream(stream));
}

int sapphire_gemv_softmax_dev(int dt, int layout, const void *w, int M, int K, const float *x, float *logits,
                              float *probs, int *argmax, void *stream) {
    if (!valid_quant_args(dt, w, M, K) || !x || !logits || (!probs && !argmax)) return -1;
    if (K % kBlock != 0) { set_error("K=%d is not a multiple of 32", K); return -1; }
    if (!valid_layout(dt, layout, M, K)) return -1;
    void *scratch = partial_scratch();
    if (!scratch) return -1;
    hipStream_t s = as_stream(stream);
    if (layout != LAYOUT_TILED) {
        if (launch_gemv_q(dt, layout, w, M, K, x, logits, s) != 0) return -1;
        return launch_softmax_argmax(logits, M, probs, argmax, standalone_part(scratch), s);
    }
    if (tiled_softmax_scratch_bytes(M) > kFusedBytes) { set_error("too many GEMV workgroups for M=%d", M); return -1; }
    return launch_gemv_tiled_softmax(dt, w, M, K, x, logits, probs, argmax, scratch, s);
}

size_t sapphire_sample_workspace_bytes(int n, int batch) {
    return sample_supported(n, batch) ? sample_workspace_bytes(n, batch) : 0;
}

int sapphire_sample_dev(float *logits, int n, int batch, int ld, float temperature, const float *draws, int *tokens,
                        void *workspace, void *stream) {
    if (!logits || !tokens || !workspace || n <= 0 || batch <= 0 || ld < n ||
        (!(temperature <= 0.0f) && !draws)) {
        set_error("bad sampling arguments");
        return -1;
    }
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) { set_error("the sampling workspace must be 256-byte aligned"); return -1; }
    if (!sample_supported(n, batch)) { set_error("sampling supports 1..2^21 logits per row, n=%d", n); return -1; }
    return launch_sample(logits, n, batch, (size_t)ld, temperature, logits, (size_t)ld, draws, nullptr, tokens,
                         workspace, as_stream(stream));
}

int sapphire_rmsnorm_delta_dev(float *out, const float *in, const float *w, float eps, int dim, int batch, void *s) {
    if (!out || !in || !w || dim <= 0 || batch <= 0 || eps < 0.f) { set_error("bad rmsnorm arguments"); return -1; }
    return launch_rmsnorm(out, in, w, eps, dim, batch, true, as_stream(s));
}

int sapphire_rmsnorm_dev(float *out, const float *in, const float *w, float eps, int dim, int batch, void *s) {
    if (!out || !in || !w || dim <= 0 || batch <= 0 || eps < 0.f) { set_error("bad rmsnorm arguments"); return -1; }
    return launch_rmsnorm(out, in, w, eps, dim, batch, false, as_stream(s));
}

int sapphire_rope_apply_dev(float *x, int n_heads, int head_dim, int pos, const float *c, const float *sn, void *s) {
    if (!x || !c || !sn || n_heads <= 0 || head_dim <= 0 || (head_dim & 1) || pos < 0) {
        set_error("bad rope arguments");
        return -1;
    }
    return launch_rope(x, n_heads, head_dim, pos, c, sn, as_stream(s));
}

int sapphire_gelu_mul_dev(float *gate, const float *up, int n, void *s) {
    if (!gate || !up || n <= 0) { set_error("bad gelu_mul arguments"); return -1; }
    return launch_gelu_mul(gate, up, n, as_stream(s));
}

int sapphire_norm_residual_dev(float *hidden, float *resid, const float *w, float eps, int dim, void *s) {
    if (!hidden || !resid || !w || dim <= 0 || eps < 0.f) { set_error("bad norm_residual arguments"); return -1; }
    return launch_norm_residual(hidden, resid, w, eps, dim, as_stream(s));
}

}  // extern "C"
