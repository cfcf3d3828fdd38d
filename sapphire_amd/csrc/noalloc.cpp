// noalloc.cpp - the LM head with its softmax / greedy epilogue for callers that cannot
// allocate device memory (code under HIP graph capture, fixed serving loops, hosts that forbid
// hipMalloc): sapphire_gemv_softmax_noalloc_dev.
//
// sapphire_gemv_softmax_dev keeps its reduction partials in a buffer the library allocates on
// a device's first call. This variant keeps them in `scratch`, a fixed array in the library's
// device code object: every GPU the library runs on holds its own copy, at its own address,
// until the process ends. Host code never passes the array's name to a kernel (on the host
// that name is a stand-in, not a device address): the address is looked up once per device
// with hipGetSymbolAddress and kept.
//
// No contents carry over between calls (each launch writes every partial it reads later), so
// nothing needs clearing. Calls that overlap on one GPU share the array and race: order them
// on one stream.
#include <mutex>

#include "../../include/sapphire_hip.h"
#include "internal.h"

namespace {

// Bytes of partials one call may use: sizeof(partial) * workgroups of the TILED GEMV (at most
// 2 per CU), or 3 * 256 floats for the PACKED / AOS layouts' two-pass softmax.
constexpr size_t kScratchBytes = 64 * 1024;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// This device's address of `scratch`, looked up on the device's first call.
void *scratch_of_current_device() {
    static std::mutex mu;
    static void *addr[kMaxDevices] = {nullptr};
    int dev = 0;
    if (!sapphire::hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= kMaxDevices) {
        sapphire::set_error("device index %d out of range", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> g(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        if (!sapphire::hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
            return nullptr;
        addr[dev] = p;
    }
    return addr[dev];
}

}  // namespace

using namespace sapphire;

extern "C" int sapphire_gemv_softmax_noalloc_dev(int dt, int layout, const void *w, int M, int K, const float *x,
                                                 float *logits, float *probs, int *argmax, void *stream) {
    if (!is_quant(dt) || !w || M <= 0 || K <= 0 || !x || !logits || (!probs && !argmax)) {
        set_error("bad gemv_softmax arguments (dtype %d, w=%p, M=%d, K=%d)", dt, w, M, K);
        return -1;
    }
    if ((reinterpret_cast<uintptr_t>(w) & 3u) != 0) { set_error("weights must be 4-byte aligned"); return -1; }
    if (K % kBlock != 0) { set_error("K=%d is not a multiple of 32", K); return -1; }
    const bool tiled = layout == LAYOUT_TILED;
    if (tiled ? !tiled_supported(dt, M, K) : (layout != LAYOUT_AOS && layout != LAYOUT_PACKED)) {
        set_error("layout %d is not valid for a %d x %d matrix", layout, M, K);
        return -1;
    }
    const size_t need = tiled ? tiled_softmax_scratch_bytes(M) : softmax_scratch_floats(M) * sizeof(float);
    if (need > kScratchBytes) {
        set_error("gemv_softmax_noalloc: %zu bytes of partials exceed the fixed %zu-byte scratch", need, kScratchBytes);
        return -1;
    }
    void *s = scratch_of_current_device();
    if (!s) return -1;
    hipStream_t st = as_stream(stream);
    if (!tiled) {
        if (launch_gemv_q(dt, layout, w, M, K, x, logits, st) != 0) return -1;
        return launch_softmax_argmax(logits, M, probs, argmax, static_cast<float *>(s), st);
    }
    return launch_gemv_tiled_softmax(dt, w, M, K, x, logits, probs, argmax, s, st);
}
