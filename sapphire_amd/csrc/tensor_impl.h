// tensor_impl.h - private layout of tensor_t (not installed).
#pragma once

#include <atomic>
#include <mutex>

#include "../../include/tensor.h"
#include "internal.h"

struct tensor_t {
    void *data = nullptr;         // host data (owned unless is_external)
    int ndim = 0;
    int shape[8] = {0};
    tensor_dtype_t dtype = DTYPE_F32;
    memory_layout_t layout = LAYOUT_ROW_MAJOR;
    size_t nbytes = 0;
    int ref_count = 0;
    int is_external = 0;
    // device copy of the weights (created on first GPU use)
    std::mutex dev_mu;
    void *dev = nullptr;
    size_t dev_bytes = 0;
    int dev_layout = 0;           // sapphire::LAYOUT_AOS for F32/BF16, PACKED or TILED for Q4_0/Q8_0
    int dev_device = -1;
    // TILED copy for batched calls when the GEMV copy is PACKED (same device as dev)
    void *dev_tiled = nullptr;
    // set by tensor_set_f32: the host data changed, the device copies are rebuilt on next use
    bool dev_stale = false;
    // unique for the life of the process (never reused, unlike the tensor's address)
    uint64_t serial = 0;
    // advanced whenever the host data may have changed (tensor_set_f32) or the device copies
    // are dropped (sapphire_tensor_invalidate): holders of derived device state compare it
    std::atomic<uint64_t> gen{0};
};

namespace sapphire {
// Device copy of a 2-D weight tensor on the current device (uploaded on first use).
const void *tensor_device_weights(const tensor_t *t, int *layout, hipStream_t s);
// TILED copy of a Q4_0/Q8_0 weight tensor for the batched matrix-core GEMM (K % 128 == 0):
// the GEMV copy when that is TILED, else a second copy made on first use.
const void *tensor_device_tiled(const tensor_t *t, hipStream_t s);
void tensor_drop_device(tensor_t *t);
// Current generation of t (see tensor_t::gen).
inline uint64_t tensor_generation(const tensor_t *t) { return t->gen.load(std::memory_order_acquire); }
// Called by tensor_release before a tensor is freed: drops the device state of an engine
// session whose KV cache held it (transformer.cpp).
void transformer_tensor_released(uint64_t serial);
}  // namespace sapphire
