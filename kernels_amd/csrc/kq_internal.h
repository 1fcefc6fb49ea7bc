// kq_internal.h -- host-side launchers shared between the kernel files and the
// C ABI shim (kq_api.cpp). Launchers assume validated arguments.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "kq.h"

namespace kq {

struct Int4Cfg {
    int rows;    // VALU: rows per wave item; MFMA: K parts per workgroup
    int unroll;  // VALU: ring depth; MFMA: ring depth D, or 10 * tiles per wave + D
};

// Compute units of the current device (queried once; 256 if the query fails).
uint32_t cu_count();

// Default launch shape for a problem (tuning table).
Int4Cfg int4_valu_default(uint32_t M, uint32_t K, uint32_t batch);
size_t int4_valu_lds_bytes(uint32_t K, uint32_t batch);
// `batch` tokens on the vector path in batch-1-pass units x 100 (AUTO's crossover).
uint32_t int4_valu_cost(uint32_t M, uint32_t K, uint32_t batch);
// Modelled duration (us) of `batch` tokens on the vector path (AUTO's crossover).
double int4_valu_us(uint32_t M, uint32_t K, uint32_t G, uint32_t batch);

// gsel (device pointer, may be null): the kernel reads the matrix index
// gsel[0] and moves W, S and B by gsel[0] * gstride bytes -- one matrix of a
// pool chosen by an earlier launch, with no host round trip. Gathered calls
// take one token and split bf16 S and B (the MoE expert layout).
hipError_t launch_int4_valu(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg, hipStream_t s,
                            const uint32_t* gsel = nullptr, uint64_t gstride = 0);
bool int4_valu_supported(uint32_t K, uint32_t batch, Int4Cfg cfg);

hipError_t launch_int4_mfma(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg, hipStream_t s);
bool int4_mfma_supported(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg);
Int4Cfg int4_mfma_default(uint32_t M, uint32_t K, uint32_t batch);
// Tokens one matrix-core pass takes (all of them; 0: the shape is not supported).
uint32_t int4_mfma_tokens_per_pass(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg);
// Modelled duration (us) of one matrix-core pass (AUTO's crossover).
double int4_mfma_us(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg);

// Debug scalar path: one thread per (row, token), plain chunk loop (v0).
hipError_t launch_int4_scalar(const uint32_t* W, const uint16_t* S, const uint16_t* B,
                              int meta_kind, bool interleaved, const uint16_t* X, void* Y,
                              bool y_f32, uint32_t M, uint32_t K, uint32_t G, uint32_t batch,
                              hipStream_t s);
hipError_t launch_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch, hipStream_t s);
// unroll 0 and threads 0: the default shape (U = 1, 2048 x 256 threads)
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, uint32_t unroll,
                              uint32_t threads, hipStream_t s, uint16_t* out = nullptr,
                              uint32_t nout = 0);

bool vq_supported(uint32_t M, uint32_t K, uint32_t rows_per_cb);
hipError_t launch_vq(const uint8_t* IDX, const uint16_t* C, const uint16_t* S, const uint16_t* X,
                     void* Y, bool y_f32, uint32_t M, uint32_t K, uint32_t rows_per_cb,
                     uint32_t scale_group, uint32_t batch, hipStream_t s);

// VQ quantiser (kq_vq_quant.hip)
size_t vq_quant_ws_bytes(uint32_t M, uint32_t K, uint32_t scale_group, uint32_t rows_per_cb,
                         uint32_t sample);
uint32_t vq_quant_launches(uint32_t iters);
hipError_t launch_vq_quantize(const void* W, int w_dtype, uint32_t M, uint32_t K,
                              uint32_t rows_per_cb, uint32_t scale_group, uint32_t iters,
                              uint32_t sample, uint64_t seed, uint8_t* IDX, uint16_t* Cb,
                              uint16_t* S, void* ws, hipStream_t s);

// MoE
size_t moe_ws_bytes(const kq_moe_desc& d, uint32_t batch);
hipError_t launch_ws_zero(void* ws, size_t bytes, hipStream_t s);
hipError_t launch_moe_router(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                             const kq_moe_desc& d, uint32_t* idx, float* wgt, uint16_t* xh,
                             void* ws, hipStream_t s);
hipError_t launch_moe_gate_up(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                              const uint16_t* xh, uint16_t* H, uint32_t batch, hipStream_t s);
hipError_t launch_moe_down(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                           const float* wgt, const uint16_t* H, void* Y, bool y_f32,
                           uint32_t batch, hipStream_t s);
// Router logits only (float [batch][n_experts] to lg; xh = half(X) if X is fp32).
hipError_t launch_moe_logits(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                             const kq_moe_desc& d, uint16_t* xh, float* lg, hipStream_t s);
// One operation per launch, batch 1 (see kq_moe_unfused.hip).
size_t moe_unfused_ws_bytes(const kq_moe_desc& d);
uint32_t moe_unfused_launches(const kq_moe_desc& d);
hipError_t launch_moe_unfused(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool r_f32,
                              const void* X, bool x_f32, uint32_t* idx, float* wgt, uint16_t* xh,
                              uint16_t* H, void* Y, bool y_f32, void* ws, hipStream_t s);
// kq_moe_block on the per-device static workspace (no allocation).
hipError_t launch_moe_block_noalloc(const uint8_t* pool, const kq_moe_desc& d, const void* R,
                                    bool r_f32, const void* X, bool x_f32, uint32_t batch,
                                    uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H, void* Y,
                                    bool y_f32, hipStream_t s);
// path: KQ_MOE_PATH_* (KQ_MOE_PATH_ONE only where moe_one_supported holds)
hipError_t launch_moe_block(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool r_f32,
                            const void* X, bool x_f32, uint32_t batch, uint32_t* idx, float* wgt,
                            uint16_t* xh, uint16_t* H, void* Y, bool y_f32, void* ws,
                            hipStream_t s, int path);
// The one-launch block's limits (shape, and every workgroup resident at once).
bool moe_one_supported(const kq_moe_desc& d, uint32_t batch);
// The atomic sum(h) block's limits (the streaming gate/up and down).
bool moe_atomic_supported(const kq_moe_desc& d, uint32_t batch);

}  // namespace kq
