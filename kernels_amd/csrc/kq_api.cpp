// kq_api.cpp -- the extern "C" boundary of libkq (declared in include/kq.h).
//
// Validation happens here, on the host, before anything is enqueued: a
// malformed shape becomes KQ_EINVAL, never an out-of-bounds kernel. Launch
// failures become KQ_EHIP with the HIP code kept per host thread. Nothing
// here allocates, prints or exits (the reference harness's die() -> exit(1),
// int4-gemv/src/main.mm:38-42, is the caller's business now), and nothing
// synchronises except kq_moe_workspace_error, a read-back query.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstring>

#include "kq.h"
#include "kq_internal.h"

namespace {

thread_local int g_last_hip = 0;

kq_status hip_status(hipError_t e) {
    if (e == hipSuccess) return KQ_OK;
    g_last_hip = (int)e;
    return KQ_EHIP;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool pow2(uint32_t v) { return v && !(v & (v - 1)); }

kq_status check_int4(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                     const uint16_t* X, void* Y, kq_dtype y_dtype, uint32_t M, uint32_t K,
                     uint32_t G, uint32_t batch) {
    if (!W || !S || !X || !Y) return KQ_ENULL;
    if (M == 0 || K == 0 || batch == 0 || batch > 16) return KQ_EINVAL;
    if (K % 32 != 0) return KQ_EINVAL;
    if (!(G == 32 || G == 64 || G == 128) || K % G != 0) return KQ_EINVAL;
    if ((uint64_t)M * (K / 8) > 0xFFFFFFFFull * 4) return KQ_EINVAL;
    if (!(sb_dtype == KQ_F16 || sb_dtype == KQ_BF16)) return KQ_EUNSUPPORTED;
    if (!(y_dtype == KQ_F16 || y_dtype == KQ_F32)) return KQ_EUNSUPPORTED;
    if (!aligned(W, 16) || !aligned(X, 16)) return KQ_EALIGN;
    if (B == nullptr ? !aligned(S, 4) : (!aligned(S, 2) || !aligned(B, 2))) return KQ_EALIGN;
    if (!aligned(Y, y_dtype == KQ_F32 ? 4 : 2)) return KQ_EALIGN;
    return KQ_OK;
}

kq_status run_int4(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                   const uint16_t* X, void* Y, kq_dtype y_dtype, uint32_t M, uint32_t K,
                   uint32_t G, uint32_t batch, kq_int4_path path, const kq::Int4Cfg* forced,
                   kq_stream_t stream) {
    kq_status st = check_int4(W, S, B, sb_dtype, X, Y, y_dtype, M, K, G, batch);
    if (st != KQ_OK) return st;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int mk = sb_dtype == KQ_BF16 ? 1 : 0;
    const bool inter = B == nullptr;
    const auto* Sp = static_cast<const uint16_t*>(S);
    const auto* Bp = static_cast<const uint16_t*>(B);
    const bool yf = y_dtype == KQ_F32;

    kq::Int4Cfg vcfg = forced ? *forced : kq::int4_valu_default(M, K, batch);
    kq::Int4Cfg mcfg = forced ? *forced : kq::int4_mfma_default(M, K, batch);
    const bool valu_ok = kq::int4_valu_supported(K, batch, vcfg);
    // the matrix-core path reads a span's separate scales / biases as one
    // 4- or 8-byte word each
    const bool meta_aligned = inter || (aligned(S, 8) && aligned(B, 8));
    const bool mfma_ok = meta_aligned && kq::int4_mfma_supported(M, K, G, batch, mcfg);
    // Crossover, in batch-1 vector passes: a vector pass takes up to 4 tokens
    // (int4_valu_cost), a matrix-core pass all of them at ~1.2 (29.3-30.3 us
    // against 24.9 us at 28672 x 8192; 64-byte row pieces per load instead of
    // 1 KiB rows). Measured: the vector path wins at 1-2 tokens, the matrix
    // cores from 3 -- where the weights are large. A matrix-core pass takes
    // at least ~9 us (each wave's serial steps), so small matrices stay on the
    // vector path longer: both durations are modelled too (1024x4096: vector
    // up to 8 tokens, 4.1-9.1 against 9.2-9.9 us; 4096x4096 up to 4).
    if (path == KQ_PATH_AUTO) {
        if (!mfma_ok) {
            path = KQ_PATH_VALU;
        } else if (!valu_ok) {
            path = KQ_PATH_MFMA;
        } else {
            const uint32_t tpp = kq::int4_mfma_tokens_per_pass(M, K, G, batch, mcfg);
            const uint32_t mp = tpp ? (batch + tpp - 1) / tpp : 1000;
            const bool fewer_passes = 120 * mp < kq::int4_valu_cost(M, K, batch);
            const bool faster = mp * kq::int4_mfma_us(M, K, G, batch, mcfg) < kq::int4_valu_us(M, K, G, batch);
            path = fewer_passes && faster ? KQ_PATH_MFMA : KQ_PATH_VALU;
        }
    }
    if (path == KQ_PATH_VALU) {
        if (!valu_ok) return KQ_EUNSUPPORTED;
        return hip_status(kq::launch_int4_valu(W, Sp, Bp, mk, inter, X, Y, yf, M, K, G, batch, vcfg, s));
    }
    if (path == KQ_PATH_MFMA) {
        if (!mfma_ok) return KQ_EUNSUPPORTED;
        return hip_status(kq::launch_int4_mfma(W, Sp, Bp, mk, inter, X, Y, yf, M, K, G, batch, mcfg, s));
    }
    if (path == KQ_PATH_SCALAR)
        return hip_status(kq::launch_int4_scalar(W, Sp, Bp, mk, inter, X, Y, yf, M, K, G, batch, s));
    return KQ_EINVAL;
}

kq_status check_desc(const kq_moe_desc* d, uint32_t batch) {
    if (!d) return KQ_ENULL;
    if (batch == 0 || batch > 16) return KQ_EINVAL;
    if (d->n_experts == 0 || d->n_experts > 256) return KQ_EINVAL;
    if (d->top_k == 0 || d->top_k > 8 || d->top_k > d->n_experts) return KQ_EINVAL;
    if (d->hidden == 0 || d->inter == 0 || d->hidden % 64 || d->inter % 64) return KQ_EINVAL;
    if (d->hidden > 4096 || d->inter > 4096) return KQ_EUNSUPPORTED;
    // every sub-tensor of every projection must fit in the blob
    const uint64_t rows_gu = d->inter, cols_gu = d->hidden, rows_dn = d->hidden, cols_dn = d->inter;
    auto proj_ok = [&](uint64_t off, uint64_t rows, uint64_t cols) {
        const uint64_t wb = rows * cols / 2, sb = rows * (cols / 64) * 2, bib = rows * 2;
        return off + d->sub_w + wb <= d->blob && off + d->sub_s + sb <= d->blob &&
               off + d->sub_b + sb <= d->blob && off + d->sub_bi + bib <= d->blob &&
               (off + d->sub_w) % 16 == 0 && (off + d->sub_s) % 2 == 0 &&
               (off + d->sub_b) % 2 == 0 && (off + d->sub_bi) % 2 == 0;
    };
    if (!proj_ok(d->off_gate, rows_gu, cols_gu) || !proj_ok(d->off_up, rows_gu, cols_gu) ||
        !proj_ok(d->off_down, rows_dn, cols_dn))
        return KQ_EINVAL;
    if (d->blob % 16 != 0) return KQ_EALIGN;
    return KQ_OK;
}

kq_status check_ws(const kq_moe_desc* d, uint32_t batch, const void* ws, size_t ws_bytes) {
    if (!ws) return KQ_EWORKSPACE;
    if (ws_bytes < kq::moe_ws_bytes(*d, batch)) return KQ_EWORKSPACE;
    if (!aligned(ws, 256)) return KQ_EALIGN;
    return KQ_OK;
}

}  // namespace

namespace kq {
// One cached count per device index: every planner sizes its grid for the
// device that is current on the calling thread. The cache words are atomics,
// so threads that query the same device for the first time at once only
// store the same value twice.
uint32_t cu_count() {
    constexpr int kDevs = 64;
    static std::atomic<int> per_dev[kDevs];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::atomic<int>* slot = dev >= 0 && dev < kDevs ? &per_dev[dev] : nullptr;
    int n = slot ? slot->load(std::memory_order_relaxed) : 0;
    if (n > 0) return (uint32_t)n;
    int v = 0;
    n = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0 ? v
                                                                                                   : 256;
    if (slot) slot->store(n, std::memory_order_relaxed);
    return (uint32_t)n;
}
}  // namespace kq

extern "C" {

const char* kq_status_str(kq_status s) {
    switch (s) {
        case KQ_OK: return "ok";
        case KQ_EINVAL: return "invalid argument (shape or format contract)";
        case KQ_ENULL: return "null pointer";
        case KQ_EALIGN: return "misaligned pointer";
        case KQ_EUNSUPPORTED: return "unsupported configuration";
        case KQ_EWORKSPACE: return "workspace missing or too small";
        case KQ_EHIP: return "HIP launch error";
    }
    return "unknown status";
}

int kq_last_hip_error(void) { return g_last_hip; }

const char* kq_version(void) { return "kq 0.1 gfx950"; }

kq_status kq_int4_gemv(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                       const uint16_t* X, void* Y, kq_dtype y_dtype, uint32_t M, uint32_t K,
                       uint32_t G, uint32_t batch, kq_stream_t stream) {
    return run_int4(W, S, B, sb_dtype, X, Y, y_dtype, M, K, G, batch, KQ_PATH_AUTO, nullptr, stream);
}

kq_status kq_int4_gemv_path(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                            const uint16_t* X, void* Y, kq_dtype y_dtype, uint32_t M, uint32_t K,
                            uint32_t G, uint32_t batch, kq_int4_path path, kq_stream_t stream) {
    if (!(path == KQ_PATH_AUTO || path == KQ_PATH_VALU || path == KQ_PATH_MFMA ||
          path == KQ_PATH_SCALAR))
        return KQ_EINVAL;
    return run_int4(W, S, B, sb_dtype, X, Y, y_dtype, M, K, G, batch, path, nullptr, stream);
}

kq_status kq_int4_gemv_cfg(const uint32_t* W, const void* S, const void* B, kq_dtype sb_dtype,
                           const uint16_t* X, void* Y, kq_dtype y_dtype, uint32_t M, uint32_t K,
                           uint32_t G, uint32_t batch, kq_int4_path path, int rows, int unroll,
                           kq_stream_t stream) {
    if (!(path == KQ_PATH_VALU || path == KQ_PATH_MFMA)) return KQ_EINVAL;
    const kq::Int4Cfg cfg{rows, unroll};
    return run_int4(W, S, B, sb_dtype, X, Y, y_dtype, M, K, G, batch, path, &cfg, stream);
}

kq_status kq_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch, kq_stream_t stream) {
    if (!X || !xs) return KQ_ENULL;
    if (K == 0 || K % 32 || batch == 0) return KQ_EINVAL;
    if (!aligned(X, 16) || !aligned(xs, 4)) return KQ_EALIGN;
    return hip_status(kq::launch_xsum32(X, xs, K, batch, reinterpret_cast<hipStream_t>(stream)));
}

kq_status kq_stream_read(const void* src, size_t bytes, uint32_t* sink, kq_stream_t stream) {
    if (!src || !sink) return KQ_ENULL;
    if (bytes == 0 || bytes % 16) return KQ_EINVAL;
    if (!aligned(src, 16)) return KQ_EALIGN;
    return hip_status(
        kq::launch_stream_read(src, bytes, sink, 0, 0, reinterpret_cast<hipStream_t>(stream)));
}

kq_status kq_stream_read_cfg(const void* src, size_t bytes, uint32_t* sink, uint32_t unroll,
                             uint32_t threads, kq_stream_t stream) {
    if (!src || !sink) return KQ_ENULL;
    if (bytes == 0 || bytes % 16) return KQ_EINVAL;
    if (!(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8)) return KQ_EINVAL;
    if (threads == 0 || threads % 256 || threads > (1u << 30)) return KQ_EINVAL;
    if (!aligned(src, 16)) return KQ_EALIGN;
    return hip_status(kq::launch_stream_read(src, bytes, sink, unroll, threads,
                                             reinterpret_cast<hipStream_t>(stream)));
}

kq_status kq_stream_read_out(const void* src, size_t bytes, uint16_t* out, uint32_t out_elems,
                             uint32_t unroll, uint32_t threads, kq_stream_t stream) {
    if (!src || !out) return KQ_ENULL;
    if (bytes == 0 || bytes % 16 || out_elems == 0) return KQ_EINVAL;
    if (!(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8)) return KQ_EINVAL;
    if (threads == 0 || threads % 256 || threads > (1u << 30)) return KQ_EINVAL;
    if (!aligned(src, 16) || !aligned(out, 2)) return KQ_EALIGN;
    return hip_status(kq::launch_stream_read(src, bytes, nullptr, unroll, threads,
                                             reinterpret_cast<hipStream_t>(stream), out, out_elems));
}

kq_status kq_vq_gemv(const uint8_t* IDX, const uint16_t* C, const uint16_t* S, const uint16_t* X,
                     void* Y, kq_dtype y_dtype, uint32_t M, uint32_t K, uint32_t rows_per_cb,
                     uint32_t scale_group, uint32_t batch, kq_stream_t stream) {
    if (!IDX || !C || !S || !X || !Y) return KQ_ENULL;
    if (M == 0 || K == 0 || K % 32 || batch == 0 || batch > 16 || rows_per_cb == 0)
        return KQ_EINVAL;
    if (scale_group != K && (!pow2(scale_group) || scale_group < 32 || K % scale_group))
        return KQ_EINVAL;
    if (!(y_dtype == KQ_F16 || y_dtype == KQ_F32)) return KQ_EUNSUPPORTED;
    if (!kq::vq_supported(M, K, rows_per_cb)) return KQ_EUNSUPPORTED;  // x must fit LDS
    if (!aligned(IDX, 16) || !aligned(X, 16) || !aligned(C, 4) || !aligned(S, 2)) return KQ_EALIGN;
    if (!aligned(Y, y_dtype == KQ_F32 ? 4 : 2)) return KQ_EALIGN;
    return hip_status(kq::launch_vq(IDX, C, S, X, Y, y_dtype == KQ_F32, M, K, rows_per_cb,
                                    scale_group, batch, reinterpret_cast<hipStream_t>(stream)));
}

void kq_moe_default_desc(kq_moe_desc* d) {
    if (!d) return;
    // gpt-oss-120b as repacked by moe-stream (moe-fused/src/main.mm:23-25,76)
    d->hidden = 2880;
    d->inter = 2880;
    d->n_experts = 128;
    d->top_k = 4;
    d->blob = 14024704;
    d->off_gate = 0;
    d->off_up = 4671360;
    d->off_down = 9342720;
    d->sub_w = 0;
    d->sub_s = 4147200;
    d->sub_b = 4406400;
    d->sub_bi = 4665600;
}

size_t kq_moe_workspace_size(const kq_moe_desc* d, uint32_t batch) {
    if (check_desc(d, batch) != KQ_OK) return 0;
    return kq::moe_ws_bytes(*d, batch);
}

kq_status kq_moe_workspace_init(void* ws, size_t bytes, kq_stream_t stream) {
    if (!ws) return KQ_ENULL;
    if (!aligned(ws, 256)) return KQ_EALIGN;
    return hip_status(kq::launch_ws_zero(ws, bytes, reinterpret_cast<hipStream_t>(stream)));
}

// The one entry point that waits for the GPU: the word is read back after
// the stream's earlier work.
kq_status kq_moe_workspace_error(void* ws, size_t ws_bytes, uint32_t* err, int clear,
                                 kq_stream_t stream) {
    if (!ws || !err) return KQ_ENULL;
    if (!aligned(ws, 256)) return KQ_EALIGN;
    if (ws_bytes < 256) return KQ_EWORKSPACE;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    uint8_t* word = reinterpret_cast<uint8_t*>(ws) + KQ_MOE_WS_ERR_OFFSET;
    uint32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, word, sizeof v, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess && clear && v != 0) {
        e = kq::launch_ws_zero(word, sizeof v, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
    if (e != hipSuccess) return hip_status(e);
    *err = v;
    return KQ_OK;
}

kq_status kq_moe_router_topk(const void* R, kq_dtype r_dtype, const void* X, kq_dtype x_dtype,
                             uint32_t batch, const kq_moe_desc* d, uint32_t* idx, float* wgt,
                             uint16_t* xh, void* ws, size_t ws_bytes, kq_stream_t stream) {
    kq_status st = check_desc(d, batch);
    if (st != KQ_OK) return st;
    if (!R || !X || !idx || !wgt) return KQ_ENULL;
    if (!(r_dtype == KQ_F16 || r_dtype == KQ_F32) || !(x_dtype == KQ_F16 || x_dtype == KQ_F32))
        return KQ_EUNSUPPORTED;
    if (d->hidden % 8) return KQ_EINVAL;
    if (!aligned(R, 16) || !aligned(X, 16) || !aligned(idx, 4) || !aligned(wgt, 4)) return KQ_EALIGN;
    if (xh && !aligned(xh, 2)) return KQ_EALIGN;
    if ((st = check_ws(d, batch, ws, ws_bytes)) != KQ_OK) return st;
    return hip_status(kq::launch_moe_router(R, r_dtype == KQ_F32, X, x_dtype == KQ_F32, batch, *d,
                                            idx, wgt, xh, ws,
                                            reinterpret_cast<hipStream_t>(stream)));
}

kq_status kq_moe_gate_up_swiglu(const uint8_t* pool, const kq_moe_desc* d, const uint32_t* idx,
                                const uint16_t* xh, uint16_t* H, uint32_t batch, void* ws,
                                size_t ws_bytes, kq_stream_t stream) {
    kq_status st = check_desc(d, batch);
    if (st != KQ_OK) return st;
    if (!pool || !idx || !xh || !H) return KQ_ENULL;
    if (!aligned(pool, 16) || !aligned(xh, 16) || !aligned(H, 2) || !aligned(idx, 4))
        return KQ_EALIGN;
    (void)ws;  // this pass keeps everything on chip
    (void)ws_bytes;
    return hip_status(kq::launch_moe_gate_up(pool, *d, idx, xh, H, batch,
                                             reinterpret_cast<hipStream_t>(stream)));
}

kq_status kq_moe_down_combine(const uint8_t* pool, const kq_moe_desc* d, const uint32_t* idx,
                              const float* wgt, const uint16_t* H, void* Y, kq_dtype y_dtype,
                              uint32_t batch, void* ws, size_t ws_bytes, kq_stream_t stream) {
    kq_status st = check_desc(d, batch);
    if (st != KQ_OK) return st;
    if (!pool || !idx || !wgt || !H || !Y) return KQ_ENULL;
    if (!(y_dtype == KQ_F16 || y_dtype == KQ_F32)) return KQ_EUNSUPPORTED;
    if (!aligned(pool, 16) || !aligned(H, 16) || !aligned(idx, 4) || !aligned(wgt, 4))
        return KQ_EALIGN;
    if (!aligned(Y, y_dtype == KQ_F32 ? 4 : 2)) return KQ_EALIGN;
    (void)ws;  // the combine happens in LDS
    (void)ws_bytes;
    return hip_status(kq::launch_moe_down(pool, *d, idx, wgt, H, Y, y_dtype == KQ_F32, batch,
                                          reinterpret_cast<hipStream_t>(stream)));
}

namespace {
// Arguments of the block (everything but the workspace).
kq_status check_block(const uint8_t* pool, const kq_moe_desc* d, const void* R, kq_dtype r_dtype,
                      const void* X, kq_dtype x_dtype, uint32_t batch, uint32_t* idx, float* wgt,
                      uint16_t* xh, uint16_t* H, void* Y, kq_dtype y_dtype) {
    kq_status st = check_desc(d, batch);
    if (st != KQ_OK) return st;
    if (!pool || !R || !X || !idx || !wgt || !H || !Y) return KQ_ENULL;
    if (x_dtype == KQ_F32 && !xh) return KQ_ENULL;
    if (!(r_dtype == KQ_F16 || r_dtype == KQ_F32) || !(x_dtype == KQ_F16 || x_dtype == KQ_F32))
        return KQ_EUNSUPPORTED;
    if (!(y_dtype == KQ_F16 || y_dtype == KQ_F32)) return KQ_EUNSUPPORTED;
    if (d->hidden % 8) return KQ_EINVAL;
    if (!aligned(pool, 16) || !aligned(R, 16) || !aligned(X, 16) || !aligned(idx, 4) ||
        !aligned(wgt, 4) || !aligned(H, 16))
        return KQ_EALIGN;
    if (xh && !aligned(xh, 16)) return KQ_EALIGN;
    if (!aligned(Y, y_dtype == KQ_F32 ? 4 : 2)) return KQ_EALIGN;
    return KQ_OK;
}
}  // namespace

kq_status kq_moe_block_path(const uint8_t* pool, const kq_moe_desc* d, const void* R,
                            kq_dtype r_dtype, const void* X, kq_dtype x_dtype, uint32_t batch,
                            uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H, void* Y,
                            kq_dtype y_dtype, void* ws, size_t ws_bytes, int path,
                            kq_stream_t stream) {
    kq_status st = check_block(pool, d, R, r_dtype, X, x_dtype, batch, idx, wgt, xh, H, Y, y_dtype);
    if (st != KQ_OK) return st;
    if ((st = check_ws(d, batch, ws, ws_bytes)) != KQ_OK) return st;
    if (path != KQ_MOE_PATH_AUTO && path != KQ_MOE_PATH_LAUNCHES && path != KQ_MOE_PATH_ONE &&
        path != KQ_MOE_PATH_ATOMIC)
        return KQ_EINVAL;
    if (path == KQ_MOE_PATH_ONE &&
        !kq::moe_one_supported(*d, batch))
        return KQ_EUNSUPPORTED;
    if (path == KQ_MOE_PATH_ATOMIC && !kq::moe_atomic_supported(*d, batch)) return KQ_EUNSUPPORTED;
    return hip_status(kq::launch_moe_block(pool, *d, R, r_dtype == KQ_F32, X, x_dtype == KQ_F32,
                                           batch, idx, wgt, xh, H, Y, y_dtype == KQ_F32, ws,
                                           reinterpret_cast<hipStream_t>(stream), path));
}

kq_status kq_moe_block(const uint8_t* pool, const kq_moe_desc* d, const void* R, kq_dtype r_dtype,
                       const void* X, kq_dtype x_dtype, uint32_t batch, uint32_t* idx, float* wgt,
                       uint16_t* xh, uint16_t* H, void* Y, kq_dtype y_dtype, void* ws,
                       size_t ws_bytes, kq_stream_t stream) {
    return kq_moe_block_path(pool, d, R, r_dtype, X, x_dtype, batch, idx, wgt, xh, H, Y, y_dtype,
                             ws, ws_bytes, KQ_MOE_PATH_AUTO, stream);
}

kq_status kq_moe_block_noalloc(const uint8_t* pool, const kq_moe_desc* d, const void* R,
                               kq_dtype r_dtype, const void* X, kq_dtype x_dtype, uint32_t batch,
                               uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H, void* Y,
                               kq_dtype y_dtype, kq_stream_t stream) {
    kq_status st = check_block(pool, d, R, r_dtype, X, x_dtype, batch, idx, wgt, xh, H, Y, y_dtype);
    if (st != KQ_OK) return st;
    if (kq::moe_ws_bytes(*d, batch) > KQ_MOE_NOALLOC_WS_BYTES) return KQ_EWORKSPACE;
    return hip_status(kq::launch_moe_block_noalloc(pool, *d, R, r_dtype == KQ_F32, X,
                                                   x_dtype == KQ_F32, batch, idx, wgt, xh, H, Y,
                                                   y_dtype == KQ_F32,
                                                   reinterpret_cast<hipStream_t>(stream)));
}

size_t kq_moe_unfused_workspace_size(const kq_moe_desc* d) {
    if (check_desc(d, 1) != KQ_OK) return 0;
    return kq::moe_unfused_ws_bytes(*d);
}

namespace {
kq_status check_vq_quant(uint32_t M, uint32_t K, uint32_t rows_per_cb, uint32_t scale_group,
                         uint32_t sample) {
    if (M == 0 || K == 0 || K % 32 || rows_per_cb == 0) return KQ_EINVAL;
    if (K > (1u << 18)) return KQ_EUNSUPPORTED;  // chunk maxima of a row are staged in LDS
    if (!(scale_group == K || (scale_group >= 32 && (scale_group & (scale_group - 1)) == 0 &&
                               K % scale_group == 0)))
        return KQ_EINVAL;
    if (sample == 0 || sample > (1u << 24)) return KQ_EINVAL;
    const uint64_t rows = rows_per_cb < M ? rows_per_cb : M;
    if (rows * (K / 2) >= (1ull << 32)) return KQ_EUNSUPPORTED;  // pair indices are 32-bit
    if ((M + (uint64_t)rows_per_cb - 1) / rows_per_cb > 65535) return KQ_EUNSUPPORTED;
    return KQ_OK;
}
}  // namespace

size_t kq_vq_quantize_workspace_size(uint32_t M, uint32_t K, uint32_t rows_per_cb,
                                     uint32_t scale_group, uint32_t sample) {
    if (check_vq_quant(M, K, rows_per_cb, scale_group, sample) != KQ_OK) return 0;
    return kq::vq_quant_ws_bytes(M, K, scale_group, rows_per_cb, sample);
}

kq_status kq_vq_quantize(const void* W, kq_dtype w_dtype, uint32_t M, uint32_t K,
                         uint32_t rows_per_cb, uint32_t scale_group, uint32_t iters,
                         uint32_t sample, uint64_t seed, uint8_t* IDX, uint16_t* C, uint16_t* S,
                         void* ws, size_t ws_bytes, kq_stream_t stream) {
    kq_status st = check_vq_quant(M, K, rows_per_cb, scale_group, sample);
    if (st != KQ_OK) return st;
    if (iters > 1000) return KQ_EINVAL;
    if (!(w_dtype == KQ_F32 || w_dtype == KQ_F16 || w_dtype == KQ_BF16)) return KQ_EUNSUPPORTED;
    if (!W || !IDX || !C || !S) return KQ_ENULL;
    if (!ws || ws_bytes < kq::vq_quant_ws_bytes(M, K, scale_group, rows_per_cb, sample))
        return KQ_EWORKSPACE;
    if (!aligned(W, w_dtype == KQ_F32 ? 4 : 2) || !aligned(IDX, 4) || !aligned(C, 2) ||
        !aligned(S, 2) || !aligned(ws, 256))
        return KQ_EALIGN;
    return hip_status(kq::launch_vq_quantize(W, (int)w_dtype, M, K, rows_per_cb, scale_group,
                                             iters, sample, seed, IDX, C, S, ws,
                                             reinterpret_cast<hipStream_t>(stream)));
}

kq_status kq_moe_block_unfused(const uint8_t* pool, const kq_moe_desc* d, const void* R,
                               kq_dtype r_dtype, const void* X, kq_dtype x_dtype, uint32_t batch,
                               uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H, void* Y,
                               kq_dtype y_dtype, void* ws, size_t ws_bytes, uint32_t* n_launches,
                               kq_stream_t stream) {
    kq_status st = check_desc(d, batch);
    if (st != KQ_OK) return st;
    if (batch != 1) return KQ_EUNSUPPORTED;
    if (!pool || !R || !X || !idx || !wgt || !H || !Y) return KQ_ENULL;
    if (x_dtype == KQ_F32 && !xh) return KQ_ENULL;
    if (!(r_dtype == KQ_F16 || r_dtype == KQ_F32) || !(x_dtype == KQ_F16 || x_dtype == KQ_F32))
        return KQ_EUNSUPPORTED;
    if (!(y_dtype == KQ_F16 || y_dtype == KQ_F32)) return KQ_EUNSUPPORTED;
    if (!aligned(pool, 16) || !aligned(R, 16) || !aligned(X, 16) || !aligned(idx, 4) ||
        !aligned(wgt, 4) || !aligned(H, 16))
        return KQ_EALIGN;
    if (xh && !aligned(xh, 16)) return KQ_EALIGN;
    if (!aligned(Y, y_dtype == KQ_F32 ? 4 : 2)) return KQ_EALIGN;
    if (!ws || ws_bytes < kq::moe_unfused_ws_bytes(*d)) return KQ_EWORKSPACE;
    if (!aligned(ws, 256)) return KQ_EALIGN;
    if (!kq::int4_valu_supported(d->hidden, 1, kq::Int4Cfg{0, 0}) ||
        !kq::int4_valu_supported(d->inter, 1, kq::Int4Cfg{0, 0}))
        return KQ_EUNSUPPORTED;
    st = hip_status(kq::launch_moe_unfused(pool, *d, R, r_dtype == KQ_F32, X, x_dtype == KQ_F32,
                                           idx, wgt, xh, H, Y, y_dtype == KQ_F32, ws,
                                           reinterpret_cast<hipStream_t>(stream)));
    if (n_launches) *n_launches = st == KQ_OK ? kq::moe_unfused_launches(*d) : 0;
    return st;
}

}  // extern "C"
