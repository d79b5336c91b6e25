// legacy.cpp — the reference-signature C++ interface (include/kernels/quant.h,
// include/kernels/matvec.h, include/kv_cache.h) on top of the C ABI
// (echo_hip.h).  Each function has the reference's name, arguments and
// "never fails loudly" behaviour (void / float returns); errors go to
// ec_last_error().  Calls run on the null stream and complete before they
// return, so results are host-visible as with the reference's CPU kernels.
//
// Pointer handling: device, managed and pinned host memory are used in place
// (pinned memory through its device alias); ordinary host memory is staged
// through per-thread device buffers that grow on demand and are freed at
// thread exit.
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>

#include "echo_hip.h"
#include "kernels/matvec.h"
#include "kernels/quant.h"
#include "kv_cache.h"

extern "C" int ec_set_error(int code, const char* msg);
extern "C" int ec_set_hip_error(hipError_t e, const char* where);

namespace {

#define LG_HIP(call)                                                    \
    do {                                                                \
        hipError_t _e = (call);                                         \
        if (_e != hipSuccess) return ec_set_hip_error(_e, #call);       \
    } while (0)
#define LG_TRY(call)                  \
    do {                              \
        int _rc = (call);             \
        if (_rc != EC_OK) return _rc; \
    } while (0)

constexpr int kSlots = 4;

struct Staging {
    void* buf[kSlots] = {};
    size_t cap[kSlots] = {};
    ~Staging() {
        for (int i = 0; i < kSlots; ++i)
            if (buf[i]) (void)hipFree(buf[i]);
    }
};
thread_local Staging g_stage;

// A device-usable view of n bytes at p.  staged = true when p is ordinary host
// memory copied (copy_in) into staging slot `slot`.
struct View {
    void* dev = nullptr;
    const void* host = nullptr;
    size_t n = 0;
    bool staged = false;
};

int view(const void* p, size_t n, int slot, bool copy_in, View& v) {
    v = View{};
    v.n = n;
    if (n == 0) return EC_OK;
    if (!p) return ec_set_error(EC_ERR_ARG, "null pointer");
    hipPointerAttribute_t a;
    const hipError_t e = hipPointerGetAttributes(&a, p);
    if (e == hipSuccess && (a.type == hipMemoryTypeDevice || a.type == hipMemoryTypeManaged || a.isManaged)) {
        v.dev = const_cast<void*>(p);
        return EC_OK;
    }
    if (e == hipSuccess && a.type == hipMemoryTypeHost && a.devicePointer) {
        // pinned host memory: the device alias of the same byte
        const char* hbase = (const char*)(a.hostPointer ? a.hostPointer : p);
        v.dev = (char*)a.devicePointer + ((const char*)p - hbase);
        return EC_OK;
    }
    if (e != hipSuccess) (void)hipGetLastError();  // unregistered host memory on older runtimes
    if (g_stage.cap[slot] < n) {
        if (g_stage.buf[slot]) LG_HIP(hipFree(g_stage.buf[slot]));
        g_stage.buf[slot] = nullptr;
        g_stage.cap[slot] = 0;
        LG_HIP(hipMalloc(&g_stage.buf[slot], n));
        g_stage.cap[slot] = n;
    }
    v.dev = g_stage.buf[slot];
    v.host = p;
    v.staged = true;
    if (copy_in) LG_HIP(hipMemcpy(v.dev, p, n, hipMemcpyHostToDevice));
    return EC_OK;
}

// Copy a staged output back to its host buffer (after the kernels are done).
int finish(const View& v) {
    if (v.staged && v.n) LG_HIP(hipMemcpy(const_cast<void*>(v.host), v.dev, v.n, hipMemcpyDeviceToHost));
    return EC_OK;
}

int sync() {
    LG_HIP(hipStreamSynchronize(nullptr));
    return EC_OK;
}

size_t block_bytes(int fmt) { return fmt == EC_Q8_0 ? 34 : (fmt == EC_Q4_K ? 144 : (fmt == EC_Q2_K ? 84 : 2)); }
uint32_t block_elems(int fmt) { return fmt == EC_Q8_0 ? 32 : (fmt == EC_F16 ? 1 : 256); }

// y (M) += W (M x K, GGUF rows of K / block_elems blocks) . x
int matvec_fmt(int fmt, const void* W, const float* x, float* y, uint32_t M, uint32_t K) {
    const uint32_t be = block_elems(fmt);
    const uint32_t Kb = K / be * be;  // the reference drops a partial last block
    if (M == 0 || Kb == 0) return EC_OK;
    View w, xv, yv;
    LG_TRY(view(W, (size_t)M * (Kb / be) * block_bytes(fmt), 0, true, w));
    LG_TRY(view(x, (size_t)Kb * 4, 1, true, xv));
    LG_TRY(view(y, (size_t)M * 4, 2, true, yv));
    LG_TRY(ec_matvec_gguf_f32(fmt, w.dev, (const float*)xv.dev, (float*)yv.dev, M, Kb, nullptr));
    LG_TRY(sync());
    return finish(yv);
}

float dot_fmt(int fmt, const void* blocks, uint32_t n_blocks, const float* q) {
    float y = 0.0f;
    const uint32_t K = n_blocks * block_elems(fmt);
    if (matvec_fmt(fmt, blocks, q, &y, 1, K) != EC_OK) return 0.0f;
    return y;
}

int dequant_fp16(int fmt, const void* src, uint16_t* dst, size_t n) {
    const uint32_t be = block_elems(fmt);
    if (n % be) return ec_set_error(EC_ERR_ARG, "dequantize_*_to_fp16: n_weights must be a multiple of the block");
    if (n == 0) return EC_OK;
    View s, d;
    LG_TRY(view(src, n / be * block_bytes(fmt), 0, true, s));
    LG_TRY(view(dst, n * 2, 1, false, d));
    LG_TRY(ec_dequantize_to_fp16(fmt, s.dev, (uint16_t*)d.dev, n, nullptr));
    LG_TRY(sync());
    return finish(d);
}

}  // namespace

// ----------------------------------------------------------- kernels/quant.h
void quantize_per_token_symmetric(const float* input, int8_t* output, float* scales, uint32_t num_tokens,
                                  uint32_t num_elements) {
    [&]() -> int {
        const size_t n = (size_t)num_tokens * num_elements;
        if (n == 0) return EC_OK;
        View x, q, s;
        LG_TRY(view(input, n * 4, 0, true, x));
        LG_TRY(view(output, n, 1, false, q));
        LG_TRY(view(scales, (size_t)num_tokens * 4, 2, false, s));
        LG_TRY(ec_quantize_rows((const float*)x.dev, (int8_t*)q.dev, (float*)s.dev, num_tokens, num_elements,
                                nullptr));
        LG_TRY(sync());
        LG_TRY(finish(q));
        return finish(s);
    }();
}

void fused_dequant_dot_int8(const float* query, const int8_t* key_cache, const float* scales, float* scores,
                            uint32_t dim, uint32_t seq_len) {
    [&]() -> int {
        if (dim == 0 || seq_len == 0) return EC_OK;
        View q, k, s, o;
        LG_TRY(view(query, (size_t)dim * 4, 0, true, q));
        LG_TRY(view(key_cache, (size_t)dim * seq_len, 1, true, k));
        LG_TRY(view(scales, (size_t)seq_len * 4, 2, true, s));
        LG_TRY(view(scores, (size_t)seq_len * 4, 3, false, o));
        LG_TRY(ec_dequant_dot_int8((const float*)q.dev, (const int8_t*)k.dev, (const float*)s.dev, (float*)o.dev,
                                   dim, seq_len, nullptr));
        LG_TRY(sync());
        return finish(o);
    }();
}

float fused_dequant_dot_q8_0(const block_q8_0* blocks, uint32_t n_blocks, const float* query_fp32) {
    return dot_fmt(EC_Q8_0, blocks, n_blocks, query_fp32);
}

float fused_dequant_dot_q4_K(const block_q4_K* blocks, uint32_t n_blocks, const float* query_fp32) {
    return dot_fmt(EC_Q4_K, blocks, n_blocks, query_fp32);
}

void dequantize_q8_0_to_fp16(const void* src, uint16_t* dst, size_t n_weights) {
    (void)dequant_fp16(EC_Q8_0, src, dst, n_weights);
}
void dequantize_q4_K_to_fp16(const void* src, uint16_t* dst, size_t n_weights) {
    (void)dequant_fp16(EC_Q4_K, src, dst, n_weights);
}
void dequantize_q2_K_to_fp16(const void* src, uint16_t* dst, size_t n_weights) {
    (void)dequant_fp16(EC_Q2_K, src, dst, n_weights);
}

// ---------------------------------------------------------- kernels/matvec.h
template <uint32_t TILE_K, uint32_t TILE_M>
void matvec_fp16_fp32(const fp16_t* W, const float* x, float* y, uint32_t M, uint32_t K) {
    (void)matvec_fmt(EC_F16, W, x, y, M, K);
}
template void matvec_fp16_fp32<1024, 512>(const fp16_t*, const float*, float*, uint32_t, uint32_t);
template void matvec_fp16_fp32<2048, 1024>(const fp16_t*, const float*, float*, uint32_t, uint32_t);

void matvec_dispatch(const fp16_t* W, const float* x, float* y, uint32_t M, uint32_t K, const ModelConfig& config) {
    (void)config;  // the reference picks a CPU tile size from it; one GPU kernel serves all
    (void)matvec_fmt(EC_F16, W, x, y, M, K);
}

void matvec_q8_0(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    (void)matvec_fmt(EC_Q8_0, blocks, x, y, M, K);
}
void matvec_q4_K(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    (void)matvec_fmt(EC_Q4_K, blocks, x, y, M, K);
}
void matvec_q2_K(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    (void)matvec_fmt(EC_Q2_K, blocks, x, y, M, K);
}

// ----------------------------------------------------------------- KVCache
// storage_ holds, per layer, the reference's partition (keys, values, key
// scales, value scales; or fp32 keys, values) and, after all layers, one
// int32 slot for the append position that ec_kv_append reads on the device.
namespace {
size_t kv_layer_bytes(const ModelConfig& c) {
    const size_t rows = (size_t)c.max_seq_len * c.num_kv_heads;
    return c.use_kv_quantization ? 2 * rows * c.head_dim + 2 * rows * sizeof(float)
                                 : 2 * rows * c.head_dim * sizeof(float);
}
}  // namespace

KVCache::KVCache(const ModelConfig& config) : config_(config), layers_(nullptr), storage_(nullptr) {
    const uint32_t L = config_.num_layers;
    layers_ = new (std::nothrow) KVCacheLayer[L ? L : 1];
    if (!layers_) {
        ec_set_error(EC_ERR_ARG, "KVCache: host allocation failed");
        return;
    }
    std::memset((void*)layers_, 0, sizeof(KVCacheLayer) * (L ? L : 1));
    if (config_.max_seq_len == 0 || L == 0) return;
    const size_t per = (kv_layer_bytes(config_) + 255) & ~(size_t)255;
    const size_t total = per * L + 256;
    if (hipMalloc((void**)&storage_, total) != hipSuccess) {
        ec_set_error(EC_ERR_HIP, "KVCache: hipMalloc failed");
        storage_ = nullptr;
        return;
    }
    (void)hipMemset(storage_, 0, total);
    const size_t rows = (size_t)config_.max_seq_len * config_.num_kv_heads;
    for (uint32_t l = 0; l < L; ++l) {
        uint8_t* p = storage_ + per * l;
        KVCacheLayer& y = layers_[l];
        if (config_.use_kv_quantization) {
            y.keys_int8 = (int8_t*)p;
            y.values_int8 = (int8_t*)(p + rows * config_.head_dim);
            y.key_scales = (float*)(p + 2 * rows * config_.head_dim);
            y.val_scales = y.key_scales + rows;
        } else {
            y.keys_fp32 = (float*)p;
            y.values_fp32 = y.keys_fp32 + rows * config_.head_dim;
        }
        y.seq_len = 0;
    }
}

KVCache::~KVCache() {
    if (storage_) (void)hipFree(storage_);
    delete[] layers_;
}

KVCacheLayer& KVCache::layer(uint32_t layer_idx) {
    if (layer_idx >= config_.num_layers) ec_set_error(EC_ERR_ARG, "KVCache::layer: index out of range");
    return layers_[layer_idx < config_.num_layers ? layer_idx : 0];
}

const KVCacheLayer& KVCache::layer(uint32_t layer_idx) const {
    if (layer_idx >= config_.num_layers) ec_set_error(EC_ERR_ARG, "KVCache::layer: index out of range");
    return layers_[layer_idx < config_.num_layers ? layer_idx : 0];
}

void KVCache::append(uint32_t layer_idx, const float* k_proj, const float* v_proj) {
    [&]() -> int {
        if (!storage_) return ec_set_error(EC_ERR_ARG, "KVCache::append: cache has no storage");
        if (layer_idx >= config_.num_layers) return ec_set_error(EC_ERR_ARG, "KVCache::append: layer out of range");
        KVCacheLayer& y = layers_[layer_idx];
        if (y.seq_len >= config_.max_seq_len) return ec_set_error(EC_ERR_ARG, "KVCache::append: cache is full");
        const size_t row = (size_t)config_.num_kv_heads * config_.head_dim;
        View k, v;
        LG_TRY(view(k_proj, row * 4, 0, true, k));
        LG_TRY(view(v_proj, row * 4, 1, true, v));
        const int32_t pos = (int32_t)y.seq_len;
        if (config_.use_kv_quantization) {
            const size_t per = (kv_layer_bytes(config_) + 255) & ~(size_t)255;
            int32_t* dpos = (int32_t*)(storage_ + per * config_.num_layers);
            LG_HIP(hipMemcpy(dpos, &pos, sizeof(pos), hipMemcpyHostToDevice));
            LG_TRY(ec_kv_append((const float*)k.dev, (const float*)v.dev, y.keys_int8, y.values_int8, y.key_scales,
                                y.val_scales, dpos, 1, (uint64_t)config_.max_seq_len * row, config_.num_kv_heads,
                                config_.head_dim, nullptr));
        } else {
            LG_HIP(hipMemcpyAsync(y.keys_fp32 + pos * row, k.dev, row * 4, hipMemcpyDeviceToDevice, nullptr));
            LG_HIP(hipMemcpyAsync(y.values_fp32 + pos * row, v.dev, row * 4, hipMemcpyDeviceToDevice, nullptr));
        }
        LG_TRY(sync());
        y.seq_len++;
        return EC_OK;
    }();
}

uint32_t KVCache::seq_len() const { return config_.num_layers ? layers_[0].seq_len : 0; }

void KVCache::reset() {
    for (uint32_t l = 0; l < config_.num_layers; ++l) layers_[l].seq_len = 0;
}
