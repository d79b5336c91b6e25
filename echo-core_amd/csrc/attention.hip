// attention.hip — INT8 KV-cache append and split-K decode attention (gfx950).
//
// Cache layout per sequence (the reference's, include/kv_cache.h:7-19):
// keys/vals int8 [max_ctx][n_kv][head_dim], kscales/vscales fp32 [max_ctx][n_kv],
// one scale per (token, kv_head) row as the readers index it
// (src/inference.cpp:347,387; echo-core-zig/src/inference/engine.zig:580,601).
//
// Decode attention (engine.zig:563-616): for q head h, kv head h % n_kv,
//   s_p = (q . K_p) * ks_p / sqrt(head_dim),  a = softmax(s),  o = sum_p a_p V_p vs_p.
// Split-K over the context ("flash decoding"): a wave owns one kv head and a
// chunk of the context, serves all n_heads/n_kv query heads that share that kv
// head (each K/V byte is read once for the whole GQA group), keeps a running
// max / sum / output per head (online softmax) and writes one partial per
// chunk; a second kernel merges the partials.
#include "common.hpp"

namespace ec {

constexpr uint32_t kAttnChunk = 256;  // context positions per workgroup

// ------------------------------------------------------------------ append
// grid (n_kv, n_seq, 2): one wave quantizes one (token, kv_head) row of K or V
// with the reference quantizer (src/kernels/quant.cpp:18-98).
__global__ __launch_bounds__(64) void k_kv_append(const float* __restrict__ k, const float* __restrict__ v,
                                                  int8_t* __restrict__ keys, int8_t* __restrict__ vals,
                                                  float* __restrict__ kscales, float* __restrict__ vscales,
                                                  const int32_t* __restrict__ pos, uint64_t seq_stride, uint32_t n_kv,
                                                  uint32_t hd) {
    const uint32_t kvh = blockIdx.x, s = blockIdx.y, which = blockIdx.z, lane = threadIdx.x;
    const int32_t p = pos[s];
    if (p < 0 || (uint64_t)p >= seq_stride / ((uint64_t)n_kv * hd)) return;  // outside the sequence's cache
    const float* src = (which == 0 ? k : v) + ((size_t)s * n_kv + kvh) * hd;
    int8_t* dst = (which == 0 ? keys : vals) + s * seq_stride + ((size_t)p * n_kv + kvh) * hd;
    float* sc = (which == 0 ? kscales : vscales) + s * (seq_stride / hd) + (size_t)p * n_kv + kvh;
    float amax = 0.0f;
    for (uint32_t i = lane; i < hd; i += 64) amax = fmaxf(amax, fabsf(src[i]));
    amax = wave_max(amax);
    const float scale = q_scale(amax);
    const float inv = __fdiv_rn(1.0f, scale);
    const uint32_t body = hd & ~7u;
    for (uint32_t i = lane; i < hd; i += 64) dst[i] = (i < body) ? q_body(src[i], inv) : q_tail(src[i], scale);
    if (lane == 0) *sc = scale;
}

// --------------------------------------------------------------- partials
// grid (n_chunks, n_kv, n_seq), one wave.  HD = head_dim, G = heads per kv head.
// Partial record per (seq, chunk, head): [m, l, o[HD]].
template <int HD, int G>
__global__ __launch_bounds__(64) void k_attn_partial(const float* __restrict__ q, const int8_t* __restrict__ keys,
                                                     const int8_t* __restrict__ vals,
                                                     const float* __restrict__ kscales,
                                                     const float* __restrict__ vscales, const int32_t* __restrict__ ctx,
                                                     uint64_t seq_stride, uint32_t n_kv, uint32_t n_chunks_max,
                                                     uint32_t max_ctx, float* __restrict__ ws) {
    constexpr int DPL = HD / 64;  // dims per lane in the PV phase
    __shared__ float q_s[G][HD];
    __shared__ float p_s[64][G];
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z, lane = threadIdx.x;
    const int32_t L = min(ctx[s], (int32_t)max_ctx);
    const uint32_t c0 = chunk * kAttnChunk;
    if (L <= 0 || c0 >= (uint32_t)L) return;
    const uint32_t c1 = min((uint32_t)L, c0 + kAttnChunk);
    const uint32_t n_heads = n_kv * G;
    const float scale = 1.0f / sqrtf((float)HD);
    for (int g = 0; g < G; ++g)
        for (int d = lane; d < HD; d += 64) q_s[g][d] = q[((size_t)s * n_heads + kvh + n_kv * g) * HD + d];
    __syncthreads();

    const int8_t* kbase = keys + s * seq_stride + (size_t)kvh * HD;
    const int8_t* vbase = vals + s * seq_stride + (size_t)kvh * HD;
    const float* ksb = kscales + s * (seq_stride / HD) + kvh;
    const float* vsb = vscales + s * (seq_stride / HD) + kvh;
    const size_t row = (size_t)n_kv * HD;

    float m[G], l[G], o[G][DPL];
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
        for (int e = 0; e < DPL; ++e) o[g][e] = 0.0f;
    }
    for (uint32_t p0 = c0; p0 < c1; p0 += 64) {
        // ---- scores: lane = token
        const uint32_t p = p0 + lane;
        const bool valid = p < c1;
        float acc[G];
        for (int g = 0; g < G; ++g) acc[g] = 0.0f;
        if (valid) {
            const int8_t* kr = kbase + p * row;
#pragma unroll 4
            for (int c = 0; c < HD / 16; ++c) {
                const uint4 kw = *(const uint4*)(kr + 16 * c);
                const uint32_t w4[4] = {kw.x, kw.y, kw.z, kw.w};
                float kf[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) kf[i] = (float)(int8_t)((w4[i >> 2] >> (8 * (i & 3))) & 0xFF);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float4* qv = (const float4*)&q_s[g][16 * c];
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4) {
                        const float4 qq = qv[i4];
                        acc[g] = fmaf(qq.x, kf[4 * i4 + 0], acc[g]);
                        acc[g] = fmaf(qq.y, kf[4 * i4 + 1], acc[g]);
                        acc[g] = fmaf(qq.z, kf[4 * i4 + 2], acc[g]);
                        acc[g] = fmaf(qq.w, kf[4 * i4 + 3], acc[g]);
                    }
                }
            }
        }
        const float ks = valid ? ksb[(size_t)p * n_kv] : 0.0f;
        const float vs = valid ? vsb[(size_t)p * n_kv] : 0.0f;
        for (int g = 0; g < G; ++g) {
            const float sc = valid ? acc[g] * ks * scale : -INFINITY;
            const float mn = fmaxf(m[g], wave_max(sc));
            const float corr = __expf(m[g] - mn);
            const float e = valid ? __expf(sc - mn) : 0.0f;
            l[g] = l[g] * corr + wave_sum(e);
            m[g] = mn;
            for (int d = 0; d < DPL; ++d) o[g][d] *= corr;
            p_s[lane][g] = e * vs;
        }
        __syncthreads();
        // ---- values: lane = dims [DPL*lane, DPL*lane+DPL)
        const uint32_t nt = c1 - p0 < 64 ? c1 - p0 : 64;
        for (uint32_t j = 0; j < nt; ++j) {
            const int8_t* vr = vbase + (size_t)(p0 + j) * row + DPL * lane;
            float vf[DPL];
            if constexpr (DPL == 4) {
                const uint32_t vw = *(const uint32_t*)vr;
                for (int i = 0; i < 4; ++i) vf[i] = (float)(int8_t)((vw >> (8 * i)) & 0xFF);
            } else {
                for (int i = 0; i < DPL; ++i) vf[i] = (float)vr[i];
            }
            for (int g = 0; g < G; ++g) {
                const float pg = p_s[j][g];
                for (int d = 0; d < DPL; ++d) o[g][d] = fmaf(pg, vf[d], o[g][d]);
            }
        }
        __syncthreads();
    }
    for (int g = 0; g < G; ++g) {
        float* rec = ws + (((size_t)s * n_chunks_max + chunk) * n_heads + kvh + n_kv * g) * (HD + 2);
        if (lane == 0) {
            rec[0] = m[g];
            rec[1] = l[g];
        }
        for (int d = 0; d < DPL; ++d) rec[2 + DPL * lane + d] = o[g][d];
    }
}

// grid (n_heads, n_seq): merge the chunk partials of one head.
template <int HD>
__global__ __launch_bounds__(64) void k_attn_combine(const float* __restrict__ ws, const int32_t* __restrict__ ctx,
                                                     float* __restrict__ out, uint32_t n_heads,
                                                     uint32_t n_chunks_max, uint32_t max_ctx) {
    constexpr int DPL = HD / 64;
    const uint32_t h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
    const int32_t L = min(ctx[s], (int32_t)max_ctx);
    float* dst = out + ((size_t)s * n_heads + h) * HD + DPL * lane;
    if (L <= 0) {
        for (int d = 0; d < DPL; ++d) dst[d] = 0.0f;
        return;
    }
    const uint32_t nc = ((uint32_t)L + kAttnChunk - 1) / kAttnChunk;
    const float* base = ws + ((size_t)s * n_chunks_max * n_heads + h) * (HD + 2);
    const size_t cstride = (size_t)n_heads * (HD + 2);
    float M = -INFINITY;
    for (uint32_t c = 0; c < nc; ++c) M = fmaxf(M, base[c * cstride]);
    float den = 0.0f, acc[DPL];
    for (int d = 0; d < DPL; ++d) acc[d] = 0.0f;
    for (uint32_t c = 0; c < nc; ++c) {
        const float* rec = base + c * cstride;
        const float w = __expf(rec[0] - M);
        den = fmaf(w, rec[1], den);
        for (int d = 0; d < DPL; ++d) acc[d] = fmaf(w, rec[2 + DPL * lane + d], acc[d]);
    }
    const float inv = 1.0f / den;
    for (int d = 0; d < DPL; ++d) dst[d] = acc[d] * inv;
}

template <int HD, int G>
static void launch_attn(const float* q, const int8_t* keys, const int8_t* vals, const float* ks, const float* vs,
                        float* out, const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride, uint32_t n_kv,
                        uint32_t ncm, uint32_t max_ctx, float* ws, hipStream_t st) {
    hipLaunchKernelGGL((k_attn_partial<HD, G>), dim3(ncm, n_kv, n_seq), dim3(64), 0, st, q, keys, vals, ks, vs, ctx,
                       seq_stride, n_kv, ncm, max_ctx, ws);
    hipLaunchKernelGGL((k_attn_combine<HD>), dim3(n_kv * G, n_seq), dim3(64), 0, st, ws, ctx, out, n_kv * G, ncm,
                       max_ctx);
}

}  // namespace ec

using namespace ec;

extern "C" int ec_kv_append(const float* k, const float* v, int8_t* keys, int8_t* vals, float* kscales,
                            float* vscales, const int32_t* pos, uint32_t n_seq, uint64_t seq_stride, uint32_t n_kv,
                            uint32_t head_dim, void* stream) {
    if (n_seq == 0) return EC_OK;
    if (!k || !v || !keys || !vals || !kscales || !vscales || !pos || n_kv == 0 || head_dim == 0 ||
        seq_stride % head_dim)
        return ec_set_error(EC_ERR_ARG, "ec_kv_append: bad argument");
    hipLaunchKernelGGL(k_kv_append, dim3(n_kv, n_seq, 2), dim3(64), 0, (hipStream_t)stream, k, v, keys, vals, kscales,
                       vscales, pos, seq_stride, n_kv, head_dim);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" size_t ec_attn_ws_bytes(uint32_t n_seq, uint32_t n_heads, uint32_t head_dim, uint32_t max_ctx) {
    const size_t ncm = (max_ctx + kAttnChunk - 1) / kAttnChunk;
    return (size_t)n_seq * (ncm ? ncm : 1) * n_heads * (head_dim + 2) * sizeof(float);
}

extern "C" int ec_attn_decode(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                              const float* vscales, float* out, const int32_t* ctx, uint32_t n_seq,
                              uint64_t seq_stride, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
                              uint32_t max_ctx, void* ws, void* stream) {
    if (n_seq == 0) return EC_OK;
    if (!q || !keys || !vals || !kscales || !vscales || !out || !ctx || !ws || n_kv == 0 || n_heads % n_kv ||
        max_ctx == 0 || seq_stride < (uint64_t)max_ctx * n_kv * head_dim)
        return ec_set_error(EC_ERR_ARG, "ec_attn_decode: bad argument");
    const uint32_t G = n_heads / n_kv;
    const uint32_t ncm = (max_ctx + kAttnChunk - 1) / kAttnChunk;
    hipStream_t st = (hipStream_t)stream;
    float* w = (float*)ws;
#define EC_ATTN(HD_, G_) \
    launch_attn<HD_, G_>(q, keys, vals, kscales, vscales, out, ctx, n_seq, seq_stride, n_kv, ncm, max_ctx, w, st)
    if (head_dim == 256 && G == 4) EC_ATTN(256, 4);
    else if (head_dim == 256 && G == 1) EC_ATTN(256, 1);
    else if (head_dim == 256 && G == 2) EC_ATTN(256, 2);
    else if (head_dim == 256 && G == 8) EC_ATTN(256, 8);
    else if (head_dim == 128 && G == 4) EC_ATTN(128, 4);
    else if (head_dim == 128 && G == 1) EC_ATTN(128, 1);
    else if (head_dim == 128 && G == 2) EC_ATTN(128, 2);
    else if (head_dim == 128 && G == 8) EC_ATTN(128, 8);
    else if (head_dim == 64 && G == 1) EC_ATTN(64, 1);
    else if (head_dim == 64 && G == 2) EC_ATTN(64, 2);
    else if (head_dim == 64 && G == 4) EC_ATTN(64, 4);
    else
        return ec_set_error(EC_ERR_UNSUPPORTED,
                            "ec_attn_decode: head_dim must be 64/128/256 and n_heads/n_kv in {1,2,4,8}");
#undef EC_ATTN
    EC_CHECK_LAUNCH();
    return EC_OK;
}
