/*
 * oracle.c — CPU restatement of echo-core's decode hot path (see oracle.h).
 * TEST INFRASTRUCTURE ONLY: the checker, never the product.
 *
 * Built with plain gcc, no -ffast-math, no FMA (-ffp-contract=off), so every
 * float operation below rounds exactly as written.
 */
#include "oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>

/* ------------------------------------------------------------------ fp16 */
/* Exact binary16 -> binary32 (include/types.h:13-15 uses F16C, which is exact). */
float oc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even (include/types.h:17-19, imm 0 = RNE). */
uint16_t oc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    }
    if (ax >= 0x477FF000u) { /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax < 0x38800000u) { /* below min normal half: subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 -> 0 (ties to even at 2^-25 -> 0) */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); half subnormal unit 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal */
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------- RNG */
uint64_t oc_splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* ------------------------------------------------------------- quantizer */
/* src/kernels/quant.cpp:18-98.  Pass 1 (:29-60) is max|x| over the row.
 * scale (:63): amax>0 ? amax/127 : 1.  Body (:70-88): elements of whole
 * 8-chunks use x * (1/scale) rounded half-to-even (_MM_FROUND_TO_NEAREST_INT),
 * then packs_epi32/packs_epi16 saturation to [-128,127].  Tail (:90-96):
 * std::round(x/scale) (half away from zero) clamped to [-127,127]. */
void oc_quantize_per_token_symmetric(const float* input, int8_t* output, float* scales,
                                     uint32_t num_tokens, uint32_t num_elements) {
    for (uint32_t t = 0; t < num_tokens; ++t) {
        const float* row = input + (size_t)t * num_elements;
        int8_t* out = output + (size_t)t * num_elements;
        float amax = 0.0f;
        for (uint32_t i = 0; i < num_elements; ++i) {
            float a = fabsf(row[i]);
            if (a > amax) amax = a;
        }
        float scale = (amax > 0.0f) ? (amax / 127.0f) : 1.0f;
        scales[t] = scale;
        float inv = 1.0f / scale;
        uint32_t body = num_elements & ~7u;
        for (uint32_t i = 0; i < body; ++i) {
            float r = rintf(row[i] * inv);
            int v = (int)r;
            if (v > 127) v = 127;
            if (v < -128) v = -128;
            out[i] = (int8_t)v;
        }
        for (uint32_t i = body; i < num_elements; ++i) {
            int v = (int)roundf(row[i] / scale);
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            out[i] = (int8_t)v;
        }
    }
}

/* src/kernels/quant.cpp:100-144 (and echo-core-zig/src/kernels/quant.zig:89-110
 * for the scalar order used here: score += k * scale * q). */
void oc_fused_dequant_dot_int8(const float* query, const int8_t* key_cache, const float* scales,
                               float* scores, uint32_t dim, uint32_t seq_len) {
    for (uint32_t p = 0; p < seq_len; ++p) {
        const int8_t* key = key_cache + (size_t)p * dim;
        float s = 0.0f;
        for (uint32_t k = 0; k < dim; ++k) s += (float)key[k] * scales[p] * query[k];
        scores[p] = s;
    }
}

/* -------------------------------------------------------------- Q4_K unpack */
/* src/kernels/quant.cpp:222-242 (= get_scale_min_k4). */
void oc_q4k_scale_min(const uint8_t* q, int j, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

uint32_t oc_q4k_pos(uint32_t s, uint32_t i) {
    uint32_t g = s >> 1, p = s & 1;
    return (i < 16) ? (64 * g + 16 * p + i) : (64 * g + 32 + 16 * p + (i - 16));
}

static inline uint8_t q4k_nib(const uint8_t* qs, uint32_t s, uint32_t i) {
    return (i < 16) ? (qs[16 * s + i] & 0x0F) : (qs[16 * s + i - 16] >> 4);
}

/* ------------------------------------------------------------- row dots */
static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

double oc_dot_q8_0_f64(const uint8_t* blocks, uint32_t n_blocks, const float* x) {
    double acc = 0.0;
    for (uint32_t b = 0; b < n_blocks; ++b) {
        const uint8_t* bp = blocks + 34 * (size_t)b;
        double d = oc_fp16_to_fp32(rd16(bp));
        const int8_t* qs = (const int8_t*)(bp + 2);
        for (int j = 0; j < 32; ++j) acc += d * (double)qs[j] * (double)x[32 * b + j];
    }
    return acc;
}

double oc_dot_q4_K_f64(const uint8_t* blocks, uint32_t n_blocks, const float* x) {
    double acc = 0.0;
    for (uint32_t b = 0; b < n_blocks; ++b) {
        const uint8_t* bp = blocks + 144 * (size_t)b;
        double d = oc_fp16_to_fp32(rd16(bp)), dmin = oc_fp16_to_fp32(rd16(bp + 2));
        const uint8_t* sc12 = bp + 4;
        const uint8_t* qs = bp + 16;
        for (uint32_t s = 0; s < 8; ++s) {
            uint8_t sc, m;
            oc_q4k_scale_min(sc12, (int)s, &sc, &m);
            for (uint32_t i = 0; i < 32; ++i) {
                double w = d * sc * q4k_nib(qs, s, i) - dmin * m;
                acc += w * (double)x[256 * b + oc_q4k_pos(s, i)];
            }
        }
    }
    return acc;
}

/* src/kernels/matvec.cpp:62-87: per block float block_sum over j in order,
 * then sum += d * block_sum; y[m] += sum.  K%32 tail ignored (:65). */
void oc_matvec_q8_0(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    const uint8_t* base = (const uint8_t*)blocks;
    uint32_t nb = K / 32;
    for (uint32_t m = 0; m < M; ++m) {
        float sum = 0.0f;
        const uint8_t* row = base + (size_t)m * nb * 34;
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t* bp = row + (size_t)b * 34;
            float d = oc_fp16_to_fp32(rd16(bp));
            const int8_t* qs = (const int8_t*)(bp + 2);
            float bs = 0.0f;
            for (int j = 0; j < 32; ++j) bs += (float)qs[j] * x[32 * b + j];
            sum += d * bs;
        }
        y[m] += sum;
    }
}

/* src/kernels/matvec.cpp:92-142, same interleaved order of the four 16-runs. */
void oc_matvec_q4_K(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    const uint8_t* base = (const uint8_t*)blocks;
    uint32_t nb = K / 256;
    for (uint32_t m = 0; m < M; ++m) {
        float sum = 0.0f;
        const uint8_t* row = base + (size_t)m * nb * 144;
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t* bp = row + (size_t)b * 144;
            float d = oc_fp16_to_fp32(rd16(bp)), dmin = oc_fp16_to_fp32(rd16(bp + 2));
            const uint8_t* sc = bp + 4;
            const uint8_t* qs = bp + 16;
            const float* xb = x + 256 * b;
            for (int blk = 0; blk < 4; ++blk) {
                uint8_t sc0, mn0, sc1, mn1;
                oc_q4k_scale_min(sc, 2 * blk, &sc0, &mn0);
                oc_q4k_scale_min(sc, 2 * blk + 1, &sc1, &mn1);
                float rs0 = d * sc0, rm0 = dmin * mn0, rs1 = d * sc1, rm1 = dmin * mn1;
                int qo = blk * 32, wo = blk * 64;
                for (int j = 0; j < 16; ++j) {
                    sum += (rs0 * (qs[qo + j] & 0x0F) - rm0) * xb[wo + j];
                    sum += (rs1 * (qs[qo + 16 + j] & 0x0F) - rm1) * xb[wo + 16 + j];
                    sum += (rs0 * (qs[qo + j] >> 4) - rm0) * xb[wo + 32 + j];
                    sum += (rs1 * (qs[qo + 16 + j] >> 4) - rm1) * xb[wo + 48 + j];
                }
            }
        }
        y[m] += sum;
    }
}

/* ------------------------------------------------- activation quantization */
void oc_quantize_act_q8_0(const float* x, int8_t* xq, float* xd, uint32_t K) {
    oc_quantize_per_token_symmetric(x, xq, xd, K / 32, 32);
}

void oc_quantize_act_q4_K(const float* x, int8_t* xq, float* xd, int32_t* xsum, uint32_t K) {
    float tmp[32];
    uint32_t nsb = K / 32;
    for (uint32_t sb = 0; sb < nsb; ++sb) {
        uint32_t b = sb / 8, s = sb % 8;
        for (uint32_t i = 0; i < 32; ++i) tmp[i] = x[256 * b + oc_q4k_pos(s, i)];
        oc_quantize_per_token_symmetric(tmp, xq + 32 * sb, xd + sb, 1, 32);
        int32_t acc = 0;
        for (uint32_t i = 0; i < 32; ++i) acc += xq[32 * sb + i];
        if (xsum) xsum[sb] = acc;
    }
}

/* Two-piece activation (design): piece 0 is the reference quantizer per
 * 32-element block (scale s = amax/127, q0 = sat8(rne(x * (1/s)))); piece 1
 * quantizes the residual r = fma(-q0, s, x) with the scale s/256:
 * q1 = sat8(rne(r * ((1/s) * 256))).  x ~ q0*s + q1*(s/256), |error| <=
 * s/512 except where q0 saturated.  xd holds s per block. */
void oc_quantize_act2_q8_0(const float* x, int8_t* xq0, int8_t* xq1, float* xd, uint32_t K) {
    oc_quantize_per_token_symmetric(x, xq0, xd, K / 32, 32);
    for (uint32_t k = 0; k < K; ++k) {
        const float sc = xd[k / 32];
        const float inv1 = (1.0f / sc) * 256.0f;
        const float r = fmaf(-(float)xq0[k], sc, x[k]);
        int v = (int)rintf(r * inv1);
        if (v > 127) v = 127;
        if (v < -128) v = -128;
        xq1[k] = (int8_t)v;
    }
}

void oc_dequant_act2_q8_0(const int8_t* xq0, const int8_t* xq1, const float* xd, float* x_deq, uint32_t K) {
    for (uint32_t k = 0; k < K; ++k) {
        const float sc = xd[k / 32];
        x_deq[k] = (float)xq0[k] * sc + (float)xq1[k] * (sc * (1.0f / 256.0f));
    }
}

/* Two pieces per 32-element Q4_K sub-block (positions in oc_q4k_pos order, as
 * oc_quantize_act_q4_K): piece 0 the reference quantizer of the sub-block,
 * piece 1 its residual at scale/256 as in oc_quantize_act2_q8_0. */
void oc_quantize_act2_q4_K(const float* x, int8_t* xq0, int8_t* xq1, float* xd, uint32_t K) {
    float tmp[32];
    for (uint32_t sb = 0; sb < K / 32; ++sb) {
        uint32_t b = sb / 8, s = sb % 8;
        for (uint32_t i = 0; i < 32; ++i) tmp[i] = x[256 * b + oc_q4k_pos(s, i)];
        oc_quantize_act2_q8_0(tmp, xq0 + 32 * sb, xq1 + 32 * sb, xd + sb, 32);
    }
}

void oc_dequant_act2_q4_K(const int8_t* xq0, const int8_t* xq1, const float* xd, float* x_deq, uint32_t K) {
    for (uint32_t sb = 0; sb < K / 32; ++sb) {
        uint32_t b = sb / 8, s = sb % 8;
        float tmp[32];
        oc_dequant_act2_q8_0(xq0 + 32 * sb, xq1 + 32 * sb, xd + sb, tmp, 32);
        for (uint32_t i = 0; i < 32; ++i) x_deq[256 * b + oc_q4k_pos(s, i)] = tmp[i];
    }
}

void oc_dequant_act_q8_0(const int8_t* xq, const float* xd, float* x_deq, uint32_t K) {
    for (uint32_t k = 0; k < K; ++k) x_deq[k] = (float)xq[k] * xd[k / 32];
}

void oc_dequant_act_q4_K(const int8_t* xq, const float* xd, float* x_deq, uint32_t K) {
    for (uint32_t sb = 0; sb < K / 32; ++sb) {
        uint32_t b = sb / 8, s = sb % 8;
        for (uint32_t i = 0; i < 32; ++i) x_deq[256 * b + oc_q4k_pos(s, i)] = (float)xq[32 * sb + i] * xd[sb];
    }
}

/* -------------------------------------------------------- integer dots */
void oc_block_dots_q8_0(const void* blocks, const int8_t* xq, int32_t* out, uint32_t M, uint32_t K) {
    const uint8_t* base = (const uint8_t*)blocks;
    uint32_t nb = K / 32;
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t b = 0; b < nb; ++b) {
            const int8_t* qs = (const int8_t*)(base + ((size_t)m * nb + b) * 34 + 2);
            int32_t acc = 0;
            for (int j = 0; j < 32; ++j) acc += (int32_t)qs[j] * xq[32 * b + j];
            out[(size_t)m * nb + b] = acc;
        }
}

void oc_block_dots_q4_K(const void* blocks, const int8_t* xq, int32_t* out, uint32_t M, uint32_t K) {
    const uint8_t* base = (const uint8_t*)blocks;
    uint32_t nb = K / 256;
    for (uint32_t m = 0; m < M; ++m)
        for (uint32_t b = 0; b < nb; ++b) {
            const uint8_t* qs = base + ((size_t)m * nb + b) * 144 + 16;
            for (uint32_t s = 0; s < 8; ++s) {
                int32_t acc = 0;
                for (uint32_t i = 0; i < 32; ++i) acc += (int32_t)q4k_nib(qs, s, i) * xq[(8 * b + s) * 32 + i];
                out[(size_t)m * (K / 32) + 8 * b + s] = acc;
            }
        }
}

/* --------------------------------------------------------------- KV cache */
/* src/kv_cache.cpp:89-113 quantizes one token's row; the readers index the
 * scale as pos*n_kv + kv_head (src/inference.cpp:347,387), so each
 * (token, kv_head) row of head_dim gets its own scale here. */
void oc_kv_append(const float* k, const float* v, int8_t* keys, int8_t* vals,
                  float* kscales, float* vscales, uint32_t pos, uint32_t n_kv, uint32_t head_dim) {
    size_t row = (size_t)n_kv * head_dim;
    oc_quantize_per_token_symmetric(k, keys + pos * row, kscales + (size_t)pos * n_kv, n_kv, head_dim);
    oc_quantize_per_token_symmetric(v, vals + pos * row, vscales + (size_t)pos * n_kv, n_kv, head_dim);
}

/* ------------------------------------------------------------- attention */
/* echo-core-zig/src/inference/engine.zig:563-616 with core/math.zig:39-52. */
void oc_attn_decode_int8(const float* q, const int8_t* keys, const int8_t* vals,
                         const float* kscales, const float* vscales, float* out,
                         uint32_t n_heads, uint32_t n_kv, uint32_t head_dim, uint32_t ctx) {
    size_t kv_dim = (size_t)n_kv * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    float* sc_all = (float*)malloc(sizeof(float) * (size_t)n_heads * (ctx ? ctx : 1));
#pragma omp parallel for schedule(static)
    for (uint32_t h = 0; h < n_heads; ++h) {
        float* sc = sc_all + (size_t)h * (ctx ? ctx : 1);
        uint32_t kvh = h % n_kv;
        const float* qh = q + (size_t)h * head_dim;
        for (uint32_t p = 0; p < ctx; ++p) {
            const int8_t* kp = keys + p * kv_dim + (size_t)kvh * head_dim;
            float ks = kscales[(size_t)p * n_kv + kvh];
            float s = 0.0f;
            for (uint32_t d = 0; d < head_dim; ++d) s += qh[d] * (float)kp[d] * ks;
            sc[p] = s * scale;
        }
        float mx = -INFINITY;
        for (uint32_t p = 0; p < ctx; ++p) if (sc[p] > mx) mx = sc[p];
        float sum = 0.0f;
        for (uint32_t p = 0; p < ctx; ++p) { sc[p] = expf(sc[p] - mx); sum += sc[p]; }
        for (uint32_t p = 0; p < ctx; ++p) sc[p] /= sum;
        float* oh = out + (size_t)h * head_dim;
        for (uint32_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
        for (uint32_t p = 0; p < ctx; ++p) {
            const int8_t* vp = vals + p * kv_dim + (size_t)kvh * head_dim;
            float vsc = vscales[(size_t)p * n_kv + kvh];
            for (uint32_t d = 0; d < head_dim; ++d) oh[d] += sc[p] * ((float)vp[d] * vsc);
        }
    }
    free(sc_all);
}

/* -------------------------------------------------------------- delta-net */
/* echo-core-zig/src/kernels/qwen_linear.zig:207-250 (one token). */
void oc_deltanet_step(float* state, const float* q, const float* k, const float* v,
                      const float* decay, const float* beta, float* out,
                      uint32_t n_v, uint32_t n_k, uint32_t d_k, uint32_t d_v) {
    uint32_t rep = n_v / n_k;
    float scale = 1.0f / sqrtf((float)d_k);
#pragma omp parallel for schedule(static)
    for (uint32_t h = 0; h < n_v; ++h) {
        float delta[256]; /* d_v <= 256, as qwen_linear.zig:224-225 */
        uint32_t qh = h / rep;
        const float* kh = k + (size_t)qh * d_k;
        const float* qv = q + (size_t)qh * d_k;
        float* S = state + (size_t)h * d_k * d_v;
        float dc = decay[h], bt = beta[h];
        for (size_t i = 0; i < (size_t)d_k * d_v; ++i) S[i] *= dc;               /* :221-222 */
        for (uint32_t vi = 0; vi < d_v; ++vi) {                                  /* :227-233 */
            float kv = 0.0f;
            for (uint32_t ki = 0; ki < d_k; ++ki) kv += S[(size_t)ki * d_v + vi] * kh[ki];
            delta[vi] = (v[(size_t)h * d_v + vi] - kv) * bt;
        }
        for (uint32_t ki = 0; ki < d_k; ++ki)                                    /* :235-240 */
            for (uint32_t vi = 0; vi < d_v; ++vi) S[(size_t)ki * d_v + vi] += kh[ki] * delta[vi];
        for (uint32_t vi = 0; vi < d_v; ++vi) {                                  /* :242-249 */
            float o = 0.0f;
            for (uint32_t ki = 0; ki < d_k; ++ki) o += S[(size_t)ki * d_v + vi] * (qv[ki] * scale);
            out[(size_t)h * d_v + vi] = o;
        }
    }
}

/* ------------------------------------------------------------------ glue */
void oc_rmsnorm(const float* x, const float* w, float* out, uint32_t n) {
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    float rms = sqrtf(ss / (float)n + 1e-6f);
    float inv = 1.0f / rms;
    for (uint32_t i = 0; i < n; ++i) out[i] = x[i] * inv * w[i];
}

void oc_head_rmsnorm(float* x, const float* w, uint32_t n_heads, uint32_t head_dim) {
    for (uint32_t h = 0; h < n_heads; ++h) oc_rmsnorm(x + (size_t)h * head_dim, w, x + (size_t)h * head_dim, head_dim);
}

void oc_rope_inv_freq(float* inv_freq, uint32_t head_dim, float base) {
    for (uint32_t i = 0; i < head_dim; i += 2) inv_freq[i / 2] = 1.0f / powf(base, (float)i / (float)head_dim);
}

void oc_rope(float* x, uint32_t n_heads, uint32_t head_dim, uint32_t pos, const float* inv_freq) {
    for (uint32_t h = 0; h < n_heads; ++h) {
        float* xh = x + (size_t)h * head_dim;
        for (uint32_t i = 0; i < head_dim; i += 2) {
            float ang = (float)pos * inv_freq[i / 2];
            float c = cosf(ang), s = sinf(ang);
            float a = xh[i], b = xh[i + 1];
            xh[i] = a * c - b * s;
            xh[i + 1] = a * s + b * c;
        }
    }
}

float oc_silu(float x) { return x / (1.0f + expf(-x)); }

float oc_softplus(float x) { return (x > 20.0f) ? x : log1pf(expf(x)); }

void oc_l2norm_heads(float* x, uint32_t n_heads, uint32_t head_dim) {
    for (uint32_t h = 0; h < n_heads; ++h) {
        float* xh = x + (size_t)h * head_dim;
        float ss = 0.0f;
        for (uint32_t d = 0; d < head_dim; ++d) ss += xh[d] * xh[d];
        float inv = 1.0f / sqrtf(ss + 1e-6f);
        for (uint32_t d = 0; d < head_dim; ++d) xh[d] *= inv;
    }
}

void oc_conv_step(float* st, const float* x, const float* w, float* out, uint32_t C, uint32_t kernel) {
    for (uint32_t t = kernel - 1; t > 0; --t) memcpy(st + (size_t)t * C, st + (size_t)(t - 1) * C, sizeof(float) * C);
    memcpy(st, x, sizeof(float) * C);
    for (uint32_t c = 0; c < C; ++c) {
        float acc = 0.0f;
        for (uint32_t t = 0; t < kernel; ++t) acc += st[(size_t)t * C + c] * w[(size_t)(kernel - 1 - t) * C + c];
        out[c] = oc_silu(acc);
    }
}

uint32_t oc_argmax(const float* x, uint32_t n) {
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; ++i) if (x[i] > x[best]) best = i;
    return best;
}

/* ---------------------------------------------------------------- decoder */
#ifdef OC_BASELINE
/* AVX2 + OpenMP row kernel (baseline_avx2.c) for the CPU-baseline build. */
void ob_matvec_q8_0_avx2(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K);
#define OC_MV_IMPL ob_matvec_q8_0_avx2
#else
#define OC_MV_IMPL oc_matvec_q8_0
#endif

/* Embedding row of a Q8_0 table (engine.zig:41-50): x[i] = d_b * qs[i]. */
void oc_embed_row_q8_0(const uint8_t* embed, uint32_t H, uint32_t token, float* x) {
    uint32_t nb = H / 32;
    const uint8_t* row = embed + (size_t)token * nb * 34;
    for (uint32_t bb = 0; bb < nb; ++bb) {
        float d = oc_fp16_to_fp32(rd16(row + 34 * bb));
        const int8_t* qs = (const int8_t*)(row + 34 * bb + 2);
        for (int j = 0; j < 32; ++j) x[32 * bb + j] = d * (float)qs[j];
    }
}

void oc_embed_row(int fmt, const void* embed, uint32_t H, uint32_t token, float* x) {
    if (fmt == OC_F16) {
        const uint8_t* row = (const uint8_t*)embed + (size_t)token * H * 2;
        for (uint32_t i = 0; i < H; ++i) x[i] = oc_fp16_to_fp32(rd16(row + 2 * i));
    } else if (fmt == OC_F32) {
        memcpy(x, (const float*)embed + (size_t)token * H, H * sizeof(float));
    } else {
        oc_embed_row_q8_0((const uint8_t*)embed, H, token, x);
    }
}

/* echo-core-zig/src/kernels/qwen_linear.zig:215-219 (per value head h):
 * beta = 1/(1+exp(-b)), g = -exp(A_log)*softplus(alpha + dt_bias), decay = exp(g). */
void oc_deltanet_gates(const float* alpha, const float* beta_logit, const float* a_log, const float* dt_bias,
                       float* decay, float* beta, uint32_t n_v) {
    for (uint32_t h = 0; h < n_v; ++h) {
        beta[h] = 1.0f / (1.0f + expf(-beta_logit[h]));
        float g = -expf(a_log[h]) * oc_softplus(alpha[h] + dt_bias[h]);
        decay[h] = expf(g);
    }
}

/* echo-core-zig/src/kernels/qwen_linear.zig:244-257 (per value head h of d_v):
 * core <- core * (1/sqrt(sum(core^2)/d_v + 1e-6)) * w[i] * silu(z), squares
 * summed in index order as the readout loop accumulates them. */
void oc_gated_rmsnorm(float* core, const float* z, const float* w, uint32_t n_v, uint32_t d_v) {
    for (uint32_t h = 0; h < n_v; ++h) {
        float* oh = core + (size_t)h * d_v;
        float rms = 0.0f;
        for (uint32_t vi = 0; vi < d_v; ++vi) rms += oh[vi] * oh[vi];
        rms = sqrtf(rms / (float)d_v + 1e-6f);
        float inv = 1.0f / rms;
        for (uint32_t vi = 0; vi < d_v; ++vi) {
            float nrm = oh[vi] * inv * w[vi];
            oh[vi] = nrm * oc_silu(z[(size_t)h * d_v + vi]);
        }
    }
}

typedef struct {
    uint32_t H, q_dim, kv_dim, value_dim, n_v, d_v, key_dim, d_k, n_k, conv_dim, maxK, big;
} dims_t;

static dims_t dims_of(const oc_model_cfg* c) {
    dims_t d;
    d.H = c->hidden;
    d.q_dim = c->n_heads * c->head_dim;
    d.kv_dim = c->n_kv * c->head_dim;
    /* ssm_heads == 0: a model without delta-net blocks (every block attention) */
    d.value_dim = c->ssm_inner;
    d.n_v = c->ssm_heads;
    d.d_v = d.n_v ? d.value_dim / d.n_v : 0;
    d.key_dim = d.value_dim / 2; /* qwen_linear.zig:117-124 */
    d.d_k = d.d_v;
    d.n_k = d.d_k ? d.key_dim / d.d_k : 0;
    d.conv_dim = 2 * d.key_dim + d.value_dim;
    d.maxK = d.H;
    if (c->ffn > d.maxK) d.maxK = c->ffn;
    if (d.value_dim > d.maxK) d.maxK = d.value_dim;
    if (d.q_dim > d.maxK) d.maxK = d.q_dim;
    d.big = d.conv_dim;
    if (c->ffn > d.big) d.big = c->ffn;
    if (d.q_dim + 2 * d.kv_dim > d.big) d.big = d.q_dim + 2 * d.kv_dim;
    return d;
}

/* Scratch for mv(): the quantized activation and its dequantized copy. */
typedef struct {
    float* deq;
    int8_t* qq;
    int8_t* qq1;
    float* qd;
} mv_scratch;

static mv_scratch mv_alloc(uint32_t maxK) {
    mv_scratch m;
    m.deq = (float*)calloc(maxK, sizeof(float));
    m.qq = (int8_t*)calloc(maxK, 1);
    m.qq1 = (int8_t*)calloc(maxK, 1);
    m.qd = (float*)calloc(maxK / 32 + 1, sizeof(float));
    return m;
}
static void mv_free(mv_scratch* m) { free(m->deq); free(m->qq); free(m->qq1); free(m->qd); }

/* Matvec with optional activation quantization: y = W * x (y zeroed first).
 * quant_act 0: fp32 x (reference); 1: x quantized per 32-block; 2: x as two
 * int8 pieces per 32-block (oc_quantize_act2_q8_0).  A Q4_K matrix quantizes
 * its input per 32-element sub-block (oc_quantize_act_q4_K, or
 * oc_quantize_act2_q4_K for 2). */
static void mv_fmt(int fmt, const uint8_t* W, const float* x, float* y, uint32_t M, uint32_t K, int quant_act,
                   mv_scratch* s) {
    memset(y, 0, sizeof(float) * M);
    if (fmt == OC_Q4_K) {
        if (quant_act == 2) {
            oc_quantize_act2_q4_K(x, s->qq, s->qq1, s->qd, K);
            oc_dequant_act2_q4_K(s->qq, s->qq1, s->qd, s->deq, K);
            oc_matvec_q4_K(W, s->deq, y, M, K);
        } else if (quant_act) {
            oc_quantize_act_q4_K(x, s->qq, s->qd, NULL, K);
            oc_dequant_act_q4_K(s->qq, s->qd, s->deq, K);
            oc_matvec_q4_K(W, s->deq, y, M, K);
        } else {
            oc_matvec_q4_K(W, x, y, M, K);
        }
    } else if (quant_act == 2) {
        oc_quantize_act2_q8_0(x, s->qq, s->qq1, s->qd, K);
        oc_dequant_act2_q8_0(s->qq, s->qq1, s->qd, s->deq, K);
        OC_MV_IMPL(W, s->deq, y, M, K);
    } else if (quant_act) {
        oc_quantize_act_q8_0(x, s->qq, s->qd, K);
        oc_dequant_act_q8_0(s->qq, s->qd, s->deq, K);
        OC_MV_IMPL(W, s->deq, y, M, K);
    } else {
        OC_MV_IMPL(W, x, y, M, K);
    }
}

static void mv(const uint8_t* W, const float* x, float* y, uint32_t M, uint32_t K, int quant_act, mv_scratch* s) {
    mv_fmt(OC_Q8_0, W, x, y, M, K, quant_act, s);
}

void oc_matvec_act_q8_0(const void* W, const float* x, float* y, uint32_t M, uint32_t K, int quant_act) {
    mv_scratch s = mv_alloc(K);
    mv((const uint8_t*)W, x, y, M, K, quant_act, &s);
    mv_free(&s);
}

void oc_matvec_act(int fmt, const void* W, const float* x, float* y, uint32_t M, uint32_t K, int quant_act) {
    mv_scratch s = mv_alloc(K);
    mv_fmt(fmt, (const uint8_t*)W, x, y, M, K, quant_act, &s);
    mv_free(&s);
}

/* Format of matrix `which` (0 w_qkv|w_z|w_ab, 1 w_out, 2 w_gate|w_up, 3
 * w_down) of layer l; l == n_layers: 0 lm_head, 1 the embedding. */
static int fmt_of(const oc_model_w* w, uint32_t l, int which) { return w->fmt ? w->fmt[4 * l + which] : OC_Q8_0; }

static int is_attn_layer(const oc_model_cfg* c, uint32_t l) {
    return c->attn_interval != 0 && ((l + 1) % c->attn_interval) == 0;
}

static int all_zero(const float* w, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) if (w[i] != 0.0f) return 0;
    return 1;
}

/* qwen_linear.forward (echo-core-zig/src/kernels/qwen_linear.zig:103-271) of
 * block l: projections :141-180, conv shift + conv + SiLU :182-201, q/k L2
 * norms :203-204, gates :215-219, delta rule :221-249 (oc_deltanet_step),
 * gated RMSNorm :252-257, out projection :260-270. */
void oc_deltanet_block(const oc_model_cfg* c, const oc_model_w* w, uint32_t l, float* conv_state, float* ssm_state,
                       const float* in, float* out, int quant_act) {
    const dims_t d = dims_of(c);
    mv_scratch s = mv_alloc(d.maxK);
    float* a = (float*)calloc(d.conv_dim, sizeof(float));
    float* b = (float*)calloc(d.conv_dim, sizeof(float));
    float* z = (float*)calloc(d.value_dim, sizeof(float));
    float* core = (float*)calloc(d.value_dim, sizeof(float));
    float* ab = (float*)calloc(2 * d.n_v, sizeof(float));
    float* dec = (float*)calloc(d.n_v, sizeof(float));
    float* bet = (float*)calloc(d.n_v, sizeof(float));
    const int fin = fmt_of(w, l, 0), fo = fmt_of(w, l, 1);
    mv_fmt(fin, w->w_qkv[l], in, a, d.conv_dim, d.H, quant_act, &s);
    mv_fmt(fin, w->w_z[l], in, z, d.value_dim, d.H, quant_act, &s);
    mv_fmt(fin, w->w_ab[l], in, ab, 2 * d.n_v, d.H, quant_act, &s);
    oc_conv_step(conv_state, a, w->conv_w[l], b, d.conv_dim, c->conv_kernel);
    oc_l2norm_heads(b, d.n_k, d.d_k);
    oc_l2norm_heads(b + d.key_dim, d.n_k, d.d_k);
    oc_deltanet_gates(ab, ab + d.n_v, w->a_log[l], w->dt_bias[l], dec, bet, d.n_v);
    oc_deltanet_step(ssm_state, b, b + d.key_dim, b + 2 * d.key_dim, dec, bet, core, d.n_v, d.n_k, d.d_k, d.d_v);
    oc_gated_rmsnorm(core, z, w->ssm_norm[l], d.n_v, d.d_v);
    mv_fmt(fo, w->w_out[l], core, out, d.H, d.value_dim, quant_act, &s);
    free(a); free(b); free(z); free(core); free(ab); free(dec); free(bet);
    mv_free(&s);
}

/* Attention block l (echo-core-zig/src/inference/engine.zig:520-621): fused
 * q|k|v projection :537-539, q/k head RMSNorm when the weight is not all zero
 * :548-553, RoPE at position pos :556-558, KV append before attending :561,
 * INT8 attention over pos+1 positions :563-616, output projection :619.  The
 * block attends over its own layer's cache length (the reference reads layer
 * 0's, cache.zig:131-134, which a hybrid stack never appends to). */
void oc_attention_block(const oc_model_cfg* c, const oc_model_w* w, uint32_t l, int8_t* keys, int8_t* vals,
                        float* kscales, float* vscales, uint32_t pos, const float* in, float* out, int quant_act) {
    const dims_t d = dims_of(c);
    mv_scratch s = mv_alloc(d.maxK);
    float* a = (float*)calloc(d.q_dim + 2 * d.kv_dim, sizeof(float));
    float* core = (float*)calloc(d.q_dim, sizeof(float));
    float* inv_freq = (float*)calloc(c->head_dim / 2 + 1, sizeof(float));
    oc_rope_inv_freq(inv_freq, c->head_dim, c->rope_base);
    mv_fmt(fmt_of(w, l, 0), w->w_qkv[l], in, a, d.q_dim + 2 * d.kv_dim, d.H, quant_act, &s);
    float* q = a;
    float* k = a + d.q_dim;
    float* v = a + d.q_dim + d.kv_dim;
    if (!all_zero(w->q_norm[l], c->head_dim)) oc_head_rmsnorm(q, w->q_norm[l], c->n_heads, c->head_dim);
    if (!all_zero(w->k_norm[l], c->head_dim)) oc_head_rmsnorm(k, w->k_norm[l], c->n_kv, c->head_dim);
    oc_rope(q, c->n_heads, c->head_dim, pos, inv_freq);
    oc_rope(k, c->n_kv, c->head_dim, pos, inv_freq);
    oc_kv_append(k, v, keys, vals, kscales, vscales, pos, c->n_kv, c->head_dim);
    oc_attn_decode_int8(q, keys, vals, kscales, vscales, core, c->n_heads, c->n_kv, c->head_dim, pos + 1);
    mv_fmt(fmt_of(w, l, 1), w->w_out[l], core, out, d.H, d.q_dim, quant_act, &s);
    free(a); free(core); free(inv_freq);
    mv_free(&s);
}

/* engine.zig:769-772: out[i] = silu(gate[i]) * up[i] (out may alias gate). */
void oc_swiglu(const float* gate, const float* up, float* out, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) out[i] = oc_silu(gate[i]) * up[i];
}

/* SwiGLU FFN of block l (echo-core-zig/src/inference/engine.zig:748-781):
 * out = W_down (silu(W_gate in) * (W_up in)). */
void oc_ffn_block(const oc_model_cfg* c, const oc_model_w* w, uint32_t l, const float* in, float* out,
                  int quant_act) {
    const dims_t d = dims_of(c);
    mv_scratch s = mv_alloc(d.maxK);
    float* g = (float*)calloc(c->ffn, sizeof(float));
    float* u = (float*)calloc(c->ffn, sizeof(float));
    const int fgu = fmt_of(w, l, 2);
    mv_fmt(fgu, w->w_gate[l], in, g, c->ffn, d.H, quant_act, &s);
    mv_fmt(fgu, w->w_up[l], in, u, c->ffn, d.H, quant_act, &s);
    oc_swiglu(g, u, g, c->ffn);
    mv_fmt(fmt_of(w, l, 3), w->w_down[l], g, out, d.H, c->ffn, quant_act, &s);
    free(g); free(u);
    mv_free(&s);
}

/* echo-core-zig/src/inference/engine.zig:360-389 (forwardToken) with
 * layerForward :397-463 (qwen_linear and attention blocks: residual + norm +
 * block, then residual + post-attention norm + FFN), final norm and the vocab
 * projection :375-385. */
void oc_decoder_token(const oc_model_cfg* c, const oc_model_w* w, oc_seq_state* st,
                      uint32_t token, float* logits, int quant_act) {
    const dims_t d = dims_of(c);
    const uint32_t H = d.H;
    float* x = (float*)calloc(H, sizeof(float));
    float* hbuf = (float*)calloc(H, sizeof(float));
    float* tmp = (float*)calloc(H, sizeof(float));
    mv_scratch s = mv_alloc(d.maxK);
    oc_embed_row(fmt_of(w, c->n_layers, 1), w->embed, H, token, x);
    for (uint32_t l = 0; l < c->n_layers; ++l) {
        oc_rmsnorm(x, w->attn_norm[l], hbuf, H);
        if (!is_attn_layer(c, l))
            oc_deltanet_block(c, w, l, st->conv_state[l], st->ssm_state[l], hbuf, tmp, quant_act);
        else
            oc_attention_block(c, w, l, st->keys[l], st->vals[l], st->kscales[l], st->vscales[l], st->pos, hbuf, tmp,
                               quant_act);
        for (uint32_t i = 0; i < H; ++i) x[i] = x[i] + tmp[i];
        oc_rmsnorm(x, w->ffn_norm[l], hbuf, H);
        oc_ffn_block(c, w, l, hbuf, tmp, quant_act);
        for (uint32_t i = 0; i < H; ++i) x[i] = x[i] + tmp[i];
    }
    oc_rmsnorm(x, w->final_norm, hbuf, H);
    mv_fmt(fmt_of(w, c->n_layers, 0), w->lm_head, hbuf, logits, c->vocab, H, quant_act, &s);
    st->pos += 1;
    free(x); free(hbuf); free(tmp);
    mv_free(&s);
}
