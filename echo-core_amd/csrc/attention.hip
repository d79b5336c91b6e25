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
#include <atomic>

#include "common.hpp"
#include "layout.hpp"

namespace ec {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ long pack2(uint32_t lo, uint32_t hi) {
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

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

// ===================================================================== MFMA path
// head_dim 256.  QK^T runs on v_mfma_i32_16x16x32_i8.  q of each head is split
// into three int8 vectors, q ~ s0*Q0 + s1*Q1 + s2*Q2 with s0 = max|q|/127,
// s1 = s0/254, s2 = s1/254 (each piece quantizes the previous residual, so
// |q - approx| <= max|q|/16387064, below fp32 rounding of the dot products);
// the pieces occupy A rows g, G+g and 2G+g.  K stays int8 (B operand), every
// dot product is an exact int32 and
//   score = ks * (s0*dot0 + s1*dot1 + s2*dot2) / sqrt(256).
// One workgroup of four waves owns a 64-position (or 128-position) chunk of
// one kv head for all G query heads of its GQA group and writes one partial
// (max / sum / output) per head.  Wave w scores positions 16w .. 16w+15 (+64q)
// and stages their V rows in LDS, transposed to [dim][position]; wave g takes
// the softmax of head g over the chunk and splits probability x V row scale
// into three int8 pieces the same way; softmax(.)V then runs on the same MFMA,
// wave w producing dims 64w .. 64w+63 as exact int32 sums per piece.
//
// Packed q layout: layout.hpp (store_q_pieces).
constexpr uint32_t kChunk64 = 64;
constexpr uint32_t kRec64 = 260;  // partial record [m, l, -, -, o[256]] (16-byte aligned output)

// grid (n_heads, n_seq), block 256 (thread = dim): pack q [n_seq][n_heads][256].
__global__ __launch_bounds__(256) void k_pack_q(const float* __restrict__ q, uint8_t* __restrict__ qa,
                                                float* __restrict__ qsc, uint32_t n_heads, uint32_t n_kv) {
    __shared__ float mx[4];
    const uint32_t head = blockIdx.x, s = blockIdx.y, d = threadIdx.x;
    const float val = q[((size_t)s * n_heads + head) * 256 + d];
    const float a = wave_max(fabsf(val));
    if ((d & 63) == 0) mx[d >> 6] = a;
    __syncthreads();
    const float amax = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
    store_q_pieces(val, amax, d, s, head, n_heads, n_kv, qa, qsc);
}

// PQ: q arrives as fp32 [n_seq][n_heads][256] (qf) and the workgroup packs
// its G heads itself (into LDS that the scores reuse); otherwise qa / qsc hold
// the packed q.
template <int G, int CH, bool PQ>
__global__ __launch_bounds__(256) void k_attn_mfma(const uint8_t* __restrict__ qa, const float* __restrict__ qsc,
                                                   const float* __restrict__ qf,
                                                   const int8_t* __restrict__ keys, const int8_t* __restrict__ vals,
                                                   const float* __restrict__ kscales, const float* __restrict__ vscales,
                                                   const int32_t* __restrict__ ctx, uint64_t seq_stride, uint32_t n_kv,
                                                   uint32_t n_chunks_max, uint32_t max_ctx, float* __restrict__ ws) {
    static_assert(G == 1 || G == 2 || G == 4, "3G A rows must fit the 16 MFMA rows");
    static_assert(CH == 64 || CH == 128, "chunk of 64 or 128 positions");
    constexpr uint32_t HD = 256;
    constexpr uint32_t NR = kQPieces * G;  // A rows in use
    constexpr int NPW = CH / 64;           // 16-position groups per wave
    // per-piece scores (times the K row scale); PQ: packed q first.  Rows
    // padded by 4 floats: the score stores (lane = row 4*gq + c, position
    // 16*wv + r16) then fall in 64 distinct banks instead of 16.
    __shared__ float part_s[NR][CH + 4];
    // probability pieces, A rows 4g + piece, rows padded by 8 bytes so the
    // PV operand reads (lane = row r16, 8 bytes at 8*gq) hit distinct banks
    // (unpadded: 4-way at 64 positions, 8-way at 128)
    constexpr uint32_t PAS = CH + 8;
    __shared__ uint32_t pA_w[4 * G * PAS / 4];
    __shared__ float qsc_s[PQ ? NR : 1];
    __shared__ float qmx_s[PQ ? G : 1][4];
    // the chunk's V transposed, [dim][position slots]: a dword holds 4 positions
    // (slot s = 16q + 4w + r: positions 64q + 16w + r + 4e, e = 0..3), rows
    // padded by one dword
    constexpr uint32_t RS = CH / 4 + 1;
    __shared__ uint32_t vT[256 * RS];
    __shared__ float psc_s[4][4];          // per head: scales of the probability pieces
    const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int32_t L = min(ctx[s], (int32_t)max_ctx);
    const uint32_t c0 = chunk * CH;
    if (L <= 0 || c0 >= (uint32_t)L) return;
    const uint32_t ntok = min((uint32_t)L - c0, (uint32_t)CH);
    const uint32_t n_heads = n_kv * G;
    const size_t row = (size_t)n_kv * HD;
    const int8_t* kb = keys + s * seq_stride + (size_t)kvh * HD;
    const int8_t* vb = vals + s * seq_stride + (size_t)kvh * HD;
    const float* ksb = kscales + s * (seq_stride / HD) + kvh;
    const float* vsb = vscales + s * (seq_stride / HD) + kvh;
    const uint32_t r16 = lane & 15, gq = lane >> 4;

    // ---- loads, in the order they are consumed (waitcnt retires them in order):
    // A operand (packed q) and scales, K of this wave's 16-position groups
    // (group q: positions 64q + 16*wv ..), then their V.
    const bool arow = r16 < NR;
    u32x4 aq[4];
    float rs[4];  // scale of the A row of each C element this lane holds
    float qv[G];  // PQ: dim tid of each head of the group
    if constexpr (!PQ) {
        const uint8_t* qp = qa + ((((size_t)s * n_kv + kvh) * NR + (arow ? r16 : 0)) * 4 + gq) * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) aq[i] = *(const u32x4*)(qp + 16 * i);
        const float* scq = qsc + ((size_t)s * n_kv + kvh) * NR;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t r = 4 * gq + c;
            rs[c] = scq[r < NR ? r : 0];
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) qv[g] = qf[((size_t)s * n_heads + kvh + n_kv * g) * HD + tid];
    }
    float ksv[NPW], vsv[NPW];
    u32x4 kw[NPW][4];
#pragma unroll
    for (int q = 0; q < NPW; ++q) {
        const uint32_t t = 64 * q + 16 * wv + r16;  // position of this lane's B column
        const uint32_t tc = t < ntok ? t : 0;
        ksv[q] = ksb[(size_t)(c0 + tc) * n_kv];
        const uint32_t tl = 64 * q + lane;  // used by wave 0 (lane = position)
        vsv[q] = vsb[(size_t)(c0 + (tl < ntok ? tl : 0)) * n_kv];
        const int8_t* kr = kb + (size_t)(c0 + tc) * row + 16 * gq;
#pragma unroll
        for (int i = 0; i < 4; ++i) kw[q][i] = __builtin_nontemporal_load((const u32x4*)(kr + 64 * i));
    }
    // V: instruction (q, j) brings positions 64q + 16*wv + 4j .. +3 (256 bytes each, lane = 16 bytes)
    u32x4 vv[NPW][4];
#pragma unroll
    for (int q = 0; q < NPW; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t tv = 64 * q + 16 * wv + 4 * j + (lane >> 4);
            vv[q][j] = __builtin_nontemporal_load(
                (const u32x4*)(vb + (size_t)(c0 + (tv < ntok ? tv : 0)) * row + 16 * (lane & 15)));
        }

    if constexpr (PQ) {
        // pack q (its loads were issued before K and V), then take the A operand from LDS
        uint8_t* qa_s = (uint8_t*)&part_s[0][0];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float m = wave_max(fabsf(qv[g]));
            if (lane == 0) qmx_s[g][wv] = m;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float amax = fmaxf(fmaxf(qmx_s[g][0], qmx_s[g][1]), fmaxf(qmx_s[g][2], qmx_s[g][3]));
            pack_q_pieces(qv[g], amax, tid, g, G, qa_s, qsc_s);
        }
        __syncthreads();
        const uint8_t* qp = qa_s + ((arow ? r16 : 0) * 4 + gq) * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) aq[i] = *(const u32x4*)(qp + 16 * i);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t r = 4 * gq + c;
            rs[c] = qsc_s[r < NR ? r : 0];
        }
        __syncthreads();  // part_s is written below
    }

    // ---- scores of 16 positions per group: 8 accumulating MFMAs; C row r = 4*gq + c
#pragma unroll
    for (int q = 0; q < NPW; ++q) {
        v4i C = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const long A = arow ? ((m & 1) ? pack2(aq[m / 2].z, aq[m / 2].w) : pack2(aq[m / 2].x, aq[m / 2].y)) : 0l;
            const u32x4 w = kw[q][m / 2];
            const long B = (m & 1) ? pack2(w.z, w.w) : pack2(w.x, w.y);
            C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, C, 0, 0, 0);
        }
        const uint32_t t = 64 * q + 16 * wv + r16;
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (4 * gq + c < NR) part_s[4 * gq + c][t] = (float)C[c] * rs[c] * ksv[q];
        // V: dword c of the lane's 16 bytes for positions +0, +4, +8, +12 (loads
        // j = 0..3) -> four dims x those positions (4x4 byte transpose)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t w0 = vv[q][0][c], w1 = vv[q][1][c], w2 = vv[q][2][c], w3 = vv[q][3][c];
            const uint32_t a0 = __builtin_amdgcn_perm(w1, w0, 0x05010400u), a1 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);
            const uint32_t b0 = __builtin_amdgcn_perm(w3, w2, 0x05010400u), b1 = __builtin_amdgcn_perm(w3, w2, 0x07030602u);
            const uint32_t tb[4] = {__builtin_amdgcn_perm(b0, a0, 0x05040100u), __builtin_amdgcn_perm(b0, a0, 0x07060302u),
                                    __builtin_amdgcn_perm(b1, a1, 0x05040100u), __builtin_amdgcn_perm(b1, a1, 0x07060302u)};
            const uint32_t slot = 16 * q + 4 * wv + gq;
#pragma unroll
            for (int b = 0; b < 4; ++b) vT[(16 * r16 + 4 * c + b) * RS + slot] = tb[b];
        }
    }
    __syncthreads();

    // ---- softmax over the chunk: wave g takes head g (lane = positions lane
    // + 64q); it reads score rows g, G+g, 2G+g and writes its probability
    // pieces over row g only, so the waves touch disjoint rows
    constexpr float scale = 1.0f / 16.0f;  // 1/sqrt(256)
    if (wv < (uint32_t)G) {
        const uint32_t g = wv;
        float sc[NPW], pr[NPW], mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < NPW; ++q) {
            const uint32_t tl = 64 * q + lane;
            const float raw = (part_s[g][tl] + part_s[G + g][tl]) + part_s[2 * G + g][tl];
            sc[q] = tl < ntok ? raw * scale : -INFINITY;
            mx = fmaxf(mx, sc[q]);
        }
        const float m = wave_max(mx);
        float es = 0.0f;
#pragma unroll
        for (int q = 0; q < NPW; ++q) {
            const float e = 64 * q + lane < ntok ? __expf(sc[q] - m) : 0.0f;
            es += e;
            pr[q] = e * vsv[q];
        }
        const float l = wave_sum(es);
        // probabilities x V row scale as three int8 pieces (as q): A rows
        // 4g + piece of pA, bytes in the slot order of vT
        uint8_t* pA = (uint8_t*)pA_w;
        const uint32_t rr = lane & 15;
        float pm = 0.0f;
#pragma unroll
        for (int q = 0; q < NPW; ++q) pm = fmaxf(pm, pr[q]);
        pm = wave_max(pm);
#pragma unroll
        for (int q = 0; q < NPW; ++q) {
            const uint32_t byte = 4 * (16 * q + 4 * (lane >> 4) + (rr & 3)) + (rr >> 2);
            int8_t pcs[kQPieces];
            float steps[kQPieces];
            split_pieces(pr[q], pm, pcs, steps);
#pragma unroll
            for (uint32_t pc = 0; pc < kQPieces; ++pc) {
                pA[(4 * g + pc) * PAS + byte] = (uint8_t)pcs[pc];
                if (lane == 0 && q == 0) psc_s[g][pc] = steps[pc];
            }
        }
        if (lane == 0) {
            float* rec = ws + (((size_t)s * n_chunks_max + chunk) * n_heads + kvh + n_kv * g) * kRec64;
            *(float4*)rec = make_float4(m, l, 0.0f, 0.0f);
        }
    }
    __syncthreads();

    // ---- softmax . V on v_mfma_i32_16x16x32_i8: A = the probability pieces (row
    // 4g + piece), B = vT (wave wv: dims 64wv .. +63, four 16-dim tiles), K =
    // positions in slot order; C element e of lane group g is piece e of head
    // g, exact int32.  Positions past the chunk end carry p = 0.
    const uint8_t* pA = (const uint8_t*)pA_w;
    v4i Cv[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (uint32_t ks = 0; ks < CH / 32; ++ks) {
        // rows 4G .. 15 feed only C rows that are not stored: read row 0 there
        const uint32_t* ap = (const uint32_t*)(pA + (r16 < 4 * G ? r16 : 0) * PAS + 32 * ks + 8 * gq);
        const long A = pack2(ap[0], ap[1]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t* bp = vT + (64 * wv + 16 * t + r16) * RS + 8 * ks + 2 * gq;
            Cv[t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, pack2(bp[0], bp[1]), Cv[t], 0, 0, 0);
        }
    }
    if (gq < (uint32_t)G) {
        const float s0 = psc_s[gq][0], s1 = psc_s[gq][1], s2 = psc_s[gq][2];
        float* rec = ws + (((size_t)s * n_chunks_max + chunk) * n_heads + kvh + n_kv * gq) * kRec64;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            rec[4 + 64 * wv + 16 * t + r16] = (s0 * (float)Cv[t][0] + s1 * (float)Cv[t][1]) + s2 * (float)Cv[t][2];
    }
}

// grid (n_heads, n_seq, DS), block 1024 (16 waves): merge chunk partials.  The
// chunk weights exp(m_c - M) go through LDS; workgroup z covers dims
// [256/DS*z, 256/DS*(z+1)) with lane = 4 dims, so one wave load brings the
// slice of DS chunk records (1 KB); wave w sums chunks DS*(w + 16i) + lane
// group, and the wave sums are added in LDS.  DS = 4 when the heads and
// sequences alone give few workgroups (one long sequence: every workgroup
// otherwise streams 1 KB per chunk through one CU).  (16 waves instead of 8:
// 32k-position context 38.7 -> 34.4 us.)
constexpr uint32_t kMergeWaves = 16;
constexpr uint32_t kMergeThreads = 64 * kMergeWaves;
constexpr uint32_t kMergeRegs = 8;  // chunk records per wave loaded per batch (the first with the maxima)

// With act != nullptr the merged rows are also quantized into the Q8_0
// activation layout (M = n_seq rows, K = n_heads*256, P pieces;
// quantize_act's format).
template <int DS>
__global__ __launch_bounds__(kMergeThreads) void k_attn_merge(const float* __restrict__ ws, const int32_t* __restrict__ ctx,
                                                    float* __restrict__ out, uint8_t* __restrict__ act,
                                                    uint32_t act_xd_off, uint32_t n_seq, uint32_t n_heads,
                                                    uint32_t n_chunks_max,
                                                    uint32_t max_ctx, uint32_t chunk, uint32_t P) {
    static_assert(DS == 1 || DS == 2 || DS == 4, "dim slices of 256, 128 or 64");
    constexpr uint32_t HD = 256, SD = HD / DS, LPR = 64 / DS;  // slice dims, lanes per record
    extern __shared__ float w_s[];
    __shared__ float red[kMergeWaves];
    __shared__ float4 acc_s[kMergeWaves][64];
    const uint32_t h = blockIdx.x, s = blockIdx.y, z = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t sub = lane / LPR, d4 = lane % LPR;  // record within the wave load, 4-dim group in the slice
    const int32_t L = min(ctx[s], (int32_t)max_ctx);
    float* dst = out + ((size_t)s * n_heads + h) * HD + SD * z;
    if (L <= 0) {
        if (tid < SD) {
            dst[tid] = 0.0f;
            if (act)
                store_act_q8_lane(0.0f, act, (float*)(act + act_xd_off), n_seq, n_heads * HD / 32, s,
                                  h * HD + SD * z + tid, P);
        }
        return;
    }
    const uint32_t nc = ((uint32_t)L + chunk - 1) / chunk;
    const float* base = ws + ((size_t)s * n_chunks_max * n_heads + h) * kRec64;
    const size_t cs = (size_t)n_heads * kRec64;
    const uint32_t doff = 4 + SD * z + 4 * d4;  // this lane's 4 dims in a record
    // the partial outputs of this lane's first kMergeRegs chunks are loaded
    // together with the chunk maxima, before any reduction
    float4 ov[kMergeRegs];
#pragma unroll
    for (int i = 0; i < (int)kMergeRegs; ++i) {
        const uint32_t c = DS * (wv + kMergeWaves * i) + sub;
        ov[i] = c < nc ? *(const float4*)(base + c * cs + doff) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    float M = -INFINITY;
    for (uint32_t c = tid; c < nc; c += kMergeThreads) M = fmaxf(M, base[c * cs]);
    M = wave_max(M);
    if (lane == 0) red[wv] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int i = 1; i < (int)kMergeWaves; ++i) M = fmaxf(M, red[i]);
    __syncthreads();
    float den = 0.0f;
    for (uint32_t c = tid; c < nc; c += kMergeThreads) {
        const float w = __expf(base[c * cs] - M);
        w_s[c] = w;
        den = fmaf(w, base[c * cs + 1], den);
    }
    den = wave_sum(den);
    if (lane == 0) red[wv] = den;
    __syncthreads();
    auto add = [](float4& a, float w, const float4& o) {
        a.x = fmaf(w, o.x, a.x), a.y = fmaf(w, o.y, a.y), a.z = fmaf(w, o.z, a.z), a.w = fmaf(w, o.w, a.w);
    };
    // chunks in order i = 0, 1, ...: the first kMergeRegs from registers
    float4 a0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < (int)kMergeRegs; ++i) {
        const uint32_t c = DS * (wv + kMergeWaves * i) + sub;
        if (c < nc) add(a0, w_s[c], ov[i]);
    }
    // longer contexts: the rest in batches of kMergeRegs records, all loads of a
    // batch in flight before its first add (same order of additions)
    for (uint32_t i0 = kMergeRegs; DS * (wv + kMergeWaves * i0) < nc; i0 += kMergeRegs) {
        float4 ob[kMergeRegs];
#pragma unroll
        for (int i = 0; i < (int)kMergeRegs; ++i) {
            const uint32_t c = DS * (wv + kMergeWaves * (i0 + i)) + sub;
            ob[i] = c < nc ? *(const float4*)(base + c * cs + doff) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int i = 0; i < (int)kMergeRegs; ++i) {
            const uint32_t c = DS * (wv + kMergeWaves * (i0 + i)) + sub;
            if (c < nc) add(a0, w_s[c], ob[i]);
        }
    }
    acc_s[wv][lane] = a0;
    __syncthreads();
    if (tid < SD) {
        float dn = red[0], o = 0.0f;
#pragma unroll
        for (int i = 1; i < (int)kMergeWaves; ++i) dn += red[i];
        // dim tid of the slice: float tid of each record group's 64-float run
        const float* col = (const float*)acc_s + tid;
#pragma unroll
        for (int i = 0; i < (int)kMergeWaves; ++i)
#pragma unroll
            for (int r = 0; r < DS; ++r) o += col[i * 256 + r * SD];
        o = o / dn;
        dst[tid] = o;
        if (act)
            store_act_q8_lane(o, act, (float*)(act + act_xd_off), n_seq, n_heads * HD / 32, s, h * HD + SD * z + tid,
                              P);
    }
}

// ----------------------------------------------------------- VALU fallback
template <int HD, int G>
static void launch_attn(const float* q, const int8_t* keys, const int8_t* vals, const float* ks, const float* vs,
                        float* out, const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride, uint32_t n_kv,
                        uint32_t ncm, uint32_t max_ctx, float* ws, hipStream_t st) {
    hipLaunchKernelGGL((k_attn_partial<HD, G>), dim3(ncm, n_kv, n_seq), dim3(64), 0, st, q, keys, vals, ks, vs, ctx,
                       seq_stride, n_kv, ncm, max_ctx, ws);
    hipLaunchKernelGGL((k_attn_combine<HD>), dim3(n_kv * G, n_seq), dim3(64), 0, st, ws, ctx, out, n_kv * G, ncm,
                       max_ctx);
}


// Positions per attention workgroup: 64, or 128 once 64-position chunks
// would need more workgroups than the GPU holds at once (~2048 at 7 waves per
// SIMD).  Measured on MI355X (16 heads / 4 kv heads): one sequence of 32768
// positions 34.2 -> 28.1 us with 128; 512 and 4096 positions 11.0 / 12.3 us
// with 64 vs 12.6 / 13.5 with 128.
static uint32_t attn_chunk(uint32_t max_ctx, uint32_t n_kv, uint32_t n_seq) {
    const uint64_t wgs64 = (uint64_t)((max_ctx + 63) / 64) * n_kv * n_seq;
    return wgs64 >= 2048 ? 128u : 64u;
}

template <int G>
static void launch_mfma(const uint8_t* qa, const float* qsc, const float* qf, const int8_t* keys, const int8_t* vals,
                        const float* ks,
                        const float* vs, float* out, uint8_t* act, const int32_t* ctx, uint32_t n_seq,
                        uint64_t seq_stride, uint32_t n_kv, uint32_t max_ctx, float* ws, hipStream_t st, uint32_t P) {
    const uint32_t CH = attn_chunk(max_ctx, n_kv, n_seq);
    const uint32_t ncm = (max_ctx + CH - 1) / CH;
    const dim3 grid(ncm, n_kv, n_seq);
    if (qf && CH == 128)
        hipLaunchKernelGGL((k_attn_mfma<G, 128, true>), grid, dim3(256), 0, st, qa, qsc, qf, keys, vals, ks, vs, ctx,
                           seq_stride, n_kv, ncm, max_ctx, ws);
    else if (qf)
        hipLaunchKernelGGL((k_attn_mfma<G, 64, true>), grid, dim3(256), 0, st, qa, qsc, qf, keys, vals, ks, vs, ctx,
                           seq_stride, n_kv, ncm, max_ctx, ws);
    else if (CH == 128)
        hipLaunchKernelGGL((k_attn_mfma<G, 128, false>), grid, dim3(256), 0, st, qa, qsc, qf, keys, vals, ks, vs, ctx,
                           seq_stride, n_kv, ncm, max_ctx, ws);
    else
        hipLaunchKernelGGL((k_attn_mfma<G, 64, false>), grid, dim3(256), 0, st, qa, qsc, qf, keys, vals, ks, vs, ctx,
                           seq_stride, n_kv, ncm, max_ctx, ws);
    const uint32_t xd_off = (uint32_t)act_layout(EC_Q8_0, P * n_seq, n_kv * G * 256).xd_off;
    // few (head, sequence) pairs: four workgroups per pair, 64 dims each
    if (n_kv * G * n_seq <= 32)
        hipLaunchKernelGGL(k_attn_merge<4>, dim3(n_kv * G, n_seq, 4), dim3(kMergeThreads), ncm * sizeof(float), st, ws,
                           ctx, out, act, xd_off, n_seq, n_kv * G, ncm, max_ctx, CH, P);
    else
        hipLaunchKernelGGL(k_attn_merge<1>, dim3(n_kv * G, n_seq), dim3(kMergeThreads), ncm * sizeof(float), st, ws,
                           ctx, out, act, xd_off, n_seq, n_kv * G, ncm, max_ctx, CH, P);
}

static int mfma_dispatch(uint32_t G, const uint8_t* qa, const float* qsc, const float* qf, const int8_t* keys,
                         const int8_t* vals,
                         const float* ks, const float* vs, float* out, uint8_t* act, const int32_t* ctx,
                         uint32_t n_seq, uint64_t seq_stride, uint32_t n_kv, uint32_t max_ctx, float* ws,
                         hipStream_t st, uint32_t P = 1) {
#define EC_MF(G_) launch_mfma<G_>(qa, qsc, qf, keys, vals, ks, vs, out, act, ctx, n_seq, seq_stride, n_kv, max_ctx, ws, st, P)
    switch (G) {
        case 1: EC_MF(1); break;
        case 2: EC_MF(2); break;
        case 4: EC_MF(4); break;
        default: return ec_set_error(EC_ERR_UNSUPPORTED, "packed attention: n_heads/n_kv must be 1, 2 or 4");
    }
#undef EC_MF
    return EC_OK;
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
    // partial records for the smallest chunk (64 positions), then packed q and its scales
    const size_t ncm = (max_ctx + kChunk64 - 1) / kChunk64;
    const size_t part = (size_t)n_seq * (ncm ? ncm : 1) * n_heads * (head_dim + 4) * sizeof(float);
    return ((part + 255) & ~(size_t)255) + qa_bytes(n_seq, n_heads) + (size_t)n_seq * n_heads * kQPieces * sizeof(float);
}

extern "C" int ec_attn_decode(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                              const float* vscales, float* out, const int32_t* ctx, uint32_t n_seq,
                              uint64_t seq_stride, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
                              uint32_t max_ctx, void* ws, void* stream) {
    if (n_seq == 0) return EC_OK;
    if (!q || !keys || !vals || !kscales || !vscales || !out || !ctx || !ws || n_kv == 0 || n_heads % n_kv ||
        max_ctx == 0 || (seq_stride != 0 && seq_stride < (uint64_t)max_ctx * n_kv * head_dim))
        return ec_set_error(EC_ERR_ARG, "ec_attn_decode: bad argument");
    const uint32_t G = n_heads / n_kv;
    const uint32_t ncm = (max_ctx + kAttnChunk - 1) / kAttnChunk;
    hipStream_t st = (hipStream_t)stream;
    float* w = (float*)ws;
    if (head_dim == 256 && (G == 1 || G == 2 || G == 4)) {
        const size_t part = (size_t)n_seq * ((max_ctx + kChunk64 - 1) / kChunk64) * n_heads * kRec64 * 4;
        uint8_t* qa = (uint8_t*)ws + ((part + 255) & ~(size_t)255);
        float* qsc = (float*)(qa + qa_bytes(n_seq, n_heads));
        // few sequences: each attention workgroup packs its own query heads (no
        // separate pass); many (prefill tokens): one packing pass, so that the
        // chunk workgroups of a token do not all repeat it
        const bool own = n_seq <= 16;
        if (!own) hipLaunchKernelGGL(k_pack_q, dim3(n_heads, n_seq), dim3(256), 0, st, q, qa, qsc, n_heads, n_kv);
        int rc = mfma_dispatch(G, qa, qsc, own ? q : nullptr, keys, vals, kscales, vscales, out, nullptr, ctx, n_seq,
                               seq_stride, n_kv, max_ctx, w, st);
        if (rc) return rc;
        EC_CHECK_LAUNCH();
        return EC_OK;
    }
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

extern "C" int ec_attn_decode_packed_pieces(const void* qa, const float* qsc, const int8_t* keys,
                                            const int8_t* vals, const float* kscales, const float* vscales, float* out,
                                            void* act_q8, const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride,
                                            uint32_t n_heads, uint32_t n_kv, uint32_t max_ctx, uint32_t pieces,
                                            void* ws, void* stream) {
    if (n_seq == 0) return EC_OK;
    if (!qa || !qsc || !keys || !vals || !kscales || !vscales || !out || !ctx || !ws || n_kv == 0 ||
        n_heads % n_kv || max_ctx == 0 || (seq_stride != 0 && seq_stride < (uint64_t)max_ctx * n_kv * 256) ||
        (act_q8 && n_seq > 16) || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_attn_decode_packed: bad argument");
    int rc = mfma_dispatch(n_heads / n_kv, (const uint8_t*)qa, qsc, nullptr, keys, vals, kscales, vscales, out,
                           (uint8_t*)act_q8, ctx, n_seq, seq_stride, n_kv, max_ctx, (float*)ws, (hipStream_t)stream,
                           pieces);
    if (rc) return rc;
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_attn_decode_packed(const void* qa, const float* qsc, const int8_t* keys, const int8_t* vals,
                                     const float* kscales, const float* vscales, float* out, void* act_q8,
                                     const int32_t* ctx, uint32_t n_seq, uint64_t seq_stride, uint32_t n_heads,
                                     uint32_t n_kv, uint32_t max_ctx, void* ws, void* stream) {
    return ec_attn_decode_packed_pieces(qa, qsc, keys, vals, kscales, vscales, out, act_q8, ctx, n_seq, seq_stride,
                                        n_heads, n_kv, max_ctx, 1, ws, stream);
}

extern "C" size_t ec_attn_qa_bytes(uint32_t n_seq, uint32_t n_heads) { return qa_bytes(n_seq, n_heads); }

// ------------------------------------------------ attention without allocation
// ec_attn_decode_noalloc runs ec_attn_decode with its workspace in `scratch`, a
// fixed device array that every GPU the library runs on holds until the
// process ends.  In host code `scratch` names a host-side stand-in, so its
// device address is looked up once per device (hipGetSymbolAddress, with that
// device current) and only that address is passed to kernels.
namespace {
constexpr size_t kScratchBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kScratchBytes];
std::atomic<void*> g_scratch[kMaxDevices];

int scratch_for_device(int dev, void** out) {
    if (dev < 0 || dev >= kMaxDevices) return ec_set_error(EC_ERR_ARG, "attention scratch: device index >= 64");
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return ec_set_hip_error(e, "attention scratch: hipGetSymbolAddress");
        g_scratch[dev].store(p, std::memory_order_release);  // a concurrent lookup stores the same address
    }
    *out = p;
    return EC_OK;
}
}  // namespace

// Called by ec_device_init with `device` current.
extern "C" int ec_attn_scratch_init(int device) {
    void* p = nullptr;
    return scratch_for_device(device, &p);
}

extern "C" size_t ec_attn_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" int ec_attn_decode_noalloc(const float* q, const int8_t* keys, const int8_t* vals, const float* kscales,
                                      const float* vscales, float* out, const int32_t* ctx, uint32_t n_seq,
                                      uint64_t seq_stride, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
                                      uint32_t max_ctx, void* stream) {
    if (n_seq == 0) return EC_OK;
    const size_t need = ec_attn_ws_bytes(n_seq, n_heads, head_dim, max_ctx);
    if (need > kScratchBytes) {
        char buf[192];
        snprintf(buf, sizeof buf,
                 "ec_attn_decode_noalloc: workspace of %zu bytes (n_seq %u, n_heads %u, max_ctx %u) exceeds the "
                 "fixed %zu-byte scratch; use ec_attn_decode with a caller workspace",
                 need, n_seq, n_heads, max_ctx, kScratchBytes);
        return ec_set_error(EC_ERR_ARG, buf);
    }
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ec_set_hip_error(e, "ec_attn_decode_noalloc: hipGetDevice");
    void* ws = nullptr;
    const int rc = scratch_for_device(dev, &ws);
    if (rc) return rc;
    return ec_attn_decode(q, keys, vals, kscales, vscales, out, ctx, n_seq, seq_stride, n_heads, n_kv, head_dim,
                          max_ctx, ws, stream);
}
