// glue.hip — the small per-token ops of the hybrid decode step, fused so that
// each produces exactly what the next matvec or recurrence consumes.
//
// Semantics follow the reference engine (echo-core-zig):
//   embedding row decode           inference/engine.zig:30-54 (Q8_0 branch)
//   RMSNorm                        engine.zig:783-792 (x * 1/sqrt(mean(x^2)+1e-6) * w)
//   conv shift + conv + SiLU       kernels/qwen_linear.zig:182-201 (tap-major weights)
//   L2 norm of q, k heads          qwen_linear.zig:87-101, :203-204
//   decay / beta gates             qwen_linear.zig:215-219, softplus :71-74
//   gated RMSNorm                  qwen_linear.zig:252-257
//   head RMSNorm, RoPE, KV append  engine.zig:507-518, :466-504, :556-561
//   SwiGLU                         engine.zig:748-781, core/math.zig:35-37
//   greedy argmax (first maximum)  engine.zig:860-867
// Every op that feeds a matvec quantizes its output per 32-element block with
// the reference quantizer directly into the matvec's activation layout
// (quant.hip header), token-major scales xd[slot][block].
//
// A sequence s is active when pos[s] >= 0; inactive sequences never touch
// their recurrent state, conv state or KV cache.
#include "gemm_act.hpp"

namespace ec {

// Block-wide sum over 256 threads (4 waves); every thread gets the total.
__device__ __forceinline__ float block_sum256(float v, float* sh) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    return sh[0] + sh[1] + sh[2] + sh[3];
}

__device__ __forceinline__ float block_max256(float v, float* sh) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}


// Quantize 32 values (one block) and store them into the Q8_0 activation
// layout for token slot i of an M-row activation buffer; scale to xd[i][sb].
__device__ __forceinline__ void store_block_q8(const float (&v)[32], uint8_t* act, uint32_t M, uint32_t i,
                                               uint32_t sb, uint32_t nbp, float* xd) {
    float amax = 0.0f;
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
    const float scale = q_scale(amax);
    const float inv = __fdiv_rn(1.0f, scale);
    const uint32_t G = sb / 4, j = sb % 4;
    for (int g = 0; g < 4; ++g) {
        uint32_t lo = 0, hi = 0;
        for (int e = 0; e < 4; ++e) lo |= (uint32_t)(uint8_t)q_body(v[8 * g + e], inv) << (8 * e);
        for (int e = 0; e < 4; ++e) hi |= (uint32_t)(uint8_t)q_body(v[8 * g + 4 + e], inv) << (8 * e);
        *(uint2*)(act + (((size_t)G * 4 + g) * M + i) * 32 + 8 * j) = make_uint2(lo, hi);
    }
    xd[(size_t)i * nbp + sb] = scale;
}

// ------------------------------------------------------------------ embedding
// grid (n_seq, ceil(H / 1024)), block 256: thread = 4 consecutive elements of
// one 34-byte block, all of its loads (scale, 4 quants) in one round trip
// after the token's (a workgroup per row looping over its blocks chained the
// load latencies: 6.9 -> 4.9 us on average over a decode benchmark's calls).
__global__ __launch_bounds__(256) void k_embed_q8_0(const uint8_t* __restrict__ emb, const int32_t* __restrict__ tok,
                                                    float* __restrict__ x, uint32_t H, uint32_t vocab) {
    const uint32_t s = blockIdx.x, q = blockIdx.y * 256 + threadIdx.x;
    if (4 * q >= H) return;
    int32_t t = tok[s];
    t = t < 0 ? 0 : (t >= (int32_t)vocab ? (int32_t)vocab - 1 : t);
    const uint8_t* bp = emb + ((size_t)t * (H / 32) + q / 8) * 34;
    const uint32_t o = 2 + 4 * (q % 8);
    const uint8_t b0 = bp[0], b1 = bp[1], v0 = bp[o], v1 = bp[o + 1], v2 = bp[o + 2], v3 = bp[o + 3];
    const float d = h2f((uint16_t)(b0 | (b1 << 8)));
    float* dst = x + (size_t)s * H + 4 * q;
    dst[0] = d * (float)(int8_t)v0;
    dst[1] = d * (float)(int8_t)v1;
    dst[2] = d * (float)(int8_t)v2;
    dst[3] = d * (float)(int8_t)v3;
}

// F16 / F32 embedding rows (engine.zig:30-54 reads fp16, f32 and Q8_0 tables).
template <typename T>
__global__ __launch_bounds__(256) void k_embed_rows(const T* __restrict__ emb, const int32_t* __restrict__ tok,
                                                    float* __restrict__ x, uint32_t H, uint32_t vocab) {
    const uint32_t s = blockIdx.x;
    int32_t t = tok[s];
    t = t < 0 ? 0 : (t >= (int32_t)vocab ? (int32_t)vocab - 1 : t);
    for (uint32_t i = threadIdx.x; i < H; i += 256) {
        if constexpr (sizeof(T) == 2) x[(size_t)s * H + i] = h2f(emb[(size_t)t * H + i]);
        else x[(size_t)s * H + i] = emb[(size_t)t * H + i];
    }
}

// ---------------------------------------------------------- RMSNorm + quantize
// grid (ceil(Kp/256), M), block 256: every block reads the whole row i of x
// [M][H] for the sum of squares (float4 loads, all issued before the
// reduction) and quantizes its own 256 elements into act (Q8_0 layout,
// K = H); thread = element, so each 32-lane half-wave quantizes one block.
__global__ __launch_bounds__(256) void k_rmsnorm_quant(const float* __restrict__ x, const float* __restrict__ w,
                                                       uint8_t* __restrict__ act, uint32_t M, uint32_t H,
                                                       uint32_t xd_off, uint32_t P) {
    __shared__ float sh[4];
    const uint32_t i = blockIdx.y, t = threadIdx.x, k = blockIdx.x * 256 + t;
    const float* xr = x + (size_t)i * H;
    const float4* x4 = (const float4*)xr;
    const uint32_t Kp = round_up(H, 128);
    const float xk = k < H ? xr[k] : 0.0f;
    const float wk = k < H ? w[k] : 0.0f;
    float ss = 0.0f;
    uint32_t c = t;
    for (; c + 3 * 256 < H / 4; c += 4 * 256) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = x4[c + 256 * u];
#pragma unroll
        for (int u = 0; u < 4; ++u) ss = fmaf(v[u].x, v[u].x, fmaf(v[u].y, v[u].y, fmaf(v[u].z, v[u].z, fmaf(v[u].w, v[u].w, ss))));
    }
    for (; c < H / 4; c += 256) {
        const float4 v = x4[c];
        ss = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
    }
    ss = block_sum256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)H + 1e-6f);
    if (k >= Kp) return;  // whole 32-lane blocks leave together
    store_act_q8_lane(xk * inv * wk, act, (float*)(act + xd_off), M, Kp / 32, i, k, P);
}

// Residual add of split-K partial sums fused with RMSNorm + quantize:
// x_out = ((x + parts[0]) + parts[1]) + ... (fixed order), then x_out's
// RMSNorm quantized like k_rmsnorm_quant.  Every block recomputes the whole row
// of x_out for the sum (the same operations in the same order as the element it
// writes), so blocks never read what another block writes; x_out != x.
// parts: [NP][M][H].  grid (ceil(Kp/256), M), thread = element.
template <int NP>
__global__ __launch_bounds__(256) void k_add_rmsnorm_quant(const float* __restrict__ x, const float* __restrict__ parts,
                                                           float* __restrict__ x_out, const float* __restrict__ w,
                                                           uint8_t* __restrict__ act, uint32_t M, uint32_t H,
                                                           uint32_t xd_off, uint32_t P) {
    __shared__ float sh[4];
    const uint32_t i = blockIdx.y, t = threadIdx.x, k = blockIdx.x * 256 + t;
    const size_t ps = (size_t)M * H;
    const float* xr = x + (size_t)i * H;
    const float* pr = parts + (size_t)i * H;
    const uint32_t Kp = round_up(H, 128);
    float xk = 0.0f;
    if (k < H) {
        float pk[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) pk[p] = pr[p * ps + k];
        xk = xr[k];
#pragma unroll
        for (int p = 0; p < NP; ++p) xk += pk[p];
    }
    const float wk = k < H ? w[k] : 0.0f;
    float ss = 0.0f;
    // the row's float4s, 1024 per pass with every load of a pass issued
    // before the first add (H = 2560: one pass)
    constexpr uint32_t U = 4;
    for (uint32_t c0 = 0; c0 < H / 4; c0 += 256 * U) {
        float4 v[U], pv[U][NP];
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            const uint32_t c = c0 + t + 256 * u;
            const bool ok = c < H / 4;
            v[u] = ok ? ((const float4*)xr)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int p = 0; p < NP; ++p) pv[u][p] = ok ? ((const float4*)(pr + p * ps))[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (uint32_t u = 0; u < U; ++u) {
            float4 a = v[u];
#pragma unroll
            for (int p = 0; p < NP; ++p) a.x += pv[u][p].x, a.y += pv[u][p].y, a.z += pv[u][p].z, a.w += pv[u][p].w;
            ss = fmaf(a.x, a.x, fmaf(a.y, a.y, fmaf(a.z, a.z, fmaf(a.w, a.w, ss))));
        }
    }
    ss = block_sum256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)H + 1e-6f);
    if (k >= Kp) return;  // whole 32-lane blocks leave together
    if (k < H) x_out[(size_t)i * H + k] = xk;
    store_act_q8_lane(xk * inv * wk, act, (float*)(act + xd_off), M, Kp / 32, i, k, P);
}

// Row variant: grid (M), block Kp/4 threads rounded up to whole waves (Kp <=
// 4096), thread = 4 consecutive elements (one float4 of x and of each
// partial); the row is read once.  Eight lanes form one Q8_0 block (max over
// 8 lanes), each stores its 4 quantized bytes (per piece) as one word; the
// threads past Kp/4 only add zeros to the sum.
template <int NP>
__global__ __launch_bounds__(1024) void k_add_rmsnorm_quant_row(const float* __restrict__ x,
                                                               const float* __restrict__ parts,
                                                               float* __restrict__ x_out, const float* __restrict__ w,
                                                               uint8_t* __restrict__ act, uint32_t M, uint32_t H,
                                                               uint32_t xd_off, uint32_t P) {
    __shared__ float sh[16];
    const uint32_t i = blockIdx.x, t = threadIdx.x, k = 4 * t, lane = t & 63, wv = t >> 6;
    const size_t ps = (size_t)M * H;
    const uint32_t Kp = round_up(H, 128), nbp = Kp / 32;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), wk = a;
    if (k < H) {
        float4 pv[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) pv[p] = *(const float4*)(parts + p * ps + (size_t)i * H + k);
        a = *(const float4*)(x + (size_t)i * H + k);
        wk = *(const float4*)(w + k);
#pragma unroll
        for (int p = 0; p < NP; ++p) a.x += pv[p].x, a.y += pv[p].y, a.z += pv[p].z, a.w += pv[p].w;
        *(float4*)(x_out + (size_t)i * H + k) = a;
    }
    float ss = fmaf(a.x, a.x, fmaf(a.y, a.y, fmaf(a.z, a.z, a.w * a.w)));
    ss = wave_sum(ss);
    if (lane == 0) sh[wv] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (uint32_t v = 0; v < blockDim.x / 64; ++v) tot += sh[v];
    const float inv = 1.0f / sqrtf(tot / (float)H + 1e-6f);
    if (k >= Kp) return;  // whole 8-lane blocks (Kp % 32 == 0)
    const float v0 = a.x * inv * wk.x, v1 = a.y * inv * wk.y, v2 = a.z * inv * wk.z, v3 = a.w * inv * wk.w;
    float amax = fmaxf(fmaxf(fabsf(v0), fabsf(v1)), fmaxf(fabsf(v2), fabsf(v3)));
    amax = fmaxf(amax, lane_xor<1>(amax));
    amax = fmaxf(amax, lane_xor<2>(amax));
    amax = fmaxf(amax, lane_xor<4>(amax));
    const float scale = q_scale(amax);
    const float iq = __fdiv_rn(1.0f, scale);
    const int8_t q0[4] = {q_body(v0, iq), q_body(v1, iq), q_body(v2, iq), q_body(v3, iq)};
    const uint32_t word = (uint32_t)(uint8_t)q0[0] | ((uint32_t)(uint8_t)q0[1] << 8) |
                          ((uint32_t)(uint8_t)q0[2] << 16) | ((uint32_t)(uint8_t)q0[3] << 24);
    const uint32_t sb = k / 32, e = k % 32, G = sb / 4, j = sb % 4;
    uint8_t* dst = act + (((size_t)G * 4 + e / 8) * (P * M) + P * i) * 32 + 8 * j + (e % 8);
    *(uint32_t*)dst = word;
    if (P == 2) {
        const uint32_t w1 = (uint32_t)(uint8_t)q_piece1(v0, q0[0], scale, iq) |
                            ((uint32_t)(uint8_t)q_piece1(v1, q0[1], scale, iq) << 8) |
                            ((uint32_t)(uint8_t)q_piece1(v2, q0[2], scale, iq) << 16) |
                            ((uint32_t)(uint8_t)q_piece1(v3, q0[3], scale, iq) << 24);
        *(uint32_t*)(dst + 32) = w1;
    }
    if (e == 0) ((float*)(act + xd_off))[(size_t)i * nbp + sb] = scale;
}

// ------------------------------------------------------- SwiGLU + quantize
// gu [M][2F] (gate rows then up rows) -> act (K = F).  grid (ceil(Kp/256), M),
// thread = element.
// NP > 1: gu holds NP partial sums [NP][M][2F] (a split-K matvec's output),
// added in part order.
template <int NP>
__global__ __launch_bounds__(256) void k_swiglu_quant(const float* __restrict__ gu, uint8_t* __restrict__ act,
                                                      uint32_t M, uint32_t F, uint32_t xd_off, uint32_t P) {
    const uint32_t Kp = round_up(F, 128);
    const uint32_t i = blockIdx.y, k = blockIdx.x * 256 + threadIdx.x;
    if (k >= Kp) return;  // whole 32-lane blocks leave together (Kp % 32 == 0)
    const float* g = gu + (size_t)i * 2 * F;
    const size_t ps = (size_t)M * 2 * F;
    float v = 0.0f;
    if (k < F) {
        float gp[NP], up[NP];
#pragma unroll
        for (int q = 0; q < NP; ++q) gp[q] = g[q * ps + k], up[q] = g[q * ps + F + k];
        float a = gp[0], b = up[0];
#pragma unroll
        for (int q = 1; q < NP; ++q) a += gp[q], b += up[q];
        v = silu(a) * b;
    }
    store_act_q8_lane(v, act, (float*)(act + xd_off), M, Kp / 32, i, k, P);
}

// ------------------------------------------------ delta-net conv + norms + gates
// grid (conv_dim/128, n_seq), block 128: one 128-channel head of the q, k or v
// region per block, thread = channel.  Conv state [n_seq][kern][conv_dim] is a
// ring over positions: slot p % kern holds the input of position p, so a step
// writes one slot and reads the kern-1 older ones (zero after reset).  q and k
// heads are L2-normalized; v heads also compute their decay / beta gates.
__global__ __launch_bounds__(128) void k_conv_gates(const float* __restrict__ proj, uint32_t Nin,
                                                    float* __restrict__ conv_state, const float* __restrict__ conv_w,
                                                    const float* __restrict__ a_log, const float* __restrict__ dt_bias,
                                                    float* __restrict__ q_out, float* __restrict__ k_out,
                                                    float* __restrict__ v_out, float* __restrict__ dec,
                                                    float* __restrict__ beta, const int32_t* __restrict__ pos,
                                                    uint32_t n_k, uint32_t n_v, uint32_t kern) {
    __shared__ float sh[2];
    const uint32_t hb = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    const int32_t p = pos[s];
    if (p < 0) return;
    const uint32_t key_dim = n_k * 128, value_dim = n_v * 128, conv_dim = 2 * key_dim + value_dim;
    const float* pr = proj + (size_t)s * Nin;
    float* st = conv_state + (size_t)s * kern * conv_dim;
    const uint32_t c = hb * 128 + i;
    const float xin = pr[c];
    const float a = silu(conv_ring(st, conv_w, xin, (uint32_t)p, kern, conv_dim, c));
    st[(size_t)((uint32_t)p % kern) * conv_dim + c] = xin;
    if (c >= 2 * key_dim) {  // v head
        const uint32_t h = hb - 2 * n_k;
        v_out[((size_t)s * n_v + h) * 128 + i] = a;
        if (i == 0) {
            const float al = pr[conv_dim + value_dim + h];
            const float br = pr[conv_dim + value_dim + n_v + h];
            const float sp_in = al + dt_bias[h];
            const float sp = sp_in > 20.0f ? sp_in : log1pf(expf(sp_in));
            const float g = -expf(a_log[h]) * sp;
            dec[(size_t)s * n_v + h] = expf(g);
            beta[(size_t)s * n_v + h] = 1.0f / (1.0f + expf(-br));
        }
        return;
    }
    // q or k head: L2 norm over its 128 channels (two waves)
    const float ss = wave_sum(a * a);
    if ((i & 63) == 0) sh[i >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((sh[0] + sh[1]) + 1e-6f);
    const bool is_q = c < key_dim;
    const uint32_t h = is_q ? hb : hb - n_k;
    (is_q ? q_out : k_out)[((size_t)s * n_k + h) * 128 + i] = a * inv;
}

// ------------------------------------- chunked prefill: conv + gates, T tokens
// One sequence, T consecutive tokens at positions p0 .. p0+T-1 (proj rows
// [T][Nin]).  grid (2*n_k + n_v, ceil(T / kConvTokensPerBlock)), block 128:
// kConvTokensPerBlock consecutive tokens of one 128-channel head (their shared
// taps come from L1), the same sums as k_conv_gates (conv_ring's tap order)
// with the taps of positions >= p0 read from earlier rows of the chunk and
// older ones from the ring.  The ring is updated afterwards by
// k_conv_ring_chunk (in the four-tap kernel by the token-group-0 workgroups
// themselves).  (One token per workgroup: 32768 two-wave workgroups for a
// 512-token chunk, 19.9 us.)
constexpr uint32_t kConvTokensPerBlock = 8;
// Four-tap case (the model's conv kernel): the 8 tokens' inputs and their 3
// earlier taps are loaded once into registers (11 loads per thread, all in
// flight), the 8 tokens computed together, one barrier for their L2 norms.
// The workgroups of token group 0 are the only readers of the ring: each then
// writes its channels' new ring slots (the chunk's last min(T, 4) inputs),
// after its taps have been used.
__global__ __launch_bounds__(128) void k_conv_gates_chunk4(const float* __restrict__ proj, uint32_t Nin,
                                                           float* ring,
                                                           const float* __restrict__ conv_w,
                                                           const float* __restrict__ a_log,
                                                           const float* __restrict__ dt_bias, float* __restrict__ q_out,
                                                           float* __restrict__ k_out, float* __restrict__ v_out,
                                                           float* __restrict__ dec, float* __restrict__ beta,
                                                           uint32_t T, uint32_t p0, uint32_t n_k, uint32_t n_v) {
    constexpr uint32_t KERN = 4, TPB = kConvTokensPerBlock;
    __shared__ float sh[TPB][2];
    const uint32_t hb = blockIdx.x, i = threadIdx.x;
    const uint32_t key_dim = n_k * 128, value_dim = n_v * 128, conv_dim = 2 * key_dim + value_dim;
    const uint32_t c = hb * 128 + i;
    const int32_t t0 = (int32_t)(blockIdx.y * TPB);
    // xs[j] = input of chunk row t0 - 3 + j (earlier positions from the ring, 0 before position 0)
    float xs[TPB + KERN - 1];
#pragma unroll
    for (int j = 0; j < (int)(TPB + KERN - 1); ++j) {
        const int32_t t = t0 - (int32_t)(KERN - 1) + j;
        float x = 0.0f;
        if (t >= 0) {
            if (t < (int32_t)T) x = proj[(size_t)t * Nin + c];
        } else if ((int32_t)p0 + t >= 0) {
            x = ring[(size_t)(((int32_t)p0 + t) % (int32_t)KERN) * conv_dim + c];
        }
        xs[j] = x;
    }
    float wv[KERN];
#pragma unroll
    for (int k = 0; k < (int)KERN; ++k) wv[k] = conv_w[(size_t)k * conv_dim + c];
    float a[TPB];
#pragma unroll
    for (int tt = 0; tt < (int)TPB; ++tt) {
        // the sum of k_conv_gates in its order: newest tap first
        float acc = __fmul_rn(xs[tt + KERN - 1], wv[KERN - 1]);
#pragma unroll
        for (int k = 1; k < (int)KERN; ++k) acc = fmaf(xs[tt + KERN - 1 - k], wv[KERN - 1 - k], acc);
        a[tt] = silu(acc);
    }
    if (blockIdx.y == 0) {
        for (uint32_t j = 0; j < min(T, KERN); ++j) {
            const uint32_t t = T - 1 - j;
            ring[(size_t)((p0 + t) % KERN) * conv_dim + c] = proj[(size_t)t * Nin + c];
        }
    }
    const uint32_t nt = min((uint32_t)TPB, T - (uint32_t)t0);
    if (c >= 2 * key_dim) {  // v head (the whole workgroup)
        const uint32_t h = hb - 2 * n_k;
#pragma unroll
        for (int tt = 0; tt < (int)TPB; ++tt)
            if ((uint32_t)tt < nt) v_out[((size_t)(t0 + tt) * n_v + h) * 128 + i] = a[tt];
        if (i < nt) {
            const float* pr = proj + (size_t)(t0 + i) * Nin;
            const float al = pr[conv_dim + value_dim + h];
            const float br = pr[conv_dim + value_dim + n_v + h];
            const float sp_in = al + dt_bias[h];
            const float sp = sp_in > 20.0f ? sp_in : log1pf(expf(sp_in));
            const float g = -expf(a_log[h]) * sp;
            dec[(size_t)(t0 + i) * n_v + h] = expf(g);
            beta[(size_t)(t0 + i) * n_v + h] = 1.0f / (1.0f + expf(-br));
        }
        return;
    }
#pragma unroll
    for (int tt = 0; tt < (int)TPB; ++tt) {
        const float ss = wave_sum(a[tt] * a[tt]);
        if ((i & 63) == 0) sh[tt][i >> 6] = ss;
    }
    __syncthreads();
    const bool is_q = c < key_dim;
    const uint32_t h = is_q ? hb : hb - n_k;
#pragma unroll
    for (int tt = 0; tt < (int)TPB; ++tt) {
        if ((uint32_t)tt >= nt) break;
        const float inv = 1.0f / sqrtf((sh[tt][0] + sh[tt][1]) + 1e-6f);
        (is_q ? q_out : k_out)[((size_t)(t0 + tt) * n_k + h) * 128 + i] = a[tt] * inv;
    }
}

// Any number of taps: one token per iteration.
__global__ __launch_bounds__(128) void k_conv_gates_chunk(const float* __restrict__ proj, uint32_t Nin,
                                                          const float* __restrict__ ring,
                                                          const float* __restrict__ conv_w,
                                                          const float* __restrict__ a_log,
                                                          const float* __restrict__ dt_bias, float* __restrict__ q_out,
                                                          float* __restrict__ k_out, float* __restrict__ v_out,
                                                          float* __restrict__ dec, float* __restrict__ beta,
                                                          uint32_t T, uint32_t p0, uint32_t n_k, uint32_t n_v,
                                                          uint32_t kern) {
    __shared__ float sh[2][2];  // per-wave sums of squares, alternating between tokens
    const uint32_t hb = blockIdx.x, i = threadIdx.x;
    const uint32_t key_dim = n_k * 128, value_dim = n_v * 128, conv_dim = 2 * key_dim + value_dim;
    const uint32_t c = hb * 128 + i;
    const uint32_t t_end = min((blockIdx.y + 1) * kConvTokensPerBlock, T);
    for (uint32_t t = blockIdx.y * kConvTokensPerBlock; t < t_end; ++t) {
        const float* pr = proj + (size_t)t * Nin;
        const uint32_t p = p0 + t;
        float acc = __fmul_rn(pr[c], conv_w[(size_t)(kern - 1) * conv_dim + c]);
        for (uint32_t k = 1; k < kern; ++k) {
            float x = 0.0f;
            if (k <= t) x = proj[(size_t)(t - k) * Nin + c];
            else if (k <= p) x = ring[(size_t)((p - k) % kern) * conv_dim + c];
            acc = fmaf(x, conv_w[(size_t)(kern - 1 - k) * conv_dim + c], acc);
        }
        const float a = silu(acc);
        if (c >= 2 * key_dim) {  // v head (the whole workgroup)
            const uint32_t h = hb - 2 * n_k;
            v_out[((size_t)t * n_v + h) * 128 + i] = a;
            if (i == 0) {
                const float al = pr[conv_dim + value_dim + h];
                const float br = pr[conv_dim + value_dim + n_v + h];
                const float sp_in = al + dt_bias[h];
                const float sp = sp_in > 20.0f ? sp_in : log1pf(expf(sp_in));
                const float g = -expf(a_log[h]) * sp;
                dec[(size_t)t * n_v + h] = expf(g);
                beta[(size_t)t * n_v + h] = 1.0f / (1.0f + expf(-br));
            }
            continue;
        }
        float* shb = sh[t & 1];
        const float ss = wave_sum(a * a);
        if ((i & 63) == 0) shb[i >> 6] = ss;
        __syncthreads();  // also orders this token's reads of sh[t & 1] before token t+2 rewrites it
        const float inv = 1.0f / sqrtf((shb[0] + shb[1]) + 1e-6f);
        const bool is_q = c < key_dim;
        const uint32_t h = is_q ? hb : hb - n_k;
        (is_q ? q_out : k_out)[((size_t)t * n_k + h) * 128 + i] = a * inv;
    }
}

// Ring update after a chunk: the inputs of the last min(T, kern) positions.
// grid (ceil(conv_dim/256), min(T, kern)), block 256.
__global__ __launch_bounds__(256) void k_conv_ring_chunk(const float* __restrict__ proj, uint32_t Nin,
                                                         float* __restrict__ ring, uint32_t conv_dim, uint32_t T,
                                                         uint32_t p0, uint32_t kern) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x;
    const uint32_t t = T - 1 - blockIdx.y;  // chunk row
    if (c >= conv_dim) return;
    ring[(size_t)((p0 + t) % kern) * conv_dim + c] = proj[(size_t)t * Nin + c];
}

// --------------------------------------------- fp32 row ops (chunked prefill)
// RMSNorm rows: y[i] = x[i] * 1/sqrt(mean(x[i]^2) + 1e-6) * w.  grid (M), block 256.
// Rows of H <= 4096 with H % 4 == 0 and 16-byte aligned rows: float4 loads
// kept in registers for the second pass (kRowRegs per thread); others scalar.
constexpr uint32_t kRowRegs = 4;
__global__ __launch_bounds__(256) void k_rmsnorm_rows(const float* __restrict__ x, const float* __restrict__ w,
                                                      float* __restrict__ y, uint32_t H) {
    __shared__ float sh[4];
    const uint32_t i = blockIdx.x, t = threadIdx.x;
    const float* xr = x + (size_t)i * H;
    float* yr = y + (size_t)i * H;
    const bool vec = H % 4 == 0 && H <= 1024 * kRowRegs && (((uintptr_t)xr | (uintptr_t)yr | (uintptr_t)w) & 15) == 0;
    if (vec) {
        const uint32_t n4 = H / 4;
        float4 v[kRowRegs];
        float ss = 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < kRowRegs; ++u) {
            const uint32_t k = t + 256 * u;
            v[u] = k < n4 ? ((const float4*)xr)[k] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (uint32_t u = 0; u < kRowRegs; ++u) {
            ss = fmaf(v[u].x, v[u].x, ss);
            ss = fmaf(v[u].y, v[u].y, ss);
            ss = fmaf(v[u].z, v[u].z, ss);
            ss = fmaf(v[u].w, v[u].w, ss);
        }
        ss = block_sum256(ss, sh);
        const float inv = 1.0f / sqrtf(ss / (float)H + 1e-6f);
#pragma unroll
        for (uint32_t u = 0; u < kRowRegs; ++u) {
            const uint32_t k = t + 256 * u;
            if (k < n4) {
                const float4 wv = ((const float4*)w)[k];
                ((float4*)yr)[k] = make_float4(v[u].x * inv * wv.x, v[u].y * inv * wv.y, v[u].z * inv * wv.z,
                                               v[u].w * inv * wv.w);
            }
        }
        return;
    }
    float ss = 0.0f;
    for (uint32_t k = t; k < H; k += 256) ss = fmaf(xr[k], xr[k], ss);
    ss = block_sum256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)H + 1e-6f);
    for (uint32_t k = t; k < H; k += 256) yr[k] = xr[k] * inv * w[k];
}

// SwiGLU rows: gu [M][2F] (gate | up) -> y [M][F].  grid (ceil(F/256), M).
__global__ __launch_bounds__(256) void k_swiglu_rows(const float* __restrict__ gu, float* __restrict__ y, uint32_t F) {
    const uint32_t i = blockIdx.y, k = blockIdx.x * 256 + threadIdx.x;
    if (k >= F) return;
    const float* g = gu + (size_t)i * 2 * F;
    y[(size_t)i * F + k] = silu(g[k]) * g[F + k];
}

// Gated RMSNorm rows: core [M][n_v][128] -> y [M][n_v*128] (k_gated_norm_quant's
// value before quantization).  grid (n_v, M), block 128.
__global__ __launch_bounds__(128) void k_gated_norm_rows(const float* __restrict__ core, const float* __restrict__ proj,
                                                         uint32_t Nin, uint32_t z_off, const float* __restrict__ norm_w,
                                                         float* __restrict__ y, uint32_t n_v) {
    __shared__ float sh[2];
    const uint32_t h = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    const float o = core[((size_t)s * n_v + h) * 128 + i];
    const float ss = wave_sum(o * o);
    if ((i & 63) == 0) sh[i >> 6] = ss;
    __syncthreads();
    const float rms = sqrtf((sh[0] + sh[1]) / 128.0f + 1e-6f);
    const float inv = 1.0f / rms;
    y[((size_t)s * n_v + h) * 128 + i] = o * inv * norm_w[i] * silu(proj[(size_t)s * Nin + z_off + h * 128 + i]);
}

// ------------------------------- prefill rows straight into the GEMM layout
// The _rows arithmetic above, quantized into the prefill GEMM's Q8_0
// activation layout (gemm_act.hpp) by the same quantizer as
// ec_gemm_quantize_act, so the bytes are those of _rows + quantize.  Padding
// tokens (M .. Mp) and blocks (K .. Kp) are written as the quantizer writes
// them.

// grid (Mp), block 256: k_rmsnorm_rows' float4 path (H % 32 == 0, Kp <= 4096).
__global__ __launch_bounds__(256) void k_rmsnorm_rows_gemm_act(const float* __restrict__ x,
                                                               const float* __restrict__ w, uint8_t* __restrict__ xt,
                                                               uint32_t M, uint32_t H, uint32_t nch, uint32_t nbp,
                                                               size_t xd_off) {
    __shared__ float sh[4];
    const uint32_t i = blockIdx.x, t = threadIdx.x;
    const bool real = i < M;
    const float4* xr = (const float4*)(x + (size_t)(real ? i : 0) * H);
    const uint32_t n4 = H / 4, nq = 8 * nbp;  // float4s of the row, of the padded row
    float4 v[kRowRegs];
    float ss = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kRowRegs; ++u) {
        const uint32_t k = t + 256 * u;
        v[u] = real && k < n4 ? xr[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (uint32_t u = 0; u < kRowRegs; ++u) {
        ss = fmaf(v[u].x, v[u].x, ss);
        ss = fmaf(v[u].y, v[u].y, ss);
        ss = fmaf(v[u].z, v[u].z, ss);
        ss = fmaf(v[u].w, v[u].w, ss);
    }
    ss = block_sum256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)H + 1e-6f);
#pragma unroll
    for (uint32_t u = 0; u < kRowRegs; ++u) {
        const uint32_t k = t + 256 * u;
        if (k >= nq) continue;  // whole 8-lane groups (nq % 8 == 0)
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        if (real && k < n4) {
            const float4 wv = ((const float4*)w)[k];
            y = make_float4(v[u].x * inv * wv.x, v[u].y * inv * wv.y, v[u].z * inv * wv.z, v[u].w * inv * wv.w);
        }
        xt_q8_store4(y, i, k, real, xt, nch, nbp, xd_off);
    }
}

// grid (ceil(8 nbp / 256), Mp), block 256: thread q -> elements 4q .. 4q+3.
__global__ __launch_bounds__(256) void k_swiglu_rows_gemm_act(const float* __restrict__ gu, uint8_t* __restrict__ xt,
                                                              uint32_t M, uint32_t F, uint32_t nch, uint32_t nbp,
                                                              size_t xd_off) {
    const uint32_t m = blockIdx.y, q = blockIdx.x * 256 + threadIdx.x;
    if (q >= 8 * nbp) return;  // whole 8-lane groups
    const bool real = m < M;
    float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
    if (real && 4 * q < F) {
        const float* g = gu + (size_t)m * 2 * F + 4 * q;
        const float4 a = *(const float4*)g, b = *(const float4*)(g + F);
        y = make_float4(silu(a.x) * b.x, silu(a.y) * b.y, silu(a.z) * b.z, silu(a.w) * b.w);
    }
    xt_q8_store4(y, m, q, real, xt, nch, nbp, xd_off);
}

// grid (n_v, Mp), block 128: k_gated_norm_rows; a head's 128 outputs are 4 blocks.
__global__ __launch_bounds__(128) void k_gated_norm_rows_gemm_act(const float* __restrict__ core,
                                                                  const float* __restrict__ proj, uint32_t Nin,
                                                                  uint32_t z_off, const float* __restrict__ norm_w,
                                                                  uint8_t* __restrict__ xt, uint32_t M, uint32_t n_v,
                                                                  uint32_t nch, uint32_t nbp, size_t xd_off) {
    __shared__ float sh[2];
    const uint32_t h = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    const bool real = s < M;
    const float o = real ? core[((size_t)s * n_v + h) * 128 + i] : 0.0f;
    const float ss = wave_sum(o * o);
    if ((i & 63) == 0) sh[i >> 6] = ss;
    __syncthreads();
    const float rms = sqrtf((sh[0] + sh[1]) / 128.0f + 1e-6f);
    const float inv = 1.0f / rms;
    const float val = real ? o * inv * norm_w[i] * silu(proj[(size_t)s * Nin + z_off + h * 128 + i]) : 0.0f;
    xt_q8_store1(val, s, h * 128 + i, real, xt, nch, nbp, xd_off);
}

// ------------------------------------------------ gated RMSNorm + quantize
// grid (n_v, M), block 128: core [M][n_v][128], z at proj[s][z_off + h*128 + i]
// -> act (K = n_v*128).  The head's 128 outputs are 4 whole 32-blocks.
__global__ __launch_bounds__(128) void k_gated_norm_quant(const float* __restrict__ core,
                                                          const float* __restrict__ proj, uint32_t Nin,
                                                          uint32_t z_off, const float* __restrict__ norm_w,
                                                          uint8_t* __restrict__ act, uint32_t M, uint32_t n_v,
                                                          uint32_t xd_off, uint32_t P) {
    __shared__ float sh[2];
    const uint32_t h = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
    const float o = core[((size_t)s * n_v + h) * 128 + i];
    float ss = wave_sum(o * o);
    if ((i & 63) == 0) sh[i >> 6] = ss;
    __syncthreads();
    const float rms = sqrtf((sh[0] + sh[1]) / 128.0f + 1e-6f);
    const float inv = 1.0f / rms;
    const float val = o * inv * norm_w[i] * silu(proj[(size_t)s * Nin + z_off + h * 128 + i]);
    store_act_q8_lane(val, act, (float*)(act + xd_off), M, n_v * 4, s, h * 128 + i, P);
}

// -------------------------------------------- head norm + RoPE + KV append
// grid (n_heads + 2*n_kv, n_seq), block = head_dim (256).  proj [n_seq][Nin]
// holds q | k | v.  Head kinds: q heads -> q_out (normed, rotated); k heads ->
// normed, rotated, quantized into the cache at pos; v heads -> quantized.
__global__ __launch_bounds__(256) void k_qk_rope_append(const float* __restrict__ proj, uint32_t Nin,
                                                        const float* __restrict__ q_norm,
                                                        const float* __restrict__ k_norm, int use_qn, int use_kn,
                                                        const float* __restrict__ inv_freq, const int32_t* pos,
                                                        float* __restrict__ q_out, uint8_t* __restrict__ qa,
                                                        float* __restrict__ qsc, int8_t* __restrict__ keys,
                                                        int8_t* __restrict__ vals, float* __restrict__ kscales,
                                                        float* __restrict__ vscales, int32_t* __restrict__ ctx,
                                                        uint64_t seq_stride, uint32_t max_ctx, uint32_t n_heads,
                                                        uint32_t n_kv, uint32_t nparts, size_t pstride) {
    __shared__ float sh[4];
    const uint32_t HD = 256;
    const uint32_t head = blockIdx.x, s = blockIdx.y, d = threadIdx.x;
    const float* pr = proj + (size_t)s * Nin;
    const bool is_q = head < n_heads, is_k = !is_q && head < n_heads + n_kv;
    const uint32_t off = is_q ? head * HD : (is_k ? n_heads * HD + (head - n_heads) * HD
                                                  : n_heads * HD + n_kv * HD + (head - n_heads - n_kv) * HD);
    // inputs first: none of these loads depends on the position
    const bool norm = (is_q && use_qn) || (is_k && use_kn);
    float pv[8];  // the projection's partial sums (nparts <= 8), added in part order
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) pv[i] = i < nparts ? pr[i * pstride + off + d] : 0.0f;
    float val = pv[0];
#pragma unroll
    for (uint32_t i = 1; i < 8; ++i)
        if (i < nparts) val += pv[i];
    const float nw = norm ? (is_q ? q_norm : k_norm)[d] : 1.0f;
    const float ifr = (is_q || is_k) ? inv_freq[d / 2] : 0.0f;
    const int32_t p = pos[s];
    if (head == 0 && d == 0) ctx[s] = (p >= 0 && (uint32_t)p < max_ctx) ? p + 1 : 0;
    if (p < 0 || (uint32_t)p >= max_ctx) return;
    if (norm) {
        const float ss = block_sum256(sq_rn(val), sh);
        const float inv = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
        val = val * inv * nw;
    }
    if (is_q || is_k) {
        const float other = lane_xor<1>(val);
        val = rope_pair(val, other, d, (float)p * ifr);
    }
    if (is_q) {
        if (qa) {
            store_q_pieces(val, block_max256(fabsf(val), sh), d, s, head, n_heads, n_kv, qa, qsc);
        } else {
            q_out[(size_t)s * n_heads * HD + head * HD + d] = val;
        }
        return;
    }
    const uint32_t kvh = is_k ? head - n_heads : head - n_heads - n_kv;
    const float amax = block_max256(fabsf(val), sh);
    const float scale = q_scale(amax);
    const float inv = __fdiv_rn(1.0f, scale);
    int8_t* dst = (is_k ? keys : vals) + s * seq_stride + ((size_t)p * n_kv + kvh) * HD;
    dst[d] = q_body(val, inv);
    if (d == 0) (is_k ? kscales : vscales)[s * (seq_stride / HD) + (size_t)p * n_kv + kvh] = scale;
}

// ----------------------------------------------------------------- argmax
// First index of the maximum over l[lo, hi) (engine.zig:860-867): a value is
// taken when strictly greater than the best so far, so NaN never is and ties
// keep the lower index; thread 0 of the 1024-thread workgroup gets (best, bi),
// bi = 0x7FFFFFFF when nothing was taken.  lo is a multiple of 4.
__device__ __forceinline__ void argmax_range(const float* __restrict__ l, uint32_t lo, uint32_t hi, float& best,
                                             int32_t& bi, float* sv, int32_t* si) {
    const uint32_t t = threadIdx.x;
    best = -INFINITY;
    bi = 0x7FFFFFFF;
    // strictly greater keeps the first index among equal values within a thread
    // (its indices only grow); the reductions below break ties by index
    auto take = [&](float v, uint32_t k) {
        if (v > best) {
            best = v;
            bi = (int32_t)k;
        }
    };
    if ((((uintptr_t)(l + lo)) & 15) == 0) {
        const uint32_t n4 = (hi - lo) / 4;
        const float4* l4 = (const float4*)(l + lo);
        uint32_t k = t;
        for (; k + 3 * 1024 < n4; k += 4 * 1024) {
            float4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = l4[k + u * 1024];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t b = lo + 4 * (k + u * 1024);
                take(v[u].x, b), take(v[u].y, b + 1), take(v[u].z, b + 2), take(v[u].w, b + 3);
            }
        }
        for (; k < n4; k += 1024) {
            const float4 v = l4[k];
            const uint32_t b = lo + 4 * k;
            take(v.x, b), take(v.y, b + 1), take(v.z, b + 2), take(v.w, b + 3);
        }
        for (uint32_t r = lo + 4 * n4 + t; r < hi; r += 1024) take(l[r], r);
    } else {
        for (uint32_t k = lo + t; k < hi; k += 1024) take(l[k], k);
    }
    auto merge = [&](float ov, int32_t oi) {
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    };
    merge(lane_xor<32>(best), lane_xor_i<32>(bi));
    merge(lane_xor<16>(best), lane_xor_i<16>(bi));
    merge(lane_xor<8>(best), lane_xor_i<8>(bi));
    merge(lane_xor<4>(best), lane_xor_i<4>(bi));
    merge(lane_xor<2>(best), lane_xor_i<2>(bi));
    merge(lane_xor<1>(best), lane_xor_i<1>(bi));
    if ((t & 63) == 0) {
        sv[t >> 6] = best;
        si[t >> 6] = bi;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 16; ++w)
            if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
                best = sv[w];
                bi = si[w];
            }
    }
}

// Write the pick of sequence s (nothing taken: token 0, as the reference's
// scan) and advance its position.
__device__ __forceinline__ void argmax_commit(int32_t bi, uint32_t s, int32_t* __restrict__ gen,
                                              int32_t* __restrict__ next, int32_t* __restrict__ pos,
                                              uint32_t max_pos) {
    if (bi == 0x7FFFFFFF) bi = 0;
    if (pos[s] >= 0) {
        gen[s] = bi;
        next[s] = bi;
        // a sequence whose next position would be past the cache ends here:
        // it becomes inactive (pos -1) instead of decoding without attention
        const int32_t np = pos[s] + 1;
        pos[s] = (max_pos != 0 && (uint32_t)np >= max_pos) ? -1 : np;
    }
}

// grid (n_seq), block 1024: the whole row per workgroup.  Active sequences
// write the token to gen and next and advance pos.
__global__ __launch_bounds__(1024) void k_argmax_advance(const float* __restrict__ logits, uint32_t vocab,
                                                         int32_t* __restrict__ gen, int32_t* __restrict__ next,
                                                         int32_t* __restrict__ pos, uint32_t max_pos) {
    __shared__ float sv[16];
    __shared__ int32_t si[16];
    const uint32_t s = blockIdx.x;
    float best;
    int32_t bi;
    argmax_range(logits + (size_t)s * vocab, 0, vocab, best, bi, sv, si);
    if (threadIdx.x == 0) argmax_commit(bi, s, gen, next, pos, max_pos);
}

// Two launches over more CUs: grid (nsl, n_seq), block 1024, slice z of row s
// (a multiple of 4 entries, the last one shorter) -> part[s * nsl + z] =
// (best, index); then k_argmax_finish, grid (n_seq), one wave: the slices'
// picks merged with the same rule (greater, or equal and a lower index).
__global__ __launch_bounds__(1024) void k_argmax_slices(const float* __restrict__ logits, uint32_t vocab,
                                                        uint32_t slice, float2* __restrict__ part) {
    __shared__ float sv[16];
    __shared__ int32_t si[16];
    const uint32_t z = blockIdx.x, s = blockIdx.y, nsl = gridDim.x;
    const uint32_t lo = min(z * slice, vocab), hi = min(lo + slice, vocab);
    float best;
    int32_t bi;
    argmax_range(logits + (size_t)s * vocab, lo, hi, best, bi, sv, si);
    if (threadIdx.x == 0) part[(size_t)s * nsl + z] = make_float2(best, __int_as_float(bi));
}

__global__ __launch_bounds__(64) void k_argmax_finish(const float2* __restrict__ part, uint32_t nsl,
                                                      int32_t* __restrict__ gen, int32_t* __restrict__ next,
                                                      int32_t* __restrict__ pos, uint32_t max_pos) {
    const uint32_t s = blockIdx.x, lane = threadIdx.x;
    float best = -INFINITY;
    int32_t bi = 0x7FFFFFFF;
    auto merge = [&](float ov, int32_t oi) {
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    };
    for (uint32_t z = lane; z < nsl; z += 64) {
        const float2 p = part[(size_t)s * nsl + z];
        merge(p.x, __float_as_int(p.y));
    }
    merge(lane_xor<32>(best), lane_xor_i<32>(bi));
    merge(lane_xor<16>(best), lane_xor_i<16>(bi));
    merge(lane_xor<8>(best), lane_xor_i<8>(bi));
    merge(lane_xor<4>(best), lane_xor_i<4>(bi));
    merge(lane_xor<2>(best), lane_xor_i<2>(bi));
    merge(lane_xor<1>(best), lane_xor_i<1>(bi));
    if (lane == 0) argmax_commit(bi, s, gen, next, pos, max_pos);
}

}  // namespace ec


using namespace ec;

#define EC_GLUE_LAUNCH(...)                        \
    do {                                           \
        hipLaunchKernelGGL(__VA_ARGS__);           \
        EC_CHECK_LAUNCH();                         \
        return EC_OK;                              \
    } while (0)

extern "C" int ec_glue_embed(const void* emb, const int32_t* tok, float* x, uint32_t n_seq, uint32_t H,
                             uint32_t vocab, void* stream) {
    if (!emb || !tok || !x || H % 32) return ec_set_error(EC_ERR_ARG, "ec_glue_embed: bad argument");
    if (n_seq == 0) return EC_OK;
    EC_GLUE_LAUNCH(k_embed_q8_0, dim3(n_seq, (H / 4 + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                   (const uint8_t*)emb, tok, x, H, vocab);
}

extern "C" int ec_glue_embed_fmt(int fmt, const void* emb, const int32_t* tok, float* x, uint32_t n_seq, uint32_t H,
                                 uint32_t vocab, void* stream) {
    if (fmt == EC_Q8_0) return ec_glue_embed(emb, tok, x, n_seq, H, vocab, stream);
    if (!emb || !tok || !x || (fmt != EC_F16 && fmt != EC_F32))
        return ec_set_error(EC_ERR_ARG, "ec_glue_embed_fmt: format must be Q8_0, F16 or F32");
    if (fmt == EC_F16)
        EC_GLUE_LAUNCH(k_embed_rows<uint16_t>, dim3(n_seq), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)emb,
                       tok, x, H, vocab);
    EC_GLUE_LAUNCH(k_embed_rows<float>, dim3(n_seq), dim3(256), 0, (hipStream_t)stream, (const float*)emb, tok, x, H,
                   vocab);
}

extern "C" int ec_glue_rmsnorm_quant_pieces(const float* x, const float* w, void* act, uint32_t M, uint32_t H,
                                            uint32_t pieces, void* stream) {
    if (!x || !w || !act || M == 0 || M > 16 || H % 32 || ((uintptr_t)x & 15) || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_glue_rmsnorm_quant: bad argument");
    const ActLayout L = act_layout(EC_Q8_0, pieces * M, H);
    EC_GLUE_LAUNCH(k_rmsnorm_quant, dim3((L.Kp + 255) / 256, M), dim3(256), 0, (hipStream_t)stream, x, w,
                   (uint8_t*)act, M, H, (uint32_t)L.xd_off, pieces);
}

extern "C" int ec_glue_rmsnorm_quant(const float* x, const float* w, void* act, uint32_t M, uint32_t H,
                                     void* stream) {
    return ec_glue_rmsnorm_quant_pieces(x, w, act, M, H, 1, stream);
}

extern "C" int ec_glue_add_rmsnorm_quant_pieces(const float* x, const float* parts, uint32_t nparts, float* x_out,
                                                const float* w, void* act, uint32_t M, uint32_t H, uint32_t pieces,
                                                void* stream) {
    if (!x || !parts || !x_out || !w || !act || x == x_out || M == 0 || M > 16 || H % 32 || nparts == 0 ||
        nparts > 8 || ((uintptr_t)x & 15) || ((uintptr_t)parts & 15) || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_glue_add_rmsnorm_quant: bad argument");
    const uint32_t P = pieces;
    const ActLayout L = act_layout(EC_Q8_0, P * M, H);
    const dim3 grid((L.Kp + 255) / 256, M);
    const hipStream_t st = (hipStream_t)stream;
    uint8_t* a = (uint8_t*)act;
    const uint32_t xo = (uint32_t)L.xd_off;
    // one workgroup per row where it fits (rows up to 4096, 16-byte aligned rows): 2560-wide rows
    // 3.9 -> ~3.5 us per call in the decode step; otherwise row-parallel blocks
    if (nparts <= 4 && L.Kp <= 4096 && H % 4 == 0 && ((uintptr_t)x_out & 15) == 0 && ((uintptr_t)w & 15) == 0) {
        const dim3 g1(M), b1(round_up(L.Kp / 4, 64));  // whole waves: the sum adds every wave's part
        switch (nparts) {
            case 1: EC_GLUE_LAUNCH(k_add_rmsnorm_quant_row<1>, g1, b1, 0, st, x, parts, x_out, w, a, M, H, xo, P);
            case 2: EC_GLUE_LAUNCH(k_add_rmsnorm_quant_row<2>, g1, b1, 0, st, x, parts, x_out, w, a, M, H, xo, P);
            case 3: EC_GLUE_LAUNCH(k_add_rmsnorm_quant_row<3>, g1, b1, 0, st, x, parts, x_out, w, a, M, H, xo, P);
            default: EC_GLUE_LAUNCH(k_add_rmsnorm_quant_row<4>, g1, b1, 0, st, x, parts, x_out, w, a, M, H, xo, P);
        }
    }
    switch (nparts) {
        case 1: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<1>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        case 2: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<2>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        case 3: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<3>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        case 4: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<4>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        case 5: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<5>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        case 6: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<6>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        case 7: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<7>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
        default: EC_GLUE_LAUNCH(k_add_rmsnorm_quant<8>, grid, dim3(256), 0, st, x, parts, x_out, w, a, M, H, xo, P);
    }
}

extern "C" int ec_glue_add_rmsnorm_quant(const float* x, const float* parts, uint32_t nparts, float* x_out,
                                         const float* w, void* act, uint32_t M, uint32_t H, void* stream) {
    return ec_glue_add_rmsnorm_quant_pieces(x, parts, nparts, x_out, w, act, M, H, 1, stream);
}

extern "C" int ec_glue_swiglu_quant_split_pieces(const float* gu, uint32_t nparts, void* act, uint32_t M,
                                                 uint32_t F, uint32_t pieces, void* stream) {
    if (!gu || !act || M == 0 || M > 16 || F % 32 || nparts == 0 || nparts > 8 || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_glue_swiglu_quant");
    const uint32_t P = pieces;
    const ActLayout L = act_layout(EC_Q8_0, P * M, F);
    const dim3 grid((L.Kp + 255) / 256, M);
    const hipStream_t st = (hipStream_t)stream;
    uint8_t* a = (uint8_t*)act;
    const uint32_t xo = (uint32_t)L.xd_off;
    switch (nparts) {
        case 1: EC_GLUE_LAUNCH(k_swiglu_quant<1>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        case 2: EC_GLUE_LAUNCH(k_swiglu_quant<2>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        case 3: EC_GLUE_LAUNCH(k_swiglu_quant<3>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        case 4: EC_GLUE_LAUNCH(k_swiglu_quant<4>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        case 5: EC_GLUE_LAUNCH(k_swiglu_quant<5>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        case 6: EC_GLUE_LAUNCH(k_swiglu_quant<6>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        case 7: EC_GLUE_LAUNCH(k_swiglu_quant<7>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
        default: EC_GLUE_LAUNCH(k_swiglu_quant<8>, grid, dim3(256), 0, st, gu, a, M, F, xo, P);
    }
}

extern "C" int ec_glue_swiglu_quant_split(const float* gu, uint32_t nparts, void* act, uint32_t M, uint32_t F,
                                          void* stream) {
    return ec_glue_swiglu_quant_split_pieces(gu, nparts, act, M, F, 1, stream);
}

extern "C" int ec_glue_swiglu_quant(const float* gu, void* act, uint32_t M, uint32_t F, void* stream) {
    return ec_glue_swiglu_quant_split(gu, 1, act, M, F, stream);
}

extern "C" int ec_glue_conv_gates(const float* proj, uint32_t Nin, float* conv_state, const float* conv_w,
                                  const float* a_log, const float* dt_bias, float* q, float* k, float* v, float* dec,
                                  float* beta, const int32_t* pos, uint32_t n_seq, uint32_t n_k, uint32_t n_v,
                                  uint32_t kern, void* stream) {
    if (!proj || !conv_state || !conv_w || !a_log || !dt_bias || !q || !k || !v || !dec || !beta || !pos ||
        n_k == 0 || n_v == 0 || kern == 0 || Nin < 2 * n_k * 128 + 2 * n_v * 128 + 2 * n_v)
        return ec_set_error(EC_ERR_ARG, "ec_glue_conv_gates: bad argument");
    EC_GLUE_LAUNCH(k_conv_gates, dim3(2 * n_k + n_v, n_seq), dim3(128), 0, (hipStream_t)stream, proj, Nin,
                   conv_state, conv_w, a_log, dt_bias, q, k, v, dec, beta, pos, n_k, n_v, kern);
}

extern "C" int ec_glue_conv_gates_chunk(const float* proj, uint32_t Nin, float* ring, const float* conv_w,
                                        const float* a_log, const float* dt_bias, float* q, float* k, float* v,
                                        float* dec, float* beta, uint32_t T, uint32_t p0, uint32_t n_k, uint32_t n_v,
                                        uint32_t kern, void* stream) {
    if (T == 0) return EC_OK;
    if (!proj || !ring || !conv_w || !a_log || !dt_bias || !q || !k || !v || !dec || !beta || n_k == 0 || n_v == 0 ||
        kern == 0 || Nin < 2 * n_k * 128 + 2 * n_v * 128 + 2 * n_v)
        return ec_set_error(EC_ERR_ARG, "ec_glue_conv_gates_chunk: bad argument");
    const uint32_t conv_dim = 2 * n_k * 128 + n_v * 128;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(2 * n_k + n_v, (T + kConvTokensPerBlock - 1) / kConvTokensPerBlock);
    if (kern == 4)  // updates the ring itself
        EC_GLUE_LAUNCH(k_conv_gates_chunk4, grid, dim3(128), 0, st, proj, Nin, ring, conv_w, a_log, dt_bias, q, k, v,
                       dec, beta, T, p0, n_k, n_v);
    hipLaunchKernelGGL(k_conv_gates_chunk, grid, dim3(128), 0, st, proj, Nin, ring, conv_w, a_log, dt_bias, q, k, v,
                       dec, beta, T, p0, n_k, n_v, kern);
    EC_CHECK_LAUNCH();
    EC_GLUE_LAUNCH(k_conv_ring_chunk, dim3((conv_dim + 255) / 256, T < kern ? T : kern), dim3(256), 0, st, proj, Nin,
                   ring, conv_dim, T, p0, kern);
}

extern "C" int ec_glue_rmsnorm_rows(const float* x, const float* w, float* y, uint32_t M, uint32_t H, void* stream) {
    if (M == 0) return EC_OK;
    if (!x || !w || !y || H == 0) return ec_set_error(EC_ERR_ARG, "ec_glue_rmsnorm_rows: bad argument");
    EC_GLUE_LAUNCH(k_rmsnorm_rows, dim3(M), dim3(256), 0, (hipStream_t)stream, x, w, y, H);
}

extern "C" int ec_glue_swiglu_rows(const float* gu, float* y, uint32_t M, uint32_t F, void* stream) {
    if (M == 0) return EC_OK;
    if (!gu || !y || F == 0) return ec_set_error(EC_ERR_ARG, "ec_glue_swiglu_rows: bad argument");
    EC_GLUE_LAUNCH(k_swiglu_rows, dim3((F + 255) / 256, M), dim3(256), 0, (hipStream_t)stream, gu, y, F);
}

extern "C" int ec_glue_gated_norm_rows(const float* core, const float* proj, uint32_t Nin, uint32_t z_off,
                                       const float* norm_w, float* y, uint32_t M, uint32_t n_v, void* stream) {
    if (M == 0) return EC_OK;
    if (!core || !proj || !norm_w || !y || n_v == 0) return ec_set_error(EC_ERR_ARG, "ec_glue_gated_norm_rows");
    EC_GLUE_LAUNCH(k_gated_norm_rows, dim3(n_v, M), dim3(128), 0, (hipStream_t)stream, core, proj, Nin, z_off, norm_w,
                   y, n_v);
}

extern "C" int ec_glue_rmsnorm_rows_gemm_act(const float* x, const float* w, void* act, uint32_t M, uint32_t H,
                                              void* stream) {
    if (M == 0) return EC_OK;
    const XtLayout L = xt_layout(EC_Q8_0, M, H);
    if (!x || !w || !act || H == 0 || H % 32 || L.Kp > 1024 * kRowRegs || ((uintptr_t)x | (uintptr_t)w) & 15)
        return ec_set_error(EC_ERR_ARG, "ec_glue_rmsnorm_rows_gemm_act: need H % 32 == 0, H <= 4096, 16-byte rows");
    EC_GLUE_LAUNCH(k_rmsnorm_rows_gemm_act, dim3(L.Mp), dim3(256), 0, (hipStream_t)stream, x, w, (uint8_t*)act, M, H,
                   L.nch, L.Kp / 32, L.xd_off);
}

extern "C" int ec_glue_swiglu_rows_gemm_act(const float* gu, void* act, uint32_t M, uint32_t F, void* stream) {
    if (M == 0) return EC_OK;
    if (!gu || !act || F == 0 || F % 32 || (uintptr_t)gu & 15)
        return ec_set_error(EC_ERR_ARG, "ec_glue_swiglu_rows_gemm_act: need F % 32 == 0, 16-byte rows");
    const XtLayout L = xt_layout(EC_Q8_0, M, F);
    const uint32_t nbp = L.Kp / 32;
    EC_GLUE_LAUNCH(k_swiglu_rows_gemm_act, dim3((8 * nbp + 255) / 256, L.Mp), dim3(256), 0, (hipStream_t)stream, gu,
                   (uint8_t*)act, M, F, L.nch, nbp, L.xd_off);
}

extern "C" int ec_glue_gated_norm_rows_gemm_act(const float* core, const float* proj, uint32_t Nin, uint32_t z_off,
                                                const float* norm_w, void* act, uint32_t M, uint32_t n_v,
                                                void* stream) {
    if (M == 0) return EC_OK;
    if (!core || !proj || !norm_w || !act || n_v == 0)
        return ec_set_error(EC_ERR_ARG, "ec_glue_gated_norm_rows_gemm_act: bad argument");
    const XtLayout L = xt_layout(EC_Q8_0, M, n_v * 128);
    EC_GLUE_LAUNCH(k_gated_norm_rows_gemm_act, dim3(n_v, L.Mp), dim3(128), 0, (hipStream_t)stream, core, proj, Nin,
                   z_off, norm_w, (uint8_t*)act, M, n_v, L.nch, L.Kp / 32, L.xd_off);
}

extern "C" int ec_glue_gated_norm_quant_pieces(const float* core, const float* proj, uint32_t Nin, uint32_t z_off,
                                               const float* norm_w, void* act, uint32_t M, uint32_t n_v,
                                               uint32_t pieces, void* stream) {
    if (!core || !proj || !norm_w || !act || M == 0 || M > 16 || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_glue_gated_norm");
    const ActLayout L = act_layout(EC_Q8_0, pieces * M, n_v * 128);
    EC_GLUE_LAUNCH(k_gated_norm_quant, dim3(n_v, M), dim3(128), 0, (hipStream_t)stream, core, proj, Nin, z_off,
                   norm_w, (uint8_t*)act, M, n_v, (uint32_t)L.xd_off, pieces);
}

extern "C" int ec_glue_gated_norm_quant(const float* core, const float* proj, uint32_t Nin, uint32_t z_off,
                                        const float* norm_w, void* act, uint32_t M, uint32_t n_v, void* stream) {
    return ec_glue_gated_norm_quant_pieces(core, proj, Nin, z_off, norm_w, act, M, n_v, 1, stream);
}

extern "C" int ec_glue_qk_rope_append_split(const float* proj, uint32_t nparts, uint32_t Nin, const float* q_norm,
                                            const float* k_norm,
                                      int use_qn, int use_kn, const float* inv_freq, const int32_t* pos, float* q_out,
                                      void* q_packed, float* q_scales, int8_t* keys, int8_t* vals, float* kscales,
                                      float* vscales, int32_t* ctx, uint32_t n_seq, uint64_t seq_stride,
                                      uint32_t max_ctx, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
                                      void* stream) {
    if (head_dim != 256) return ec_set_error(EC_ERR_UNSUPPORTED, "ec_glue_qk_rope_append: head_dim must be 256");
    if (!proj || nparts == 0 || nparts > 8 || !inv_freq || !pos || (!q_out && !(q_packed && q_scales)) || !keys ||
        !vals || !kscales ||
        !vscales || !ctx || n_kv == 0 || n_heads % n_kv ||
        (seq_stride != 0 && seq_stride < (uint64_t)max_ctx * n_kv * head_dim))
        return ec_set_error(EC_ERR_ARG, "ec_glue_qk_rope_append: bad argument");
    EC_GLUE_LAUNCH(k_qk_rope_append, dim3(n_heads + 2 * n_kv, n_seq), dim3(256), 0, (hipStream_t)stream, proj, Nin,
                   q_norm, k_norm, use_qn, use_kn, inv_freq, pos, q_out, (uint8_t*)q_packed, q_scales, keys, vals,
                   kscales, vscales, ctx, seq_stride, max_ctx, n_heads, n_kv, nparts, (size_t)n_seq * Nin);
}

extern "C" int ec_glue_qk_rope_append(const float* proj, uint32_t Nin, const float* q_norm, const float* k_norm,
                                      int use_qn, int use_kn, const float* inv_freq, const int32_t* pos, float* q_out,
                                      void* q_packed, float* q_scales, int8_t* keys, int8_t* vals, float* kscales,
                                      float* vscales, int32_t* ctx, uint32_t n_seq, uint64_t seq_stride,
                                      uint32_t max_ctx, uint32_t n_heads, uint32_t n_kv, uint32_t head_dim,
                                      void* stream) {
    return ec_glue_qk_rope_append_split(proj, 1, Nin, q_norm, k_norm, use_qn, use_kn, inv_freq, pos, q_out, q_packed,
                                        q_scales, keys, vals, kscales, vscales, ctx, n_seq, seq_stride, max_ctx,
                                        n_heads, n_kv, head_dim, stream);
}

extern "C" int ec_glue_argmax_advance_bounded(const float* logits, uint32_t vocab, int32_t* gen, int32_t* next,
                                              int32_t* pos, uint32_t n_seq, uint32_t max_pos, void* stream) {
    if (!logits || !gen || !next || !pos) return ec_set_error(EC_ERR_ARG, "ec_glue_argmax_advance: bad argument");
    EC_GLUE_LAUNCH(k_argmax_advance, dim3(n_seq), dim3(1024), 0, (hipStream_t)stream, logits, vocab, gen, next, pos,
                   max_pos);
}

extern "C" int ec_glue_argmax_advance(const float* logits, uint32_t vocab, int32_t* gen, int32_t* next, int32_t* pos,
                                      uint32_t n_seq, void* stream) {
    return ec_glue_argmax_advance_bounded(logits, vocab, gen, next, pos, n_seq, 0, stream);
}

extern "C" size_t ec_glue_argmax_ws_bytes(uint32_t n_seq, uint32_t slices) {
    return (size_t)n_seq * slices * sizeof(float2);
}

extern "C" int ec_glue_argmax_advance_sliced(const float* logits, uint32_t vocab, int32_t* gen, int32_t* next,
                                             int32_t* pos, uint32_t n_seq, uint32_t max_pos, uint32_t slices,
                                             void* ws, void* stream) {
    if (!logits || !gen || !next || !pos || !ws || slices == 0 || slices > 1024 || n_seq > 65535)
        return ec_set_error(EC_ERR_ARG, "ec_glue_argmax_advance_sliced: bad argument");
    if (n_seq == 0) return EC_OK;
    const uint32_t slice = ((vocab + slices - 1) / slices + 3) / 4 * 4;
    const hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_argmax_slices, dim3(slices, n_seq), dim3(1024), 0, st, logits, vocab, slice, (float2*)ws);
    EC_CHECK_LAUNCH();
    EC_GLUE_LAUNCH(k_argmax_finish, dim3(n_seq), dim3(64), 0, st, (const float2*)ws, slices, gen, next, pos, max_pos);
}
