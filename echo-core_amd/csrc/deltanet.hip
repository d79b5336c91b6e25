// deltanet.hip — gated delta-rule recurrence (gfx950).
//
// Per value head h and token (echo-core-zig/src/kernels/qwen_linear.zig:207-250):
//   S <- decay*S;  kv = S^T k;  delta = (v - kv)*beta;  S <- S + k (x) delta;
//   o = S^T (q/sqrt(d_k))
// Every value channel (column) of S evolves independently given (q, k, decay,
// beta), so the work splits into n_seq*n_v*d_v columns of d_k = 128 floats.
// The state is stored per head TRANSPOSED relative to the reference, S[v][k],
// so one column is 512 contiguous bytes.  A DPP row of 16 lanes owns one
// column, 8 k-entries per lane in VGPRs.  The multi-token kernel takes both
// column dots of a token (S.k and S.q) from the state before its update and
// reduces them together with 4 DPP adds each inside the row (no LDS, no
// barrier): o = (decay*S.q + delta*(k.q))/sqrt(d_k) equals S'^T q/sqrt(d_k)
// for the updated S', so one reduction latency per token.  A wave holds 4
// columns (2 KB of state, two 16-byte loads per lane), a 256-thread workgroup
// 16 columns of one head.  Across the T tokens of one launch the state never
// leaves the VGPRs; the inputs (which do not depend on the recurrence) are
// staged through LDS in double-buffered blocks of 32 tokens.
#include "common.hpp"
#include "layout.hpp"

namespace ec {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Token blocks of kDnBlock tokens: the workgroup's 256 threads load the next
// block's q, k (one 128-float head each per token), the group's 16 v channels,
// decay and beta with coalesced loads into registers while the current block
// is computed from LDS, then store them into the other LDS buffer (double
// buffering).  The per-token recurrence never waits on global memory.
constexpr uint32_t kDnBlock = 32;

struct DnLds {
    f32x4 q[2][kDnBlock][32], k[2][kDnBlock][32];
    float v[2][kDnBlock][16];
    float dec[2][kDnBlock], bt[2][kDnBlock], kq[2][kDnBlock];
    float kk[2][kDnBlock / 2], kqx[2][kDnBlock / 2];  // token pair (2m, 2m+1): k_2m.k_2m+1, k_2m.q_2m+1
};

// grid (n_v * d_v/16, n_seq), block 256: threadIdx/16 = column in the group, %16 = k slice.
__global__ __launch_bounds__(256) void k_deltanet(float* __restrict__ state, const float* __restrict__ q,
                                                  const float* __restrict__ k, const float* __restrict__ v,
                                                  const float* __restrict__ decay, const float* __restrict__ beta,
                                                  float* __restrict__ out, uint32_t T, uint32_t n_seq, uint32_t n_v,
                                                  uint32_t n_k, uint32_t d_v, const int32_t* __restrict__ seq_pos) {
    __shared__ DnLds L;
    const uint32_t groups = d_v / 16;
    const uint32_t h = blockIdx.x / groups, s = blockIdx.y;
    if (seq_pos && seq_pos[s] < 0) return;
    const uint32_t row = threadIdx.x / 16, ks = threadIdx.x % 16;
    const uint32_t col0 = 16 * (blockIdx.x % groups), col = col0 + row;
    const uint32_t qh = h / (n_v / n_k);
    const float scale = 1.0f / sqrtf(128.0f);
    float* sp = state + (((size_t)s * n_v + h) * d_v + col) * 128 + 8 * ks;
    float4 s0 = *(float4*)sp, s1 = *(float4*)(sp + 4);
    float S[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};

    // staging registers of the next block (256 threads: 32 float4 of q and of
    // k per token, 16 v channels per token, decay / beta)
    constexpr uint32_t NQ = kDnBlock / 8, NV = kDnBlock * 16 / 256;
    f32x4 rq[NQ], rk[NQ];  // ext_vector_type: arrays of it stay in registers
    float rv[NV], rdb;
    const uint32_t tid = threadIdx.x;
    auto stage_load = [&](uint32_t t0) {
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t u = 0; u < NQ; ++u) {
            const uint32_t id = tid + 256 * u, t = t0 + id / 32;
            const size_t off = (((size_t)t * n_seq + s) * n_k + qh) * 128 + 4 * (id % 32);
            rq[u] = t < T ? *(const f32x4*)(q + off) : z;
            rk[u] = t < T ? *(const f32x4*)(k + off) : z;
        }
#pragma unroll
        for (uint32_t u = 0; u < NV; ++u) {
            const uint32_t id = tid + 256 * u, t = t0 + id / 16;
            rv[u] = t < T ? v[(((size_t)t * n_seq + s) * n_v + h) * d_v + col0 + id % 16] : 0.0f;
        }
        const uint32_t t = t0 + tid % kDnBlock;
        const size_t hv = ((size_t)t * n_seq + s) * n_v + h;
        rdb = (tid < 2 * kDnBlock && t < T) ? (tid < kDnBlock ? decay[hv] : beta[hv]) : 0.0f;
    };
    // also k.q of each token (32 lanes hold one token's q and k): the output
    // needs it, and it does not depend on the state
    auto stage_store = [&](uint32_t buf) {
#pragma unroll
        for (uint32_t u = 0; u < NQ; ++u) {
            const uint32_t id = tid + 256 * u;
            L.q[buf][id / 32][id % 32] = rq[u];
            L.k[buf][id / 32][id % 32] = rk[u];
            float kq = rq[u].x * rk[u].x + rq[u].y * rk[u].y + rq[u].z * rk[u].z + rq[u].w * rk[u].w;
            kq += lane_xor<1>(kq);
            kq += lane_xor<2>(kq);
            kq += lane_xor<4>(kq);
            kq += lane_xor<8>(kq);
            kq += lane_xor<16>(kq);
            if (id % 32 == 0) L.kq[buf][id / 32] = kq;
            // the pair's cross dots: token 2m's lanes take token 2m+1's k and q
            // from 32 lanes up (tokens 2m, 2m+1 share a wave)
            f32x4 nk, nq;
            nk.x = lane_xor<32>(rk[u].x), nk.y = lane_xor<32>(rk[u].y), nk.z = lane_xor<32>(rk[u].z),
            nk.w = lane_xor<32>(rk[u].w);
            nq.x = lane_xor<32>(rq[u].x), nq.y = lane_xor<32>(rq[u].y), nq.z = lane_xor<32>(rq[u].z),
            nq.w = lane_xor<32>(rq[u].w);
            float kk = rk[u].x * nk.x + rk[u].y * nk.y + rk[u].z * nk.z + rk[u].w * nk.w;
            float kx = rk[u].x * nq.x + rk[u].y * nq.y + rk[u].z * nq.z + rk[u].w * nq.w;
            kk += lane_xor<1>(kk), kx += lane_xor<1>(kx);
            kk += lane_xor<2>(kk), kx += lane_xor<2>(kx);
            kk += lane_xor<4>(kk), kx += lane_xor<4>(kx);
            kk += lane_xor<8>(kk), kx += lane_xor<8>(kx);
            kk += lane_xor<16>(kk), kx += lane_xor<16>(kx);
            if (id % 64 == 0) {
                L.kk[buf][id / 64] = kk;
                L.kqx[buf][id / 64] = kx;
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < NV; ++u) {
            const uint32_t id = tid + 256 * u;
            L.v[buf][id / 16][id % 16] = rv[u];
        }
        if (tid < kDnBlock) L.dec[buf][tid] = rdb;
        else if (tid < 2 * kDnBlock) L.bt[buf][tid - kDnBlock] = rdb;
    };

    stage_load(0);
    stage_store(0);
    __syncthreads();
    const uint32_t nb = (T + kDnBlock - 1) / kDnBlock;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint32_t buf = b & 1, t0 = b * kDnBlock;
        stage_load(t0 + kDnBlock);  // past T: zeros, no memory access
        const uint32_t nt = min(kDnBlock, T - t0);
        // Per token, both column dots come from the state before the update:
        //   a = S.k, b = S.q  (one pair of row reductions),
        //   kv = dec*a, delta = (v - kv)*beta,
        //   o = (dec*S + k delta).q/sqrt(128) = (dec*b + delta*(k.q))/sqrt(128),
        //   S <- dec*S + k delta.
        // Token j+1's operands are read from LDS while token j is computed (two
        // register sets used in turn).
        struct Ops {
            f32x4 k0, k1, q0, q1;
            float vv, dec, bt, kq;
        };
        auto read_ops = [&](uint32_t j) {
            Ops o;
            o.k0 = L.k[buf][j][2 * ks], o.k1 = L.k[buf][j][2 * ks + 1];
            o.q0 = L.q[buf][j][2 * ks], o.q1 = L.q[buf][j][2 * ks + 1];
            o.vv = L.v[buf][j][row], o.dec = L.dec[buf][j], o.bt = L.bt[buf][j], o.kq = L.kq[buf][j];
            return o;
        };
        auto token = [&](const Ops& x, uint32_t j) {
            const float kk[8] = {x.k0.x, x.k0.y, x.k0.z, x.k0.w, x.k1.x, x.k1.y, x.k1.z, x.k1.w};
            const float qq[8] = {x.q0.x, x.q0.y, x.q0.z, x.q0.w, x.q1.x, x.q1.y, x.q1.z, x.q1.w};
            float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a0 = fmaf(S[i], kk[i], a0);
                b0 = fmaf(S[i], qq[i], b0);
                a1 = fmaf(S[4 + i], kk[4 + i], a1);
                b1 = fmaf(S[4 + i], qq[4 + i], b1);
            }
            float a = a0 + a1, bq = b0 + b1;
            a += lane_xor<1>(a);
            bq += lane_xor<1>(bq);
            a += lane_xor<2>(a);
            bq += lane_xor<2>(bq);
            a += lane_xor<4>(a);
            bq += lane_xor<4>(bq);
            a += lane_xor<8>(a);
            bq += lane_xor<8>(bq);
            const float delta = (x.vv - x.dec * a) * x.bt;
            const float o = (x.dec * bq + delta * x.kq) * scale;
#pragma unroll
            for (int i = 0; i < 8; ++i) S[i] = fmaf(kk[i], delta, S[i] * x.dec);
            if (ks == 0) out[(((size_t)(t0 + j) * n_seq + s) * n_v + h) * d_v + col] = o;
        };
        // Two tokens per step (1 = j, 2 = j+1), all four column dots from the
        // state before both updates (one set of row reductions per pair):
        //   a1 = S.k1, b1 = S.q1, c = S.k2, e = S.q2
        //   delta1 = (v1 - d1 a1) b1', o1 = (d1 b1 + delta1 k1.q1)/sqrt(128)
        //   S1.k2 = d1 c + delta1 k1.k2,  S1.q2 = d1 e + delta1 k1.q2
        //   delta2 = (v2 - d2 S1.k2) b2', o2 = (d2 S1.q2 + delta2 k2.q2)/sqrt(128)
        //   S <- d1 d2 S + (d2 delta1) k1 + delta2 k2
        // (the sequential rule's values up to fp32 rounding); an odd last token
        // takes the one-token step.
        struct Ops2 {
            Ops t1, t2;
            float kk, kqx;
        };
        auto read_pair = [&](uint32_t j) {
            Ops2 o;
            o.t1 = read_ops(j), o.t2 = read_ops(j + 1);
            o.kk = L.kk[buf][j / 2], o.kqx = L.kqx[buf][j / 2];
            return o;
        };
        auto pair = [&](const Ops2& x, uint32_t j) {
            const float k1[8] = {x.t1.k0.x, x.t1.k0.y, x.t1.k0.z, x.t1.k0.w, x.t1.k1.x, x.t1.k1.y, x.t1.k1.z, x.t1.k1.w};
            const float q1[8] = {x.t1.q0.x, x.t1.q0.y, x.t1.q0.z, x.t1.q0.w, x.t1.q1.x, x.t1.q1.y, x.t1.q1.z, x.t1.q1.w};
            const float k2[8] = {x.t2.k0.x, x.t2.k0.y, x.t2.k0.z, x.t2.k0.w, x.t2.k1.x, x.t2.k1.y, x.t2.k1.z, x.t2.k1.w};
            const float q2[8] = {x.t2.q0.x, x.t2.q0.y, x.t2.q0.z, x.t2.q0.w, x.t2.q1.x, x.t2.q1.y, x.t2.q1.z, x.t2.q1.w};
            float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f, c0 = 0.f, c1 = 0.f, e0 = 0.f, e1 = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a0 = fmaf(S[i], k1[i], a0);
                b0 = fmaf(S[i], q1[i], b0);
                c0 = fmaf(S[i], k2[i], c0);
                e0 = fmaf(S[i], q2[i], e0);
                a1 = fmaf(S[4 + i], k1[4 + i], a1);
                b1 = fmaf(S[4 + i], q1[4 + i], b1);
                c1 = fmaf(S[4 + i], k2[4 + i], c1);
                e1 = fmaf(S[4 + i], q2[4 + i], e1);
            }
            float a = a0 + a1, bq = b0 + b1, c = c0 + c1, e = e0 + e1;
            a += lane_xor<1>(a), bq += lane_xor<1>(bq), c += lane_xor<1>(c), e += lane_xor<1>(e);
            a += lane_xor<2>(a), bq += lane_xor<2>(bq), c += lane_xor<2>(c), e += lane_xor<2>(e);
            a += lane_xor<4>(a), bq += lane_xor<4>(bq), c += lane_xor<4>(c), e += lane_xor<4>(e);
            a += lane_xor<8>(a), bq += lane_xor<8>(bq), c += lane_xor<8>(c), e += lane_xor<8>(e);
            const float d1 = x.t1.dec, d2 = x.t2.dec;
            const float delta1 = (x.t1.vv - d1 * a) * x.t1.bt;
            const float o1 = (d1 * bq + delta1 * x.t1.kq) * scale;
            const float sk2 = d1 * c + delta1 * x.kk, sq2 = d1 * e + delta1 * x.kqx;
            const float delta2 = (x.t2.vv - d2 * sk2) * x.t2.bt;
            const float o2 = (d2 * sq2 + delta2 * x.t2.kq) * scale;
            const float dd = d1 * d2, w1 = d2 * delta1;
#pragma unroll
            for (int i = 0; i < 8; ++i) S[i] = fmaf(k2[i], delta2, fmaf(k1[i], w1, S[i] * dd));
            if (ks == 0) {
                out[(((size_t)(t0 + j) * n_seq + s) * n_v + h) * d_v + col] = o1;
                out[(((size_t)(t0 + j + 1) * n_seq + s) * n_v + h) * d_v + col] = o2;
            }
        };
        const uint32_t np = nt / 2;
        if (np > 0) {  // pair m+1's operands are read while pair m is computed
            Ops2 A = read_pair(0);
            for (uint32_t m = 0; m < np; m += 2) {
                const Ops2 B = read_pair(m + 1 < np ? 2 * (m + 1) : 2 * m);
                pair(A, 2 * m);
                if (m + 1 >= np) break;
                A = read_pair(m + 2 < np ? 2 * (m + 2) : 2 * (m + 1));
                pair(B, 2 * (m + 1));
            }
        }
        if (nt & 1) token(read_ops(nt - 1), nt - 1);
        stage_store(buf ^ 1);
        __syncthreads();
    }
    *(float4*)sp = make_float4(S[0], S[1], S[2], S[3]);
    *(float4*)(sp + 4) = make_float4(S[4], S[5], S[6], S[7]);
}

// ------------------------------------------------------------ fused decode step
// One decode token of a delta-net block for value head h of sequence s, from
// the input projection to the output projection's activation:
//   conv + SiLU of the q/k channels of k-head h/rep and the v channels of h
//   (ring conv state, as k_conv_gates), L2 norm of q and k, decay / beta gates,
//   the delta-rule update of the head's 128x128 state, gated RMSNorm of the
//   128 outputs and Q8_0 quantization into act (K = n_v*128).
// grid (n_v, n_seq), block 1024: thread t owns column t/8 of the transposed
// state S[v][k] and k-entries 32u + 4*(t%8) + e (u, e < 4); the state is
// loaded first, so its latency overlaps the conv work.  The q/k conv state of
// a k-head shared by rep value heads is written by the block with h % rep == 0;
// the others only use slots that step leaves untouched (with kern == 4 every
// block loads all four slots before it knows the position, and the slot being
// rewritten is never selected).
// proj holds NP partial sums of the input projection, [NP][n_seq][Nin] (a
// split-K matvec's output); every element read is their sum in part order.
template <int NP>
__device__ __forceinline__ float proj_at(const float* __restrict__ pr, size_t pstride, size_t i) {
    float v[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) v[q] = pr[q * pstride + i];
    float a = v[0];
#pragma unroll
    for (int q = 1; q < NP; ++q) a += v[q];
    return a;
}

template <int NP>
__global__ __launch_bounds__(1024) void k_delta_step(const float* __restrict__ proj, uint32_t Nin,
                                                     float* __restrict__ conv_state,
                                                     const float* __restrict__ conv_w,
                                                     const float* __restrict__ a_log,
                                                     const float* __restrict__ dt_bias,
                                                     const float* __restrict__ norm_w, float* __restrict__ state,
                                                     uint8_t* __restrict__ act, uint32_t xd_off, uint32_t M,
                                                     const int32_t* __restrict__ pos, uint32_t n_k, uint32_t n_v,
                                                     uint32_t kern, float* __restrict__ yout, uint32_t P) {
    __shared__ float q_s[128], k_s[128], v_s[128], o_s[128];
    __shared__ float red[4], red2[2], gate_s[2];
    const uint32_t h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const uint32_t key_dim = n_k * 128, value_dim = n_v * 128, conv_dim = 2 * key_dim + value_dim;
    const uint32_t rep = n_v / n_k, qh = h / rep;
    const float* pr = proj + (size_t)s * Nin;
    const size_t pstride = (size_t)M * Nin;

    // Every load that does not depend on the position is issued before pos[s]
    // arrives.  State column first: thread (col, ks) holds k = 32u + 4ks + e,
    // so each load instruction reads whole 128-byte runs of 8 columns.
    const uint32_t col = t >> 3, ks = t & 7;
    float* sp = state + (((size_t)s * n_v + h) * 128 + col) * 128 + 4 * ks;
    float S[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const f32x4 v4 = __builtin_nontemporal_load((const f32x4*)(sp + 32 * u));
        S[4 * u] = v4.x, S[4 * u + 1] = v4.y, S[4 * u + 2] = v4.z, S[4 * u + 3] = v4.w;
    }
    // gated-norm inputs of output channel t
    float zg = 0.0f, nwt = 0.0f;
    if (t < 128) {
        zg = proj_at<NP>(pr, pstride, conv_dim + h * 128 + t);
        nwt = norm_w[t];
    }
    // conv inputs: threads 0..127 q channels, 128..255 k channels, 256..383 v
    // channels (with kern == 4 all four ring slots and taps); thread 384 the gates
    float* cst = conv_state + (size_t)s * kern * conv_dim;
    const uint32_t part = t >> 7, i = t & 127;
    const uint32_t c = part == 2 ? 2 * key_dim + h * 128 + i : part * key_dim + qh * 128 + i;
    const bool ring4 = kern == 4;
    float xin = 0.0f, r4[4] = {0.f, 0.f, 0.f, 0.f}, w4[4] = {0.f, 0.f, 0.f, 0.f};
    if (t < 384) {
        xin = proj_at<NP>(pr, pstride, c);
        if (ring4) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                r4[q] = cst[(size_t)q * conv_dim + c];
                w4[q] = conv_w[(size_t)q * conv_dim + c];
            }
        }
    }
    float al = 0.0f, br = 0.0f, dtb = 0.0f, alog = 0.0f;
    if (t == 384) {
        al = proj_at<NP>(pr, pstride, conv_dim + value_dim + h);
        br = proj_at<NP>(pr, pstride, conv_dim + value_dim + n_v + h);
        dtb = dt_bias[h];
        alog = a_log[h];
    }
    const int32_t p = pos[s];
    if (p < 0) return;

    if (t < 384) {
        float acc;
        if (ring4) {  // conv_ring's sum with the slots already in registers
            acc = __fmul_rn(xin, w4[3]);
#pragma unroll
            for (uint32_t k = 1; k < 4; ++k) {
                const uint32_t q = ((uint32_t)p + 4 - k) & 3;
                const float rv = q == 0 ? r4[0] : (q == 1 ? r4[1] : (q == 2 ? r4[2] : r4[3]));
                acc = fmaf(rv, w4[3 - k], acc);
            }
        } else {
            acc = conv_ring(cst, conv_w, xin, (uint32_t)p, kern, conv_dim, c);
        }
        const float a = silu(acc);
        if (part == 2 || h % rep == 0) cst[(size_t)((uint32_t)p % kern) * conv_dim + c] = xin;
        if (part == 2) {
            v_s[i] = a;
        } else {
            const float ss = wave_sum(a * a);  // part is uniform per wave
            if ((t & 63) == 0) red[t >> 6] = ss;
            (part == 0 ? q_s : k_s)[i] = a;  // normalized after the barrier
        }
    } else if (t == 384) {
        const float sp_in = al + dtb;
        const float spl = sp_in > 20.0f ? sp_in : log1pf(expf(sp_in));
        const float g = -expf(alog) * spl;
        gate_s[0] = expf(g);
        gate_s[1] = 1.0f / (1.0f + expf(-br));
    }
    __syncthreads();
    const float inv_q = 1.0f / sqrtf((red[0] + red[1]) + 1e-6f);
    const float inv_k = 1.0f / sqrtf((red[2] + red[3]) + 1e-6f);
    const float dec = gate_s[0], bt = gate_s[1];

    // delta rule on this column: S <- dec*S; kv = S.k; delta = (v - kv)*beta; S += k*delta; o = S.q/sqrt(128)
    const float scale = 1.0f / sqrtf(128.0f);
    float kk[16], qq[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        kk[i] = k_s[32 * (i >> 2) + 4 * ks + (i & 3)] * inv_k;
        qq[i] = q_s[32 * (i >> 2) + 4 * ks + (i & 3)] * inv_q;
    }
    float kvp = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        S[i] *= dec;
        kvp = fmaf(S[i], kk[i], kvp);
    }
    kvp += lane_xor<1>(kvp);
    kvp += lane_xor<2>(kvp);
    kvp += lane_xor<4>(kvp);
    const float delta = (v_s[col] - kvp) * bt;
    float op = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        S[i] = fmaf(kk[i], delta, S[i]);
        op = fmaf(S[i], qq[i] * scale, op);
    }
    op += lane_xor<1>(op);
    op += lane_xor<2>(op);
    op += lane_xor<4>(op);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const f32x4 v4 = {S[4 * u], S[4 * u + 1], S[4 * u + 2], S[4 * u + 3]};
        __builtin_nontemporal_store(v4, (f32x4*)(sp + 32 * u));
    }
    if (ks == 0) o_s[col] = op;
    __syncthreads();

    // gated RMSNorm over the head's 128 outputs (waves 0 and 1), quantized for the output projection
    float o = 0.0f;
    if (t < 128) {
        o = o_s[t];
        const float ss = wave_sum(o * o);
        if ((t & 63) == 0) red2[t >> 6] = ss;
    }
    __syncthreads();
    if (t < 128) {
        const float rms = sqrtf((red2[0] + red2[1]) / 128.0f + 1e-6f);
        const float inv = 1.0f / rms;
        const float val = o * inv * nwt * silu(zg);
        if (act) store_act_q8_lane(val, act, (float*)(act + xd_off), M, value_dim / 32, s, h * 128 + t, P);
        if (yout) yout[(size_t)s * value_dim + h * 128 + t] = val;
    }
}

}  // namespace ec

using namespace ec;

extern "C" int ec_deltanet(float* state, const float* q, const float* k, const float* v, const float* decay,
                           const float* beta, float* out, uint32_t T, uint32_t n_seq, uint32_t n_v, uint32_t n_k,
                           uint32_t d_k, uint32_t d_v, const int32_t* seq_pos, void* stream) {
    if (T == 0 || n_seq == 0) return EC_OK;
    if (!state || !q || !k || !v || !decay || !beta || !out || n_k == 0 || n_v % n_k || d_k != 128 || d_v == 0 ||
        d_v % 16)
        return ec_set_error(EC_ERR_ARG, "ec_deltanet: need d_k == 128, d_v % 16 == 0, n_v % n_k == 0");
    hipLaunchKernelGGL(k_deltanet, dim3(n_v * (d_v / 16), n_seq), dim3(256), 0, (hipStream_t)stream, state, q, k, v,
                       decay, beta, out, T, n_seq, n_v, n_k, d_v, seq_pos);
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_delta_step_out_pieces(const float* proj, uint32_t nparts, uint32_t Nin, float* conv_state,
                                        const float* conv_w, const float* a_log, const float* dt_bias,
                                        const float* norm_w, float* state, void* act, float* out, const int32_t* pos,
                                        uint32_t n_seq, uint32_t n_k, uint32_t n_v, uint32_t kern, uint32_t pieces,
                                        void* stream) {
    if (n_seq == 0) return EC_OK;
    if (!proj || !conv_state || !conv_w || !a_log || !dt_bias || !norm_w || !state || (!act && !out) || !pos || n_k == 0 ||
        n_v == 0 || n_v % n_k || kern == 0 || n_seq > 16 || nparts == 0 || nparts > 8 ||
        Nin < 2 * n_k * 128 + 2 * n_v * 128 + 2 * n_v || (pieces != 1 && pieces != 2))
        return ec_set_error(EC_ERR_ARG, "ec_delta_step: bad argument");
    const ActLayout L = act_layout(EC_Q8_0, pieces * n_seq, n_v * 128);
    const dim3 grid(n_v, n_seq);
    const hipStream_t st = (hipStream_t)stream;
#define EC_DSTEP(NP)                                                                                               \
    hipLaunchKernelGGL(k_delta_step<NP>, grid, dim3(1024), 0, st, proj, Nin, conv_state, conv_w, a_log, dt_bias, \
                       norm_w, state, (uint8_t*)act, (uint32_t)L.xd_off, n_seq, pos, n_k, n_v, kern, out, pieces)
    switch (nparts) {
        case 1: EC_DSTEP(1); break;
        case 2: EC_DSTEP(2); break;
        case 3: EC_DSTEP(3); break;
        case 4: EC_DSTEP(4); break;
        case 5: EC_DSTEP(5); break;
        case 6: EC_DSTEP(6); break;
        case 7: EC_DSTEP(7); break;
        default: EC_DSTEP(8); break;
    }
#undef EC_DSTEP
    EC_CHECK_LAUNCH();
    return EC_OK;
}

extern "C" int ec_delta_step_out(const float* proj, uint32_t nparts, uint32_t Nin, float* conv_state,
                                 const float* conv_w, const float* a_log, const float* dt_bias, const float* norm_w,
                                 float* state, void* act, float* out, const int32_t* pos, uint32_t n_seq, uint32_t n_k,
                                 uint32_t n_v, uint32_t kern, void* stream) {
    return ec_delta_step_out_pieces(proj, nparts, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, state, act, out,
                                    pos, n_seq, n_k, n_v, kern, 1, stream);
}

extern "C" int ec_delta_step_split(const float* proj, uint32_t nparts, uint32_t Nin, float* conv_state,
                                   const float* conv_w, const float* a_log, const float* dt_bias, const float* norm_w,
                                   float* state, void* act, const int32_t* pos, uint32_t n_seq, uint32_t n_k,
                                   uint32_t n_v, uint32_t kern, void* stream) {
    if (!act && n_seq) return ec_set_error(EC_ERR_ARG, "ec_delta_step: bad argument");
    return ec_delta_step_out(proj, nparts, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, state, act, nullptr, pos,
                             n_seq, n_k, n_v, kern, stream);
}

extern "C" int ec_delta_step(const float* proj, uint32_t Nin, float* conv_state, const float* conv_w,
                             const float* a_log, const float* dt_bias, const float* norm_w, float* state, void* act,
                             const int32_t* pos, uint32_t n_seq, uint32_t n_k, uint32_t n_v, uint32_t kern,
                             void* stream) {
    return ec_delta_step_split(proj, 1, Nin, conv_state, conv_w, a_log, dt_bias, norm_w, state, act, pos, n_seq, n_k,
                               n_v, kern, stream);
}
