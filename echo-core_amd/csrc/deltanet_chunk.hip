// deltanet_chunk.hip — chunked gated delta rule for prefill (gfx950).
//
// The recurrence of ec_deltanet (echo-core-zig/src/kernels/qwen_linear.zig:
// 207-250, per value head, reference orientation S[k][v]):
//   S_t = g_t S_{t-1} + k_t u_t^T,  u_t = b_t (v_t - g_t S_{t-1}^T k_t),
//   o_t = S_t^T q_t / sqrt(d_k)
// over a chunk of C tokens starting from S0, with G_t = g_1 ... g_t (G_t/G_i
// <= 1 for i <= t, computed as exp of differences of the chunk's cumulative
// log-decays, so no ratio overflows):
//   (I + A) U = B (V - G K S0),   A_ti = b_t (G_t/G_i) k_t.k_i  for i < t
//   O  = (G Q S0 + P U) / sqrt(d_k),  P_ti = (G_t/G_i) q_t.k_i  for i <= t
//   S_C = G_C S0 + K^T diag(G_C/G_t) U
// With X = (I + A)^{-1} [B G K | B V] = [W | U~] this is U = U~ - W S0: the
// chunk's W, U~ and P depend on the inputs only, so pass 1 computes them for
// every chunk of every head in parallel; pass 2 walks the chunks in order per
// (head, 16 value columns), the state slice in LDS, every product on fp32
// MFMA (v_mfma_f32_16x16x4f32).  Tokens past T are padded with g = 1, b = 0
// and zero q, k, v, which leaves the state and the real tokens' outputs as
// they are.
#include "common.hpp"
#include "layout.hpp"

namespace ec {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kCk = 64;        // tokens per chunk
constexpr uint32_t kDh = 128;       // d_k = d_v
constexpr uint32_t kVs = 16;        // value columns per scan workgroup
constexpr uint32_t kLd = kDh + 4;   // LDS row of a C x 128 matrix (floats)
constexpr uint32_t kPd = kCk + 4;   // LDS row of a C x C matrix
// workspace floats per (sequence, head, chunk): W [C][128], U~ [C][128],
// P [C][C], G [C], G_C/G_t [C], K^T [128][C] (zero past the last token)
constexpr uint32_t kWsW = 0, kWsU = kCk * kDh, kWsP = 2 * kCk * kDh, kWsG = kWsP + kCk * kCk, kWsF = kWsG + kCk;
constexpr uint32_t kWsK = kWsF + kCk;
constexpr uint32_t kWsFloats = kWsK + kDh * kCk;

// D (16 x 16) += A (16 x 4) B (4 x 16): lane l holds A[l%16][l/16],
// B[l/16][l%16] and D[4*(l/16) + r][l%16] in element r.
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ pass 1
constexpr uint32_t kXd = 2 * kDh + 4;  // LDS row of X = [B G K | B V] (256 columns)
constexpr uint32_t kTd = 16 + 4;       // LDS row of a 16 x 16 diagonal inverse
struct PrepLds {
    float K[kCk][kLd];
    float Q[kCk][kLd];
    float A[kCk][kPd];
    float X[kCk][kXd];
    float Td[kCk / 16][16][kTd];
    float lg[kCk], bt[kCk], gam[kCk];
};

// grid (chunks, n_v, n_seq), block 256: wave w solves columns 64w .. 64w+63
// of X (both halves of a thread's column stay in its own wave).
__global__ __launch_bounds__(256) void k_dn_chunk_prep(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, const float* __restrict__ decay,
                                                       const float* __restrict__ beta, float* __restrict__ ws,
                                                       uint32_t T, uint32_t n_seq, uint32_t n_v, uint32_t n_k,
                                                       const int32_t* __restrict__ seq_pos) {
    extern __shared__ __align__(16) float lds_raw[];
    PrepLds& L = *(PrepLds*)lds_raw;
    const uint32_t c = blockIdx.x, h = blockIdx.y, s = blockIdx.z, nc = gridDim.x;
    if (seq_pos && seq_pos[s] < 0) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const uint32_t qh = h / (n_v / n_k);
    const uint32_t t0 = c * kCk, n = min(kCk, T - t0);
    float* wsc = ws + ((size_t)(s * n_v + h) * nc + c) * kWsFloats;

    // every global load of the chunk is issued before the first LDS store
    constexpr uint32_t NL = kCk * (kDh / 4) / 256;  // float4 of K (of Q, of V) per thread
    f32x4 kr[NL], qr[NL], vr[NL];
#pragma unroll
    for (uint32_t u = 0; u < NL; ++u) {
        const uint32_t i = tid + 256 * u, t = min(i / (kDh / 4), n - 1), e = 4 * (i % (kDh / 4));
        const size_t off = (((size_t)(t0 + t) * n_seq + s) * n_k + qh) * kDh + e;
        kr[u] = *(const f32x4*)(k + off);
        qr[u] = *(const f32x4*)(q + off);
        vr[u] = *(const f32x4*)(v + (((size_t)(t0 + t) * n_seq + s) * n_v + h) * kDh + e);
    }
    if (w == 0) {  // inclusive scan of log(decay) over the chunk's tokens
        const size_t hv = ((size_t)(t0 + lane) * n_seq + s) * n_v + h;
        float lg = 0.f, bv = 0.f;
        if (lane < n) {
            lg = logf(fmaxf(decay[hv], 1e-30f));
            bv = beta[hv];
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float u = __shfl_up(lg, o);
            if ((int)lane >= o) lg += u;
        }
        L.lg[lane] = lg;
        L.bt[lane] = bv;
        const float gm = expf(lg);
        L.gam[lane] = gm;
        wsc[kWsG + lane] = gm;
    }
    __syncthreads();
    if (w == 0) wsc[kWsF + lane] = expf(L.lg[kCk - 1] - L.lg[lane]);
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t u = 0; u < NL; ++u) {
        const uint32_t i = tid + 256 * u, t = i / (kDh / 4), e = 4 * (i % (kDh / 4));
        const bool ok = t < n;
        *(f32x4*)&L.K[t][e] = ok ? kr[u] : z4;
        *(f32x4*)&L.Q[t][e] = ok ? qr[u] : z4;
        // right-hand sides R = [b_t G_t k_t | b_t v_t] (b_t = 0 past the last token)
        const float bg = L.bt[t] * L.gam[t], b = L.bt[t];
        *(f32x4*)&L.X[t][e] = ok ? kr[u] * bg : z4;
        *(f32x4*)&L.X[t][kDh + e] = ok ? vr[u] * b : z4;
    }
    __syncthreads();

    // K K^T -> A and Q K^T -> P on the 10 lower 16 x 16 tiles each (20 jobs,
    // wave w takes jobs w, w+4, ...)
    for (uint32_t job = w; job < 20; job += 4) {
        const bool isP = job >= 10;
        uint32_t jt = isP ? job - 10 : job, ti = 0;
        while (jt > ti) jt -= ++ti;  // job index -> (ti, tj = jt) with tj <= ti
        const uint32_t tj = jt;
        const float(*Ar)[kLd] = isP ? L.Q : L.K;
        f32x4 acc = z4;
        f32x4 a8[8], b8[8];  // lane (r, g) contracts over k = 32g .. 32g+31
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            a8[m] = *(const f32x4*)&Ar[ti * 16 + r16][32 * g4 + 4 * m];
            b8[m] = *(const f32x4*)&L.K[tj * 16 + r16][32 * g4 + 4 * m];
        }
#pragma unroll
        for (int m = 0; m < 8; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = mfma4(a8[m][e], b8[m][e], acc);
        const uint32_t j = tj * 16 + r16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = ti * 16 + 4 * g4 + r;
            const float ratio = expf(L.lg[i] - L.lg[j]);
            if (isP) wsc[kWsP + i * kCk + j] = i >= j ? ratio * acc[r] : 0.f;
            else L.A[i][j] = i > j ? L.bt[i] * ratio * acc[r] : 0.f;
        }
    }
    // upper tiles of P are never read (pass 2 stops at the diagonal tile)
    __syncthreads();

    // diagonal blocks: wave b inverts (I + A_bb), lane j < 16 solving column j
    {
        const uint32_t b = w, j = r16;
        float y[16];
#pragma unroll
        for (uint32_t t = 0; t < 16; ++t) {
            float acc = t == j ? 1.f : 0.f;
#pragma unroll
            for (uint32_t i = 0; i < t; ++i) acc = fmaf(-L.A[16 * b + t][16 * b + i], y[i], acc);
            y[t] = acc;
        }
        if (lane < 16) {
#pragma unroll
            for (uint32_t t = 0; t < 16; ++t) L.Td[b][t][j] = y[t];
        }
    }
    __syncthreads();

    // block forward substitution on the wave's four 16-column tiles:
    //   Y = X_b - sum_{c<b} A_bc X_c,  X_b = (I + A_bb)^{-1} Y
    for (uint32_t b = 0; b < kCk / 16; ++b) {
#pragma unroll
        for (uint32_t ct = 0; ct < 4; ++ct) {
            const uint32_t c0 = 64 * w + 16 * ct;
            f32x4 acc;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = L.X[16 * b + 4 * g4 + r][c0 + r16];
            for (uint32_t cb = 0; cb < b; ++cb) {
#pragma unroll
                for (uint32_t kk = 0; kk < 16; kk += 4)
                    acc = mfma4(-L.A[16 * b + r16][16 * cb + kk + g4], L.X[16 * cb + kk + g4][c0 + r16], acc);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) L.X[16 * b + 4 * g4 + r][c0 + r16] = acc[r];
        }
        __syncthreads();
#pragma unroll
        for (uint32_t ct = 0; ct < 4; ++ct) {
            const uint32_t c0 = 64 * w + 16 * ct;
            f32x4 acc = z4;
#pragma unroll
            for (uint32_t kk = 0; kk < 16; kk += 4)
                acc = mfma4(L.Td[b][r16][kk + g4], L.X[16 * b + kk + g4][c0 + r16], acc);
            __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's reads of Y are done before X_b overwrites it
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int r = 0; r < 4; ++r) L.X[16 * b + 4 * g4 + r][c0 + r16] = acc[r];
        }
        __syncthreads();
    }

    // W = X[:, 0:128], U~ = X[:, 128:256]
    const uint32_t col = tid;
    float* dst = wsc + (col < kDh ? kWsW + col : kWsU + (col - kDh));
#pragma unroll 8
    for (uint32_t t = 0; t < kCk; ++t) dst[t * kDh] = L.X[t][col];
    // K^T for the scan's state update, read so that the lanes of a wave take
    // 64 consecutive keys of one token row (no LDS bank conflicts)
#pragma unroll
    for (uint32_t u = 0; u < kDh * kCk / 4 / 256; ++u) {
        const uint32_t key = 64 * (u & 1) + lane, t = 4 * (4 * w + (u >> 1));
        const f32x4 kv = {L.K[t][key], L.K[t + 1][key], L.K[t + 2][key], L.K[t + 3][key]};
        *(f32x4*)(wsc + kWsK + key * kCk + t) = kv;
    }
}

// ------------------------------------------------------------------ pass 2
// MFMA operands are read so that each lane's share of the contraction index
// is contiguous in LDS: in step m a 16x16x4 MFMA takes from lane (r, g) the
// index 32g + m (K = 128), 16g + m (K = 64) or (K/4)g + m, instead of 4m + g,
// so a lane fetches its 32 (16, K/4) operand values with 16-byte reads issued
// before the first MFMA.  Every index is still used once.
constexpr uint32_t kKt = kCk + 4;  // LDS row of K^T and U^T (token index contiguous)
struct ScanLds {
    float S[kVs][kLd];   // state slice, S[v][k] (16 value columns)
    float W[kCk][kLd];
    float Q[kCk][kLd];
    float Kt[kDh][kKt];  // K^T: Kt[k][t]
    float P[kCk][kPd];
    float Ut[kVs][kKt];  // U^T of the slice: Ut[j][t]
    float G[kCk], F[kCk];
};

// grid (n_v * 8, n_seq), block 256: workgroup = (head, 16 value columns);
// wave w owns row tile w (tokens 16w .. 16w+15) of U and O, and key tiles
// 2w, 2w+1 of the state update.  Workgroup b serves head b % n_v: workgroups
// are dealt to the 8 XCDs round-robin, so with n_v % 8 == 0 the 8 column
// slices of a head share one XCD's L2 and its W, Q, K, P are fetched once.
__global__ __launch_bounds__(256) void k_dn_chunk_scan(float* __restrict__ state, const float* __restrict__ q,
                                                       const float* __restrict__ ws,
                                                       float* __restrict__ out, uint32_t T, uint32_t n_seq,
                                                       uint32_t n_v, uint32_t n_k, uint32_t nc,
                                                       const int32_t* __restrict__ seq_pos) {
    extern __shared__ __align__(16) float lds_raw[];
    ScanLds& L = *(ScanLds*)lds_raw;
    const uint32_t h = blockIdx.x % n_v, vs0 = kVs * (blockIdx.x / n_v), s = blockIdx.y;
    if (seq_pos && seq_pos[s] < 0) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const uint32_t qh = h / (n_v / n_k);
    const float scale = 1.0f / sqrtf((float)kDh);
    float* sp = state + ((size_t)(s * n_v + h) * kDh + vs0) * kDh;
    for (uint32_t i = tid; i < kVs * (kDh / 4); i += 256) {
        const uint32_t j = i / (kDh / 4), e = 4 * (i % (kDh / 4));
        *(f32x4*)&L.S[j][e] = *(const f32x4*)(sp + (size_t)j * kDh + e);
    }
    // A chunk's operands are loaded into registers one chunk ahead (all loads
    // of chunk c+1 are in flight while chunk c computes) and stored to LDS at
    // the start of their chunk; U~ of the wave's row tile stays in registers
    // in the MFMA D layout.
    constexpr uint32_t NL = kCk * (kDh / 4) / 256, NP = kCk * (kCk / 4) / 256;
    f32x4 rw[NL], rq[NL], rk[NL], rp[NP], ru;
    float rg = 0.f, rf = 0.f;
    // Two groups, issued at different points of the previous chunk, so that a
    // wave never has all 34 loads waiting for a slot in the memory pipeline.
    auto load_a = [&](uint32_t c) {
        const uint32_t t0 = c * kCk, n = min(kCk, T - t0);
        const float* wsc = ws + ((size_t)(s * n_v + h) * nc + c) * kWsFloats;
#pragma unroll
        for (uint32_t u = 0; u < NL; ++u) {
            const uint32_t i = tid + 256 * u, t = i / (kDh / 4), e = 4 * (i % (kDh / 4));
            rw[u] = *(const f32x4*)(wsc + kWsW + t * kDh + e);
            rq[u] = *(const f32x4*)(q + (((size_t)(t0 + min(t, n - 1)) * n_seq + s) * n_k + qh) * kDh + e);
        }
    };
    auto load_b = [&](uint32_t c) {
        const float* wsc = ws + ((size_t)(s * n_v + h) * nc + c) * kWsFloats;
#pragma unroll
        for (uint32_t u = 0; u < NL; ++u) {
            const uint32_t i = tid + 256 * u;
            rk[u] = *(const f32x4*)(wsc + kWsK + 4 * i);  // K^T row i / 16, tokens 4 (i % 16) ..
        }
#pragma unroll
        for (uint32_t u = 0; u < NP; ++u) {
            const uint32_t i = tid + 256 * u, t = i / (kCk / 4), e = 4 * (i % (kCk / 4));
            rp[u] = *(const f32x4*)(wsc + kWsP + t * kCk + e);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) ru[r] = wsc[kWsU + (16 * w + 4 * g4 + r) * kDh + vs0 + r16];
        if (tid < kCk) {
            rg = wsc[kWsG + tid];
            rf = wsc[kWsF + tid];
        }
    };
    auto store = [&](uint32_t c) {
        const uint32_t n = min(kCk, T - c * kCk);
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t u = 0; u < NL; ++u) {
            const uint32_t i = tid + 256 * u, t = i / (kDh / 4), e = 4 * (i % (kDh / 4));
            const bool ok = t < n;
            *(f32x4*)&L.W[t][e] = rw[u];
            *(f32x4*)&L.Q[t][e] = ok ? rq[u] : z4;
            *(f32x4*)&L.Kt[i / (kCk / 4)][4 * (i % (kCk / 4))] = rk[u];
        }
#pragma unroll
        for (uint32_t u = 0; u < NP; ++u) {
            const uint32_t i = tid + 256 * u, t = i / (kCk / 4), e = 4 * (i % (kCk / 4));
            *(f32x4*)&L.P[t][e] = rp[u];
        }
        if (tid < kCk) {
            L.G[tid] = rg;
            L.F[tid] = rf;
        }
    };
    load_a(0);
    load_b(0);
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c = 0; c < nc; ++c) {
        const uint32_t t0 = c * kCk, n = min(kCk, T - t0);
        __syncthreads();  // the previous chunk's readers of W, Q, K, P, U are done
        store(c);
        const f32x4 uin = ru;
        __syncthreads();
        if (c + 1 < nc) load_a(c + 1);

        // U = U~ - W S0 and QS = Q S0 for row tile w (B[k][j] = S[j][k]),
        // lane (r, g) contracting over k = 32g .. 32g+31
        f32x4 du = z4, dq = z4;
        {
            f32x4 aw[8], aq[8], bs[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                aw[m] = *(const f32x4*)&L.W[w * 16 + r16][32 * g4 + 4 * m];
                aq[m] = *(const f32x4*)&L.Q[w * 16 + r16][32 * g4 + 4 * m];
                bs[m] = *(const f32x4*)&L.S[r16][32 * g4 + 4 * m];
            }
#pragma unroll
            for (int m = 0; m < 8; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    du = mfma4(aw[m][e], bs[m][e], du);
                    dq = mfma4(aq[m][e], bs[m][e], dq);
                }
        }
        // lane holds U[16w + 4g + r][r16]: four consecutive tokens of U^T
        *(f32x4*)&L.Ut[r16][16 * w + 4 * g4] = uin - du;
        __syncthreads();  // U^T complete; S no longer read this chunk
        if (c + 1 < nc) load_b(c + 1);

        // O = (G QS + P U)/sqrt(d_k): P is lower triangular, so row tile w
        // contracts over tokens 0 .. 16w+15, lane (r, g) over 4(w+1) of them
        f32x4 po = z4;
        {
            const uint32_t kw = 4 * (w + 1), t1 = g4 * kw;
            for (uint32_t m = 0; m < kw; m += 4) {
                const f32x4 ap = *(const f32x4*)&L.P[w * 16 + r16][t1 + m];
                const f32x4 bu = *(const f32x4*)&L.Ut[r16][t1 + m];
#pragma unroll
                for (int e = 0; e < 4; ++e) po = mfma4(ap[e], bu[e], po);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t i = w * 16 + 4 * g4 + r;
            if (i < n) out[(((size_t)(t0 + i) * n_seq + s) * n_v + h) * kDh + vs0 + r16] = (L.G[i] * dq[r] + po[r]) * scale;
        }
        // S <- G_C S + U^T diag(G_C/G_t) K on key tiles 2w, 2w+1, lane (r, g)
        // contracting over tokens 16g .. 16g+15
        const float gC = L.G[kCk - 1];
        f32x4 au[4], bk0[4], bk1[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            au[m] = *(const f32x4*)&L.Ut[r16][16 * g4 + 4 * m] * *(const f32x4*)&L.F[16 * g4 + 4 * m];
            bk0[m] = *(const f32x4*)&L.Kt[(2 * w) * 16 + r16][16 * g4 + 4 * m];
            bk1[m] = *(const f32x4*)&L.Kt[(2 * w + 1) * 16 + r16][16 * g4 + 4 * m];
        }
        f32x4 ds0 = z4, ds1 = z4;
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ds0 = mfma4(au[m][e], bk0[m][e], ds0);
                ds1 = mfma4(au[m][e], bk1[m][e], ds1);
            }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint32_t j = 4 * g4 + r;
            L.S[j][(2 * w) * 16 + r16] = gC * L.S[j][(2 * w) * 16 + r16] + ds0[r];
            L.S[j][(2 * w + 1) * 16 + r16] = gC * L.S[j][(2 * w + 1) * 16 + r16] + ds1[r];
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < kVs * (kDh / 4); i += 256) {
        const uint32_t j = i / (kDh / 4), e = 4 * (i % (kDh / 4));
        *(f32x4*)(sp + (size_t)j * kDh + e) = *(const f32x4*)&L.S[j][e];
    }
}

}  // namespace ec

using namespace ec;

extern "C" size_t ec_deltanet_chunked_ws_bytes(uint32_t T, uint32_t n_seq, uint32_t n_v) {
    return (size_t)((T + kCk - 1) / kCk) * n_seq * n_v * kWsFloats * sizeof(float);
}

extern "C" int ec_deltanet_chunked(float* state, const float* q, const float* k, const float* v, const float* decay,
                                   const float* beta, float* out, uint32_t T, uint32_t n_seq, uint32_t n_v,
                                   uint32_t n_k, uint32_t d_k, uint32_t d_v, const int32_t* seq_pos, void* ws,
                                   void* stream) {
    if (T == 0 || n_seq == 0) return EC_OK;
    if (!state || !q || !k || !v || !decay || !beta || !out || !ws || n_k == 0 || n_v % n_k || d_k != kDh ||
        d_v != kDh || n_seq > 65535 || n_v > 65535)
        return ec_set_error(EC_ERR_ARG, "ec_deltanet_chunked: need d_k == d_v == 128, n_v % n_k == 0, a workspace");
    const uint32_t nc = (T + kCk - 1) / kCk;
    const hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(k_dn_chunk_prep, dim3(nc, n_v, n_seq), dim3(256), sizeof(PrepLds), st, q, k, v, decay, beta,
                       (float*)ws, T, n_seq, n_v, n_k, seq_pos);
    EC_CHECK_LAUNCH();
    hipLaunchKernelGGL(k_dn_chunk_scan, dim3(n_v * (kDh / kVs), n_seq), dim3(256), sizeof(ScanLds), st, state, q,
                       (const float*)ws, out, T, n_seq, n_v, n_k, nc, seq_pos);
    EC_CHECK_LAUNCH();
    return EC_OK;
}
