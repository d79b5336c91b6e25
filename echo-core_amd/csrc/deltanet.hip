// deltanet.hip — gated delta-rule recurrence (gfx950).
//
// Per value head h and token (echo-core-zig/src/kernels/qwen_linear.zig:207-250):
//   S <- decay*S;  kv = S^T k;  delta = (v - kv)*beta;  S <- S + k (x) delta;
//   o = S^T (q/sqrt(d_k))
// Every value channel (column) of S evolves independently given (q, k, decay,
// beta), so the work splits into n_seq*n_v*d_v columns of d_k = 128 floats.
// The state is stored per head TRANSPOSED relative to the reference, S[v][k],
// so one column is 512 contiguous bytes.  A DPP row of 16 lanes owns one
// column, 8 k-entries per lane in VGPRs: both column reductions (kv and o) are
// 4 xor-shuffle adds inside the row, no LDS and no barrier.  A wave holds 4
// columns (2 KB of state, two 16-byte loads per lane), a 256-thread workgroup
// 16 columns of one head.  Across the T tokens of one launch the state never
// leaves the VGPRs; q/k/v/decay/beta for the next token are loaded while the
// current one is computed.
#include "common.hpp"

namespace ec {

struct DnIn {
    float4 q0, q1, k0, k1;
    float v, dec, bt;
};

__device__ __forceinline__ void dn_load(DnIn& in, const float* __restrict__ q, const float* __restrict__ k,
                                        const float* __restrict__ v, const float* __restrict__ decay,
                                        const float* __restrict__ beta, uint32_t t, uint32_t s, uint32_t n_seq,
                                        uint32_t n_v, uint32_t n_k, uint32_t d_v, uint32_t h, uint32_t qh,
                                        uint32_t col, uint32_t ks) {
    const size_t qk = (((size_t)t * n_seq + s) * n_k + qh) * 128 + 8 * ks;
    in.q0 = *(const float4*)(q + qk);
    in.q1 = *(const float4*)(q + qk + 4);
    in.k0 = *(const float4*)(k + qk);
    in.k1 = *(const float4*)(k + qk + 4);
    const size_t hv = ((size_t)t * n_seq + s) * n_v + h;
    in.v = v[hv * d_v + col];
    in.dec = decay[hv];
    in.bt = beta[hv];
}

// grid (n_v * d_v/16, n_seq), block 256: threadIdx/16 = column in the group, %16 = k slice.
__global__ __launch_bounds__(256) void k_deltanet(float* __restrict__ state, const float* __restrict__ q,
                                                  const float* __restrict__ k, const float* __restrict__ v,
                                                  const float* __restrict__ decay, const float* __restrict__ beta,
                                                  float* __restrict__ out, uint32_t T, uint32_t n_seq, uint32_t n_v,
                                                  uint32_t n_k, uint32_t d_v, const int32_t* __restrict__ seq_pos) {
    const uint32_t groups = d_v / 16;
    const uint32_t h = blockIdx.x / groups, s = blockIdx.y;
    if (seq_pos && seq_pos[s] < 0) return;
    const uint32_t col = 16 * (blockIdx.x % groups) + threadIdx.x / 16, ks = threadIdx.x % 16;
    const uint32_t qh = h / (n_v / n_k);
    const float scale = 1.0f / sqrtf(128.0f);
    float* sp = state + (((size_t)s * n_v + h) * d_v + col) * 128 + 8 * ks;
    float4 s0 = *(float4*)sp, s1 = *(float4*)(sp + 4);
    float S[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};

    DnIn cur, nxt;
    dn_load(cur, q, k, v, decay, beta, 0, s, n_seq, n_v, n_k, d_v, h, qh, col, ks);
    for (uint32_t t = 0; t < T; ++t) {
        if (t + 1 < T) dn_load(nxt, q, k, v, decay, beta, t + 1, s, n_seq, n_v, n_k, d_v, h, qh, col, ks);
        const float kk[8] = {cur.k0.x, cur.k0.y, cur.k0.z, cur.k0.w, cur.k1.x, cur.k1.y, cur.k1.z, cur.k1.w};
        const float qq[8] = {cur.q0.x, cur.q0.y, cur.q0.z, cur.q0.w, cur.q1.x, cur.q1.y, cur.q1.z, cur.q1.w};
        float kvp = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            S[i] *= cur.dec;
            kvp = fmaf(S[i], kk[i], kvp);
        }
        const float kv = row16_sum(kvp);
        const float delta = (cur.v - kv) * cur.bt;
        float op = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            S[i] = fmaf(kk[i], delta, S[i]);
            op = fmaf(S[i], qq[i] * scale, op);
        }
        const float o = row16_sum(op);
        if (ks == 0) out[(((size_t)t * n_seq + s) * n_v + h) * d_v + col] = o;
        cur = nxt;
    }
    *(float4*)sp = make_float4(S[0], S[1], S[2], S[3]);
    *(float4*)(sp + 4) = make_float4(S[4], S[5], S[6], S[7]);
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
